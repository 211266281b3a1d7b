"""Float64 oracle of shared-prefix decode (test infrastructure only; see oracle/__init__.py)."""
import math

import numpy as np

from .common import softmax_attend, to64, toint


def ref64(q, kp, vp, ks, vs, slens=None, **_):
    """ops/prefix.py:57-70: per request, keys/values = [prefix ; suffix], s = q.k / sqrt(D), max-subtracted
    softmax, o = p.v.  With `slens` (this build's ragged extension) request n keeps its first slens[n] suffix rows.
    Returns (N, Hq, D) float64."""
    q, kp, vp, ks, vs = (to64(x) for x in (q, kp, vp, ks, vs))
    sl = toint(slens)
    N, Hq, d = q.shape
    Hkv = kp.shape[0]
    G = Hq // Hkv
    S = ks.shape[2]
    out = np.empty((N, Hkv, G, d))
    for n in range(N):
        sn = S if sl is None else int(sl[n])
        k = np.concatenate([kp, ks[n, :, :sn]], axis=1)          # (Hkv, P+sn, D)
        v = np.concatenate([vp, vs[n, :, :sn]], axis=1)
        with np.errstate(invalid="ignore", over="ignore"):
            s = (q[n].reshape(Hkv, G, d) @ k.transpose(0, 2, 1)) / math.sqrt(d)   # (Hkv, G, P+sn)
        out[n] = softmax_attend(s, v)
    return out.reshape(N, Hq, d)
