"""Float64 oracle of shared-prefix decode over a paged cache (test infrastructure only; see oracle/__init__.py).

The reference ships no paged variant (README.md:141-142).  The op is ops/prefix.py:57-70 over the rows the page
tables name: the prefix's pages in table order, then request n's suffix pages in table order cut at its slens[n]
rows; the rows of an absent page (id outside [0, num_pages)) are left out.  A request left with no row at all
gets NaN (the softmax over an empty set is 0/0).
"""
import math

import numpy as np

from .common import softmax_attend, to64, toint


def gather_rows(kpool, vpool, pages, nrows):
    """K and V rows (Hkv, r, D) of the first nrows rows named by `pages`, without the rows of absent pages."""
    num_pages, Hkv, ps, d = kpool.shape
    ks, vs = [], []
    for j, p in enumerate(pages):
        take = min(ps, nrows - j * ps)
        if take <= 0:
            break
        if 0 <= p < num_pages:
            ks.append(kpool[p, :, :take])
            vs.append(vpool[p, :, :take])
    if not ks:
        return np.zeros((Hkv, 0, d)), np.zeros((Hkv, 0, d))
    return np.concatenate(ks, 1), np.concatenate(vs, 1)


def ref64(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None, layout="HND", **_):
    """Returns (N, Hq, D) float64.  The pools are (num_pages, Hkv, ps, D), or (num_pages, ps, Hkv, D) with
    layout="NHD"."""
    q, kpool, vpool = to64(q), to64(k_pages), to64(v_pages)
    if layout == "NHD":
        kpool, vpool = kpool.transpose(0, 2, 1, 3), vpool.transpose(0, 2, 1, 3)
    pp, sp, sl = toint(prefix_pages), toint(suffix_pages), toint(slens)
    N, Hq, d = q.shape
    num_pages, Hkv, ps, _ = kpool.shape
    G = Hq // Hkv
    S = sp.shape[1] * ps
    kp, vp = gather_rows(kpool, vpool, pp, len(pp) * ps)
    out = np.empty((N, Hkv, G, d))
    for n in range(N):
        sn = S if sl is None else min(max(int(sl[n]), 0), S)
        ks, vs = gather_rows(kpool, vpool, sp[n], sn)
        k = np.concatenate([kp, ks], 1)
        v = np.concatenate([vp, vs], 1)
        if k.shape[1] == 0:                                # no key at all: the softmax is 0/0
            out[n] = np.nan
            continue
        with np.errstate(invalid="ignore", over="ignore"):
            s = (q[n].reshape(Hkv, G, d) @ k.transpose(0, 2, 1)) / math.sqrt(d)
        out[n] = softmax_attend(s, v)
    return out.reshape(N, Hq, d)
