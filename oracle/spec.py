"""Float64 oracle of speculative chain/tree verification (test infrastructure only; see oracle/__init__.py)."""
import math

import numpy as np

from .common import softmax_attend, to64, toint


def words(bits, kd):
    """(B, kd) int32 (reference layout) or (B, kd, W) int32 words -> (B, kd, W) uint32."""
    b = toint(bits).astype(np.int64) & 0xFFFFFFFF
    if b.ndim == 2:
        b = b[:, :, None]
    return b.astype(np.uint32)


def allowed(bits, L, kd):
    """ops/spec.py:59-66: (B, kd, L) bool, every context position plus bit j of draft i's mask for position
    L - kd + j (bit j lives in word j // 32)."""
    w = words(bits, kd).astype(np.int64)
    B = w.shape[0]
    a = np.ones((B, kd, L), dtype=bool)
    j = np.arange(kd)
    a[:, :, L - kd:] = ((w[:, :, j // 32] >> (j % 32)[None, None, :]) & 1).astype(bool)
    return a


def ref64(q, k, v, bits):
    """ops/spec.py:69-82: float64 masked GQA attention, -inf on disallowed keys, max-subtracted softmax.
    Returns (B, kd, Hq, D) float64.  Processed one batch at a time to bound memory."""
    q, k, v = (to64(x) for x in (q, k, v))
    B, kd, Hq, d = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    a = allowed(bits, L, kd)
    out = np.empty((B, Hkv, kd, G, d))
    for b in range(B):
        qb = q[b].reshape(kd, Hkv, G, d).transpose(1, 0, 2, 3)               # (Hkv, kd, G, d)
        with np.errstate(invalid="ignore", over="ignore"):
            s = (qb.reshape(Hkv, kd * G, d) @ k[b].transpose(0, 2, 1)) / math.sqrt(d)   # (Hkv, kd*G, L)
        s = s.reshape(Hkv, kd, G, L)
        s = np.where(a[b][None, :, None, :], s, -np.inf)
        out[b] = softmax_attend(s.reshape(Hkv, kd * G, L), v[b]).reshape(Hkv, kd, G, d)
    return out.transpose(0, 2, 1, 3, 4).reshape(B, kd, Hq, d)
