"""Float64 oracle of single-token decode (test infrastructure only; see oracle/__init__.py).

The reference ships no kernel module for this op: it benchmarks plain decode against llama.cpp
(llama_cpp/test-backend-ops.patch:79-83) and reports it at parity (POST.md:42-46).  The op is GQA attention of one
query per request over the request's cache, i.e. ops/spec.py:69-82 with kd = 1 (the query is the last cache position
and sees itself), restricted to the first lens[b] positions when lengths are given.
"""
import math

import numpy as np

from .common import softmax_attend, to64, toint


def ref64(q, k, v, lens=None):
    """q (B, Hq, D), k/v (B, Hkv, L, D), lens (B,) or None (all L; lengths are clamped to [1, L]).
    Returns (B, Hq, D) float64."""
    q, k, v = (to64(x) for x in (q, k, v))
    ln = toint(lens)
    B, Hq, d = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.empty((B, Hkv, G, d))
    for b in range(B):
        n = L if ln is None else min(max(int(ln[b]), 1), L)
        with np.errstate(invalid="ignore", over="ignore"):
            s = (q[b].reshape(Hkv, G, d) @ k[b, :, :n].transpose(0, 2, 1)) / math.sqrt(d)    # (Hkv, G, n)
        out[b] = softmax_attend(s, v[b, :, :n])
    return out.reshape(B, Hq, d)
