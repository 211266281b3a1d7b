"""Float64 oracle of paged single-token decode (test infrastructure only; see oracle/__init__.py).

The decode op of oracle/decode.py over the rows a page table names: request b's pages in table order, cut at its
lens[b] positions (clamped to [1, max_pages * page_size]), without the rows of absent pages (ids outside
[0, num_pages)).  A request left with no row at all gets NaN (the softmax over an empty set is 0/0).
"""
import math

import numpy as np

from .common import softmax_attend, to64, toint


def ref64(q, k_pages, v_pages, page_table, lens=None, layout="HND", **_):
    """q (B, Hq, D); pools (num_pages, Hkv, ps, D), or (num_pages, ps, Hkv, D) with layout="NHD"; page_table
    (B, max_pages); lens (B,) or None.  Returns (B, Hq, D) float64."""
    q, kpool, vpool = to64(q), to64(k_pages), to64(v_pages)
    if layout == "NHD":
        kpool, vpool = kpool.transpose(0, 2, 1, 3), vpool.transpose(0, 2, 1, 3)
    pt, ln = toint(page_table), toint(lens)
    B, Hq, d = q.shape
    num_pages, Hkv, ps, _ = kpool.shape
    G = Hq // Hkv
    L = pt.shape[1] * ps
    out = np.empty((B, Hkv, G, d))
    for b in range(B):
        n = L if ln is None else min(max(int(ln[b]), 1), L)
        ks, vs = [], []
        for j in range(-(-n // ps)):
            p = int(pt[b, j])
            if 0 <= p < num_pages:
                take = min(ps, n - j * ps)
                ks.append(kpool[p, :, :take])
                vs.append(vpool[p, :, :take])
        if not ks:                                         # no key at all: the softmax is 0/0
            out[b] = np.nan
            continue
        k, v = np.concatenate(ks, 1), np.concatenate(vs, 1)
        with np.errstate(invalid="ignore", over="ignore"):
            s = (q[b].reshape(Hkv, G, d) @ k.transpose(0, 2, 1)) / math.sqrt(d)
        out[b] = softmax_attend(s, v)
    return out.reshape(B, Hq, d)
