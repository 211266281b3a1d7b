"""Float64 oracle of DSA decode: indexer scores, top-2048 selection, sparse MLA (test infrastructure only)."""
import math

import numpy as np

from .common import softmax_attend, to64, toint

H, DC, DR, HI, DI, TOPK = 128, 512, 64, 64, 128, 2048          # ops/dsa.py:15
DK = DC + DR
SCALE = 1.0 / math.sqrt(128 + 64)                              # ops/dsa.py:17


def scores64(iq, ik, w):
    """ops/dsa.py:57-58: s[b, l] = sum_h w[b, h] * max(iq[b, h] . ik[b, l], 0) in float64."""
    iq, ik = to64(iq), to64(ik)
    w = toint(w).astype(np.float64)
    s = iq @ ik.transpose(0, 2, 1)                              # (B, HI, L)
    return (np.maximum(s, 0) * w[:, :, None]).sum(1)


def ref_select64(iq, ik, w, lens=None):
    """ops/dsa.py:53-66: scores, then per request all n positions if n <= 2048, else the 2048 largest among the
    first n (unordered, `np.argpartition`).  Returns (scores (B, L), list of index arrays)."""
    s = scores64(iq, ik, w)
    B, L = s.shape
    ln = toint(lens)
    sel = []
    for b in range(B):
        n = L if ln is None else int(ln[b])
        if n <= TOPK:
            sel.append(np.arange(n))
        else:
            sel.append(np.argpartition(-s[b, :n], TOPK - 1)[:TOPK])
    return s, sel


def ref64(q, kv, iq, ik, w, lens=None, sel=None):
    """ops/dsa.py:69-83: per request, gathered rows ks = kv[sel]; s = q . ks^T * SCALE; softmax; p @ ks[:, :512].
    Returns (B, 128, 512) float64."""
    if sel is None:
        _, sel = ref_select64(iq, ik, w, lens)
    q, kv = to64(q), to64(kv)
    B = q.shape[0]
    out = np.zeros((B, H, DC))
    for b in range(B):
        ks = kv[b, sel[b]]
        with np.errstate(invalid="ignore", over="ignore"):
            s = q[b] @ ks.T * SCALE
        out[b] = softmax_attend(s, ks[:, :DC])
    return out


def score_error_bound(iq, ik, w, lens=None):
    """Per request, a bound B on |s32(p) - s64(p)| over its positions p, where s32 is any fp32 evaluation of
    ops/dsa.py:57-58 from the same 16-bit inputs (this build's indexer: MFMA products, fp32 sums).

    Derivation (u = 2^-24, gamma_n = n u / (1 - n u)):
      * a product of two fp16 or bf16 values needs at most 22 significand bits, so it is exact in fp32;
      * the 128-term dot product, summed in any order, errs by at most gamma_127 * sum_i |iq_hi ik_pi|;
      * max(., 0) is 1-Lipschitz; w_h times it rounds once (u);
      * the 64-term weighted sum errs by at most gamma_63 times the sum of its terms' magnitudes.
    To first order the total is gamma_(DI+HI) * sum_h |w_h| * sum_i |iq_hi ik_pi|; gamma_(DI+HI+2) covers the
    second-order terms.  B is its maximum over the request's first n positions."""
    iq, ik = np.abs(to64(iq)), np.abs(to64(ik))
    w = np.abs(toint(w).astype(np.float64))
    nu = (DI + HI + 2) * 2.0 ** -24
    gamma = nu / (1.0 - nu)
    mag = ((iq @ ik.transpose(0, 2, 1)) * w[:, :, None]).sum(1)          # (B, L)
    ln = toint(lens)
    out = np.zeros(mag.shape[0])
    for b in range(mag.shape[0]):
        n = mag.shape[1] if ln is None else int(ln[b])
        out[b] = gamma * mag[b, :max(n, 1)].max()
    return out


def topk_set_check(idx, cnt, s64, n, bound):
    """This build's top-k exactness check for one request.  `idx` are the kernel's selected positions (first `cnt`
    entries valid), `s64` the float64 scores, `bound` the request's score_error_bound.  Passes when the count is
    min(n, 2048), the indices are distinct and in [0, n), and the selected set equals the float64 top set on every
    position whose score is farther than 2 * bound from the 2048-th largest score tau.  Within that band an fp32
    evaluation may legitimately reorder: every fp32 score is within `bound` of its float64 value, so the fp32
    2048-th score is within `bound` of tau, and a position more than 2 * bound above (below) tau is above (below)
    it in fp32 too.  Returns (ok, detail dict); detail["boundary"] counts the positions inside the band and
    detail["swapped"] the selected positions outside the float64 top set (ties at tau taken by position)."""
    idx = np.asarray(idx)[:cnt].astype(np.int64)
    k = min(n, TOPK)
    det = dict(cnt=int(cnt), expected=k)
    if cnt != k:
        return False, dict(det, error="count")
    if len(np.unique(idx)) != k or (k and (idx.min() < 0 or idx.max() >= n)):
        return False, dict(det, error="indices not distinct or out of range")
    if n <= TOPK:
        return bool(np.array_equal(np.sort(idx), np.arange(n))), det
    s = s64[:n]
    tau = np.partition(s, n - TOPK)[n - TOPK]
    band = 2.0 * float(bound)
    must = np.nonzero(s > tau + band)[0]
    never = s < tau - band
    chosen = np.zeros(n, dtype=bool)
    chosen[idx] = True
    missing = int((~chosen[must]).sum())
    wrong = int((chosen & never).sum())
    top = np.zeros(n, dtype=bool)
    top[np.argsort(-s, kind="stable")[:TOPK]] = True
    det.update(tau=float(tau), band=band, missing=missing, wrong=wrong,
               boundary=int(((s >= tau - band) & (s <= tau + band)).sum()), swapped=int((chosen & ~top).sum()))
    return missing == 0 and wrong == 0, det
