"""DELIBERATELY WRONG kernel for op `decode` (a verifier calibration fixture for the row-invariance layer L4).

Numerically sound on every call: fp32 scores, max-subtracted softmax per chunk of keys and an exact log-sum-exp
merge of the chunks.  But the keys are cut into B + 1 chunks, one more than the batch has requests, so the
rounding of a request's output depends on how many requests share the call.  L1, L2, L3, X and CFG accept it;
only L4 (a row alone against the same row in the batch, byte for byte) rejects it.  It uses no libvmk kernel: run the
verifier with --skip-gate."""
import math

import torch


def kernel(q, k, v, lens=None):
    B, Hq, d = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    s = torch.matmul(q.float().reshape(B, Hkv, G, d), k.float().transpose(-1, -2).contiguous()) / math.sqrt(d)
    if lens is not None:
        n = lens.to(q.device).long().clamp(1, L)
        past = torch.arange(L, device=q.device)[None, :] >= n[:, None]
        s = s.masked_fill(past[:, None, None, :], float("-inf"))
    vf = v.float()
    edges = torch.linspace(0, L, B + 2).round().long().tolist()
    M = torch.full((B, Hkv, G, 1), float("-inf"), device=q.device)
    num = torch.zeros(B, Hkv, G, d, device=q.device)
    den = torch.zeros(B, Hkv, G, 1, device=q.device)
    for a, b in zip(edges[:-1], edges[1:]):
        if b <= a:
            continue
        sc = s[..., a:b]
        m = sc.amax(-1, keepdim=True)
        ms = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(m), m)
        p = torch.exp(sc - ms)
        o = torch.matmul(p, vf[:, :, a:b])
        l = p.sum(-1, keepdim=True)
        Mn = torch.maximum(M, m)
        Mu = torch.where(torch.isinf(Mn) & (Mn < 0), torch.zeros_like(Mn), Mn)
        al, be = torch.exp(M - Mu), torch.exp(m - Mu)
        num = num * al + o * be
        den = den * al + l * be
        M = Mn
    return (num / den).half().reshape(B, Hq, d)
