"""Calibration fixture for op `spec`: a kernel that is wrong on purpose, and must be REJECTED.

Its flaw: the exponentials of the softmax are taken of the raw scaled scores, with no maximum subtracted first
(the reference's calibration set has the same flaw, wrong_kernels/spec_cheat_nomax.py).  With unit-scale inputs
exp() stays in float32 range and the outputs agree with the standard op and with float64, so layers L1 and L3
accept it.  The fuzz case with inputs scaled by 8 drives exp() past float32's range: inf / inf gives NaN where
float64 is finite, and L2 rejects it.  Plain torch code, no libvmk call: verify it with --skip-gate."""
import math

import torch


def kernel(q, k, v, bits):
    B, kd, Hq, d = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qf = q.reshape(B, kd, Hkv, G, d).permute(0, 2, 1, 3, 4).reshape(B, Hkv, kd * G, d)
    s = torch.matmul(qf.float(), k.float().transpose(-1, -2).contiguous()) * (1 / math.sqrt(d))
    w = bits.long() & 0xFFFFFFFF
    w = w.reshape(B, kd, -1)
    j = torch.arange(kd, device=q.device)
    tail = ((w[:, :, j // 32] >> (j % 32)) & 1).bool()
    m = torch.cat([torch.ones(B, kd, L - kd, dtype=torch.bool, device=q.device), tail], -1)
    m = m.repeat_interleave(G, dim=1)[:, None]
    e = torch.where(m, torch.exp(s), torch.zeros((), device=q.device))
    p = (e / e.sum(-1, keepdim=True)).half()
    o = torch.matmul(p, v)
    return o.reshape(B, Hkv, kd, G, d).permute(0, 2, 1, 3, 4).reshape(B, kd, Hq, d)
