"""DELIBERATELY WRONG kernel for op `spec` (a verifier calibration fixture; restates the reference's
wrong_kernels/spec_cheat_nomax.py:1-28 as a PyTorch composition).

The "optimisation": softmax without subtracting the running maximum, exponentials in fp32.  On ordinary inputs the
result matches (L1 and L3 pass); with large scores exp() overflows and the output is NaN where the float64 reference
is finite, so the fuzzing layer rejects it.  It uses no libvmk kernel: run the verifier with --skip-gate."""
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
