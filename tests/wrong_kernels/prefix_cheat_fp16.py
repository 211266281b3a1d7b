"""Calibration fixture for op `prefix`: a kernel that is wrong on purpose, and must be REJECTED.

Its flaw: half precision where the softmax needs single.  Scores are rounded to fp16 before the exponentials,
the probabilities are fp16, and each softmax sum is a running fp16 total rounded again after every 64-key block
(the reference's calibration set carries the same idea in wrong_kernels/prefix_cheat_fp16.py).  On the nominal
shape the rounding stays under L1's 1e-2 tolerance; over longer contexts the accumulated rounding exceeds twice
the standard op's error, so L3 (and some L2 cases) reject it.  Plain torch code, no libvmk call: verify it with
--skip-gate."""
import math

import torch


def _sum16(p):
    """Sum over the last axis with the running total rounded to fp16 after every 64-element block."""
    L = p.shape[-1]
    pad = (-L) % 64
    if pad:
        p = torch.cat([p, torch.zeros(p.shape[:-1] + (pad,), dtype=p.dtype, device=p.device)], -1)
    blocks = p.reshape(p.shape[:-1] + (-1, 64)).sum(-1).half()
    acc = torch.zeros(p.shape[:-1], dtype=torch.float16, device=p.device)
    for i in range(blocks.shape[-1]):
        acc = (acc + blocks[..., i]).half()
    return acc[..., None]


def kernel(q, kp, vp, ks, vs, slens=None):
    N, Hq, d = q.shape
    Hkv = kp.shape[0]
    G = Hq // Hkv
    sc = 1 / math.sqrt(d)
    qp = q.reshape(N, Hkv, G, d).permute(1, 0, 2, 3).reshape(Hkv, N * G, d)
    s1 = (torch.matmul(qp, kp.transpose(-1, -2).contiguous()) * sc).half()
    m1 = s1.max(-1, keepdim=True).values
    p1 = torch.exp(s1 - m1).half()
    l1 = _sum16(p1)
    o1 = torch.matmul(p1, vp).float().reshape(Hkv, N, G, d).permute(1, 0, 2, 3)
    m1 = m1.float().reshape(Hkv, N, G, 1).permute(1, 0, 2, 3)
    l1 = l1.float().reshape(Hkv, N, G, 1).permute(1, 0, 2, 3)
    s2 = (torch.matmul(q.reshape(N, Hkv, G, d), ks.transpose(-1, -2).contiguous()) * sc).half()
    if slens is not None:
        pos = torch.arange(ks.shape[2], device=q.device)
        s2 = s2.masked_fill(pos[None, None, None, :] >= slens.long()[:, None, None, None], float("-inf"))
    m2 = s2.max(-1, keepdim=True).values
    p2 = torch.exp(s2 - m2).half()
    l2 = _sum16(p2)
    o2 = torch.matmul(p2, vs).float()
    m = torch.maximum(m1, m2.float())
    a, b = torch.exp(m1 - m), torch.exp(m2.float() - m)
    return ((o1 * a + o2 * b) / (l1 * a + l2.float() * b)).half().reshape(N, Hq, d)
