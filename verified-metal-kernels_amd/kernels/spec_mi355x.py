"""Speculative chain/tree verification on MI355X: the `kernel(q, k, v, bits)` module of the op contract
(ops/spec.py:1-3; the reference's kernels/spec_opus55_v7.py:467-521 is the Metal counterpart).

One call = one split-K MFMA partial launch + one LSE-combine launch of libvmk (vmk_spec_verify).
bits: (B, kd) int32 (reference layout, kd <= 32) or (B, kd, W) int32 words (W = ceil(kd/32))."""
import torch

import vmk


def kernel(q, k, v, bits):
    dt = torch.bfloat16 if torch.bfloat16 in (q.dtype, k.dtype, v.dtype) else torch.float16
    q, k, v = (x.to(dt).contiguous() for x in (q, k, v))
    B, kd = q.shape[0], q.shape[1]
    words = bits.to(device=q.device, dtype=torch.int32)
    if words.dim() == 2:
        words = words.reshape(B, kd, 1)
    return vmk.spec_verify(q, k, v, words.contiguous())
