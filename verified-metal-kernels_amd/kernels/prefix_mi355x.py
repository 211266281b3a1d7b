"""Shared-prefix decode on MI355X: the `kernel(q, kp, vp, ks, vs)` module of the op contract (ops/prefix.py:1-4; the
reference's kernels/prefix_opus55_v8.py:282-355 is the Metal counterpart), with optional ragged suffix lengths.

One call = one partial launch (prefix items streaming the shared prefix once per KV head and row block, suffix items
per request) + one LSE-combine launch of libvmk (vmk_prefix_decode)."""
import torch

import vmk


def kernel(q, kp, vp, ks, vs, slens=None):
    dt = torch.bfloat16 if any(x.dtype == torch.bfloat16 for x in (q, kp, vp, ks, vs)) else torch.float16
    q, kp, vp, ks, vs = (x.to(dt).contiguous() for x in (q, kp, vp, ks, vs))
    if slens is not None:
        slens = slens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.prefix_decode(q, kp, vp, ks, vs, slens)
