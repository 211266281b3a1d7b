"""Single-token decode on MI355X: the `kernel(q, k, v, lens)` module of the decode op contract (vmk.ops.decode).

One call = the verify path's split-K MFMA partial launch and LSE-combine launch of libvmk with one query row per
request and no mask (vmk_decode)."""
import torch

import vmk


def kernel(q, k, v, lens=None):
    if q.dtype == torch.bfloat16 or k.dtype == torch.bfloat16 or v.dtype == torch.bfloat16:
        raise TypeError("decode kernel reads fp16 inputs; bf16 is not supported")
    q, k, v = (x.to(torch.float16).contiguous() for x in (q, k, v))
    if lens is not None:
        lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.decode(q, k, v, lens)
