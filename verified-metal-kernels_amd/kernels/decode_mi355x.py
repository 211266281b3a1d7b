"""Single-token decode on MI355X: the `kernel(q, k, v, lens)` module of the decode op contract (vmk.ops.decode).

One call = the verify path's split-K MFMA partial launch and LSE-combine launch of libvmk with one query row per
request and no mask (vmk_decode)."""
import torch

import vmk


def kernel(q, k, v, lens=None):
    dt = torch.bfloat16 if torch.bfloat16 in (q.dtype, k.dtype, v.dtype) else torch.float16
    q, k, v = (x.to(dt).contiguous() for x in (q, k, v))
    if lens is not None:
        lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.decode(q, k, v, lens)
