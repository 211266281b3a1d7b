"""DSA decode on MI355X: the `kernel(q, kv, iq, ik, w, lens)` module of the op contract (ops/dsa.py:1-9; the
reference's kernels/dsa_opus55_v7.py:946-977 is the Metal counterpart).

One call = indexer (MFMA scores + fused radix histogram, skipped when L <= 2048) -> exact top-2048 select ->
sparse absorbed-MLA partials -> LSE combine: four launches of libvmk (vmk_dsa_decode)."""
import torch

import vmk


def kernel(q, kv, iq, ik, w, lens=None):
    dt = torch.bfloat16 if any(x.dtype == torch.bfloat16 for x in (q, kv, iq, ik)) else torch.float16
    q, kv, iq, ik = (x.to(dt).contiguous() for x in (q, kv, iq, ik))
    w = w.to(device=q.device, dtype=torch.float32).contiguous()
    if lens is not None:
        lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.dsa_decode(q, kv, iq, ik, w, lens)


def select(iq, ik, w, lens=None):
    """The indexer + exact top-2048 stage alone: returns idx (B, 2048) int32 and cnt (B,) int32."""
    dt = torch.bfloat16 if torch.bfloat16 in (iq.dtype, ik.dtype) else torch.float16
    iq, ik = (x.to(dt).contiguous() for x in (iq, ik))
    w = w.to(device=iq.device, dtype=torch.float32).contiguous()
    if lens is not None:
        lens = lens.to(device=iq.device, dtype=torch.int32).contiguous()
    return vmk.dsa_indexer_select(iq, ik, w, lens)
