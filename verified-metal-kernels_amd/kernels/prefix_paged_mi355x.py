"""Shared-prefix decode over a paged cache on MI355X: the `kernel(q, k_pages, v_pages, prefix_pages, suffix_pages,
slens)` module of the prefix_paged op contract (vmk.ops.prefix_paged).

One call = libvmk's prefix launches with page-table tile addressing (vmk_prefix_decode_paged, or
vmk_prefix_decode_paged_nhd for a pool laid out (num_pages, page_size, Hkv, D) with layout="NHD")."""
import torch

import vmk


def kernel(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None, layout="HND"):
    dt = torch.bfloat16 if torch.bfloat16 in (q.dtype, k_pages.dtype, v_pages.dtype) else torch.float16
    q, k_pages, v_pages = (x.to(dt).contiguous() for x in (q, k_pages, v_pages))
    prefix_pages = prefix_pages.to(device=q.device, dtype=torch.int32).contiguous()
    suffix_pages = suffix_pages.to(device=q.device, dtype=torch.int32).contiguous()
    if slens is not None:
        slens = slens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.prefix_decode_paged(q, k_pages, v_pages, prefix_pages, suffix_pages, slens, layout=layout or "HND")
