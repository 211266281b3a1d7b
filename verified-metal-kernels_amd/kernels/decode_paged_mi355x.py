"""Paged single-token decode on MI355X: the `kernel(q, k_pages, v_pages, page_table, lens, layout)` module of the
paged decode op contract (vmk.ops.decode_paged).

One call = libvmk's key-split partial launch reading each request's keys through its page table, and the LSE-combine
launch (vmk_decode_paged, or vmk_decode_paged_nhd for a pool laid out (num_pages, page_size, Hkv, D))."""
import torch

import vmk


def kernel(q, k_pages, v_pages, page_table, lens=None, layout=None):
    dt = torch.bfloat16 if torch.bfloat16 in (q.dtype, k_pages.dtype, v_pages.dtype) else torch.float16
    q, k_pages, v_pages = (x.to(dt).contiguous() for x in (q, k_pages, v_pages))
    page_table = page_table.to(device=q.device, dtype=torch.int32).contiguous()
    if lens is not None:
        lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
    return vmk.decode_paged(q, k_pages, v_pages, page_table, lens, layout=layout or "HND")
