"""vmk: MI355X (gfx950) kernels for shared-prefix decode (contiguous or paged cache), speculative verification,
single-token decode (contiguous or paged cache), DSA decode and the projections that make DSA's inputs.

Host side of the C-ABI library libvmk.so (HIP kernels in ../csrc, declared in include/vmk.h).  Tensors are torch
tensors on a ROCm device; every call launches on torch's current stream and returns without synchronising.
"""
from .lib import VmkError, load  # noqa: F401
from .api import (spec_verify, spec_verify_noalloc, decode, decode_paged,  # noqa: F401
                  prefix_decode, prefix_decode_paged, dsa_decode, dsa_indexer_select, dsa_indexer, dsa_topk,
                  dsa_sparse_mla, dsa_project, workspace, reserve_workspace, device_ok)
