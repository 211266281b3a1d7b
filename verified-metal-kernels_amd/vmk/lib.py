"""ctypes binding of libvmk.so, the C-ABI declared in include/vmk.h.

The library is loaded from this directory; there is no fallback: if it is missing or the GPU is not a gfx950, every
entry point raises.  Pointers are raw device addresses (torch `data_ptr()`), streams are HIP stream handles.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvmk.so")

_lib = None
_c_vp, _c_i64, _c_sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t

# name -> argument types (return type int unless listed in _RET)
_SIGS = {
    "vmk_version": [],
    "vmk_last_error": [],
    "vmk_check_device": [],
    "vmk_debug_mfma32": [_c_vp, _c_vp, _c_vp, _c_vp],
    "vmk_debug_tile": [_c_vp] * 7 + [ctypes.c_float, _c_vp],
    "vmk_debug_select_threshold": [_c_vp, _c_vp, ctypes.c_uint32, _c_vp],
    "vmk_profile_next": [_c_vp, _c_vp, ctypes.c_int],
    "vmk_spec_workspace_size": [_c_i64] * 6,
    "vmk_spec_verify": [_c_vp] * 5 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_spec_noalloc_max_bytes": [],
    "vmk_spec_verify_noalloc": [_c_vp] * 5 + [_c_i64] * 7 + [_c_vp],
    "vmk_decode_workspace_size": [_c_i64] * 5,
    "vmk_decode": [_c_vp] * 5 + [_c_i64] * 5 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_workspace_size": [_c_i64] * 7,
    "vmk_prefix_decode": [_c_vp] * 7 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_paged_workspace_size": [_c_i64] * 7,
    "vmk_prefix_decode_paged": [_c_vp] * 7 + [_c_i64] * 8 + [_c_vp, _c_sz, _c_vp],
    "vmk_spec_verify_bf16": [_c_vp] * 5 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_decode_bf16": [_c_vp] * 5 + [_c_i64] * 5 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_decode_bf16": [_c_vp] * 7 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_decode_paged_bf16": [_c_vp] * 7 + [_c_i64] * 8 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_decode_paged_nhd": [_c_vp] * 7 + [_c_i64] * 8 + [_c_vp, _c_sz, _c_vp],
    "vmk_prefix_decode_paged_nhd_bf16": [_c_vp] * 7 + [_c_i64] * 8 + [_c_vp, _c_sz, _c_vp],
    "vmk_decode_paged_workspace_size": [_c_i64] * 6,
    "vmk_decode_paged": [_c_vp] * 6 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_decode_paged_bf16": [_c_vp] * 6 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_decode_paged_nhd": [_c_vp] * 6 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_decode_paged_nhd_bf16": [_c_vp] * 6 + [_c_i64] * 7 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_indexer_select_bf16": [_c_vp] * 6 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_sparse_mla_bf16": [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_decode_bf16": [_c_vp] * 9 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_workspace_size": [_c_i64] * 2,
    "vmk_dsa_indexer_select": [_c_vp] * 6 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_indexer": [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_indexer_bf16": [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_topk": [_c_vp] * 4 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_sparse_mla": [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_decode": [_c_vp] * 9 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_decode_single": [_c_vp] * 9 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_decode_single_bf16": [_c_vp] * 9 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_project_workspace_size": [_c_i64],
    # x, pos, rope_cos, rope_sin, rope_rows, &weights (host struct), q, iq, w, kv, ik, B, L, workspace, bytes, stream
    "vmk_dsa_project": [_c_vp] * 4 + [_c_i64, _c_vp] + [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
    "vmk_dsa_project_bf16": [_c_vp] * 4 + [_c_i64, _c_vp] + [_c_vp] * 5 + [_c_i64] * 2 + [_c_vp, _c_sz, _c_vp],
}
_RET = {"vmk_last_error": ctypes.c_char_p, "vmk_spec_workspace_size": _c_sz, "vmk_spec_noalloc_max_bytes": _c_sz, "vmk_prefix_workspace_size": _c_sz,
        "vmk_prefix_paged_workspace_size": _c_sz,
        "vmk_decode_paged_workspace_size": _c_sz,
        "vmk_dsa_workspace_size": _c_sz, "vmk_decode_workspace_size": _c_sz, "vmk_dsa_project_workspace_size": _c_sz}

# struct vmk_dsa_project_weights of include/vmk.h: device pointers of the projection weights, in its field order.
PROJECT_WEIGHT_FIELDS = ("wq_a", "q_norm", "wq_b", "w_uk", "wkv_a", "kv_norm", "iwq_b", "iwk", "ik_norm_w",
                         "ik_norm_b", "iw")


class DsaProjectWeights(ctypes.Structure):
    _fields_ = [(name, _c_vp) for name in PROJECT_WEIGHT_FIELDS]


class VmkError(RuntimeError):
    """A failed libvmk call; `code` is the entry point's return value (1 = arguments rejected, nothing launched;
    2 = HIP launch or runtime error), None for errors raised on the Python side."""

    def __init__(self, msg, code=None):
        super().__init__(msg)
        self.code = code


REJECTED, LAUNCH_ERROR = 1, 2


def load():
    """Loads libvmk.so once and declares every exported symbol; raises if the file or a symbol is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VmkError(f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in _SIGS.items():
        if not hasattr(lib, name):
            continue
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RET.get(name, ctypes.c_int)
    _lib = lib
    return lib


# Kernel ids of vmk_profile_next (include/vmk.h).
KERNEL_IDS = {"spec_partial": 0, "spec_combine": 1, "prefix_partial": 2, "prefix_combine": 3,
              "dsa_indexer": 4, "dsa_select": 5, "dsa_attn": 6, "dsa_combine": 7,
              "dsa_select_scan": 8, "dsa_project_q": 9, "dsa_single": 10}


def exported_symbols():
    return list(_SIGS)


def check(rc):
    if rc != 0:
        raise VmkError(load().vmk_last_error().decode(errors="replace") or f"libvmk error {rc}", code=rc)


def call(name, *args):
    check(getattr(load(), name)(*args))
