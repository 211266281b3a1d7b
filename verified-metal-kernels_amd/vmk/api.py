"""torch-facing wrappers of the libvmk C-ABI: argument checks, output and workspace allocation, stream plumbing.

Every wrapper launches on `torch.cuda.current_stream()` of the inputs' device and returns without synchronising.
Workspaces come from one cached byte buffer per device that only grows; calls that overlap on two streams of one
device would share it, so they must be ordered by the caller.
"""
import torch

from . import lib

_ws = {}
_dev_ok = {}


def device_ok(device):
    """Raises unless `device` is a ROCm gfx950 device and libvmk.so is loaded (checked once per device)."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _dev_ok:
        if not torch.cuda.is_available():
            raise lib.VmkError("libvmk needs a ROCm GPU; torch.cuda.is_available() is False")
        with torch.cuda.device(idx):
            lib.call("vmk_check_device")
        _dev_ok[idx] = True
    return True


def workspace(nbytes, device):
    """A cached uint8 buffer of at least `nbytes` on `device` (grown, never shrunk).

    Allocated zeroed: libvmk requires the workspace head (its first 4 MiB) to be zero before the first call, and
    every call leaves it zero again."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=dev)
        _ws[key] = buf
    return buf


def _stream(t):
    return ctypes_ptr(torch.cuda.current_stream(t.device).cuda_stream)


def ctypes_ptr(x):
    return int(x)


def _need(t, name, dtype, ndim):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a ROCm device")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


_SUFFIX = {torch.float16: "", torch.bfloat16: "_bf16"}


def _elem(q):
    """Entry-point suffix for q's dtype: fp16 or bf16 (q, keys and values share it; the output gets it too)."""
    if not isinstance(q, torch.Tensor):
        raise TypeError("q must be a torch.Tensor")
    if q.dtype not in _SUFFIX:
        raise TypeError(f"q must be float16 or bfloat16, got {q.dtype}")
    return q.dtype, _SUFFIX[q.dtype]


def spec_verify(q, k, v, words, out=None):
    """q (B, kd, Hq, 128), k/v (B, Hkv, L, 128), all fp16 or all bf16; words (B, kd, W) int32 with W = ceil(kd/32).
    Returns out (B, kd, Hq, 128) of q's dtype."""
    dt, sfx = _elem(q)
    _need(q, "q", dt, 4)
    _need(k, "k", dt, 4)
    _need(v, "v", dt, 4)
    _need(words, "bits", torch.int32, 3)
    B, kd, Hq, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    if tuple(k.shape) != (B, Hkv, L, D) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k/v shape {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if tuple(words.shape[:2]) != (B, kd):
        raise ValueError(f"bits shape {tuple(words.shape)} does not match (B, kd) = {(B, kd)}")
    device_ok(q.device)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_spec_workspace_size(B, kd, Hq, Hkv, D, L)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported spec shape B={B} kd={kd} Hq={Hq} Hkv={Hkv} D={D} L={L}")
    ws = workspace(ws_n, q.device)
    lib.call("vmk_spec_verify" + sfx, q.data_ptr(), k.data_ptr(), v.data_ptr(), words.data_ptr(), out.data_ptr(),
             B, kd, Hq, Hkv, D, L, words.shape[2], ws.data_ptr(), ws.numel(), _stream(q))
    return out


def decode(q, k, v, lens=None, out=None):
    """Single-token decode: q (B, Hq, 128), k/v (B, Hkv, L, 128), all fp16 or all bf16; lens (B,) int32 or None (all
    L in use).  Returns out (B, Hq, 128) of q's dtype."""
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    _need(k, "k", dt, 4)
    _need(v, "v", dt, 4)
    B, Hq, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    if tuple(k.shape) != (B, Hkv, L, D) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k/v shape {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
        if lens.shape[0] != B:
            raise ValueError("lens must have B entries")
    device_ok(q.device)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_decode_workspace_size(B, Hq, Hkv, D, L)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported decode shape B={B} Hq={Hq} Hkv={Hkv} D={D} L={L}")
    ws = workspace(ws_n, q.device)
    lib.call("vmk_decode" + sfx, q.data_ptr(), k.data_ptr(), v.data_ptr(), 0 if lens is None else lens.data_ptr(),
             out.data_ptr(), B, Hq, Hkv, D, L, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def prefix_decode(q, kp, vp, ks, vs, slens=None, out=None):
    """q (N, Hq, 128), kp/vp (Hkv, P, 128), ks/vs (N, Hkv, S, 128), all fp16 or all bf16; slens (N,) int32 or
    None.  Returns out (N, Hq, 128) of q's dtype."""
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    for t, n in ((kp, "kp"), (vp, "vp")):
        _need(t, n, dt, 3)
    for t, n in ((ks, "ks"), (vs, "vs")):
        _need(t, n, dt, 4)
    N, Hq, D = q.shape
    Hkv, P = kp.shape[0], kp.shape[1]
    S = ks.shape[2]
    if tuple(kp.shape) != (Hkv, P, D) or tuple(vp.shape) != tuple(kp.shape):
        raise ValueError("kp/vp shapes do not match")
    if tuple(ks.shape) != (N, Hkv, S, D) or tuple(vs.shape) != tuple(ks.shape):
        raise ValueError("ks/vs shapes do not match")
    if slens is not None:
        _need(slens, "slens", torch.int32, 1)
        if slens.shape[0] != N:
            raise ValueError("slens must have N entries")
    device_ok(q.device)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_prefix_workspace_size(N, Hq, Hkv, D, P, S, 0 if slens is None else 1)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported prefix shape N={N} Hq={Hq} Hkv={Hkv} D={D} P={P} S={S}")
    ws = workspace(ws_n, q.device)
    lib.call("vmk_prefix_decode" + sfx, q.data_ptr(), kp.data_ptr(), vp.data_ptr(), ks.data_ptr(), vs.data_ptr(),
             0 if slens is None else slens.data_ptr(), out.data_ptr(), N, Hq, Hkv, D, P, S,
             0 if slens is None else 1, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def prefix_decode_paged(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None, out=None):
    """Shared-prefix decode over a paged cache.  q (N, Hq, 128); k_pages/v_pages (num_pages, Hkv, page_size, 128)
    with page_size a multiple of 32, all fp16 or all bf16; prefix_pages (P / page_size,) int32; suffix_pages
    (N, max_sp) int32; slens (N,) int32 or None (full suffixes).  Page ids outside [0, num_pages) are absent pages
    (left out).  Returns out (N, Hq, 128) of q's dtype."""
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    for t, n in ((k_pages, "k_pages"), (v_pages, "v_pages")):
        _need(t, n, dt, 4)
    _need(prefix_pages, "prefix_pages", torch.int32, 1)
    _need(suffix_pages, "suffix_pages", torch.int32, 2)
    N, Hq, D = q.shape
    num_pages, Hkv, ps = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
    if tuple(k_pages.shape) != (num_pages, Hkv, ps, D) or tuple(v_pages.shape) != tuple(k_pages.shape):
        raise ValueError("k_pages/v_pages shapes do not match")
    if suffix_pages.shape[0] != N:
        raise ValueError("suffix_pages must have N rows")
    if slens is not None:
        _need(slens, "slens", torch.int32, 1)
        if slens.shape[0] != N:
            raise ValueError("slens must have N entries")
    P, max_sp = prefix_pages.shape[0] * ps, suffix_pages.shape[1]
    device_ok(q.device)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_prefix_paged_workspace_size(N, Hq, Hkv, D, P, ps, max_sp)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported paged prefix shape N={N} Hq={Hq} Hkv={Hkv} D={D} P={P} page_size={ps} "
                           f"max_suffix_pages={max_sp}")
    ws = workspace(ws_n, q.device)
    lib.call("vmk_prefix_decode_paged" + sfx, q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(),
             prefix_pages.data_ptr() if P else 0, suffix_pages.data_ptr() if max_sp else 0,
             0 if slens is None else slens.data_ptr(), out.data_ptr(), N, Hq, Hkv, D, num_pages, ps, P, max_sp,
             ws.data_ptr(), ws.numel(), _stream(q))
    return out


DSA_H, DSA_DK, DSA_DC, DSA_HI, DSA_DI, DSA_TOPK = 128, 576, 512, 64, 128, 2048


def _dsa_shapes(q, kv, iq, ik, w, lens):
    dt, _ = _elem(q)
    _need(q, "q", dt, 3)
    _need(kv, "kv", dt, 3)
    _need(iq, "iq", dt, 3)
    _need(ik, "ik", dt, 3)
    _need(w, "w", torch.float32, 2)
    B, L = kv.shape[0], kv.shape[1]
    if tuple(q.shape) != (B, DSA_H, DSA_DK) or kv.shape[2] != DSA_DK:
        raise ValueError(f"q {tuple(q.shape)} / kv {tuple(kv.shape)} must be (B,128,576) / (B,L,576)")
    if tuple(iq.shape) != (B, DSA_HI, DSA_DI) or tuple(ik.shape) != (B, L, DSA_DI) or tuple(w.shape) != (B, DSA_HI):
        raise ValueError("iq (B,64,128), ik (B,L,128), w (B,64) expected")
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
        if lens.shape[0] != B:
            raise ValueError("lens must have B entries")
    return B, L


def dsa_indexer_select(iq, ik, w, lens=None, idx=None, cnt=None):
    """Indexer scores + exact top-2048 per request; iq/ik both fp16 or both bf16, w fp32.  Returns idx (B, 2048)
    int32 (unordered, first cnt[b] valid) and cnt (B,) int32."""
    dt, sfx = _elem(iq)
    _need(iq, "iq", dt, 3)
    _need(ik, "ik", dt, 3)
    _need(w, "w", torch.float32, 2)
    B, L = ik.shape[0], ik.shape[1]
    if tuple(iq.shape) != (B, DSA_HI, DSA_DI) or tuple(ik.shape) != (B, L, DSA_DI) or tuple(w.shape) != (B, DSA_HI):
        raise ValueError("iq (B,64,128), ik (B,L,128), w (B,64) expected")
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
    device_ok(ik.device)
    if idx is None:
        idx = torch.empty(B, DSA_TOPK, dtype=torch.int32, device=ik.device)
    if cnt is None:
        cnt = torch.empty(B, dtype=torch.int32, device=ik.device)
    ws_n = lib.load().vmk_dsa_workspace_size(B, L)
    ws = workspace(ws_n, ik.device)
    lib.call("vmk_dsa_indexer_select" + sfx, iq.data_ptr(), ik.data_ptr(), w.data_ptr(),
             0 if lens is None else lens.data_ptr(), idx.data_ptr(), cnt.data_ptr(), B, L, ws.data_ptr(),
             ws.numel(), _stream(ik))
    return idx, cnt


def dsa_sparse_mla(q, kv, idx, cnt, out=None):
    """Sparse absorbed-MLA attention of q (B,128,576) over rows kv[b, idx[b, :cnt[b]]], q/kv both fp16 or both bf16.
    Returns (B,128,512) of q's dtype."""
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    _need(kv, "kv", dt, 3)
    _need(idx, "idx", torch.int32, 2)
    _need(cnt, "cnt", torch.int32, 1)
    B, L = kv.shape[0], kv.shape[1]
    device_ok(q.device)
    if out is None:
        out = torch.empty(B, DSA_H, DSA_DC, dtype=dt, device=q.device)
    ws_n = lib.load().vmk_dsa_workspace_size(B, L)
    ws = workspace(ws_n, q.device)
    lib.call("vmk_dsa_sparse_mla" + sfx, q.data_ptr(), kv.data_ptr(), idx.data_ptr(), cnt.data_ptr(), out.data_ptr(),
             B, L, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def dsa_decode(q, kv, iq, ik, w, lens=None, out=None, idx=None, cnt=None):
    """Full DSA decode step (indexer -> top-2048 -> sparse MLA); q, kv, iq, ik all fp16 or all bf16, w fp32.
    Returns out (B,128,512) of q's dtype; the selected indices land in `idx`/`cnt` when given."""
    B, L = _dsa_shapes(q, kv, iq, ik, w, lens)
    dt, sfx = _elem(q)
    device_ok(q.device)
    if out is None:
        out = torch.empty(B, DSA_H, DSA_DC, dtype=dt, device=q.device)
    if idx is None:
        idx = torch.empty(B, DSA_TOPK, dtype=torch.int32, device=q.device)
    if cnt is None:
        cnt = torch.empty(B, dtype=torch.int32, device=q.device)
    ws_n = lib.load().vmk_dsa_workspace_size(B, L)
    ws = workspace(ws_n, q.device)
    lib.call("vmk_dsa_decode" + sfx, q.data_ptr(), kv.data_ptr(), iq.data_ptr(), ik.data_ptr(), w.data_ptr(),
             0 if lens is None else lens.data_ptr(), out.data_ptr(), idx.data_ptr(), cnt.data_ptr(), B, L,
             ws.data_ptr(), ws.numel(), _stream(q))
    return out
