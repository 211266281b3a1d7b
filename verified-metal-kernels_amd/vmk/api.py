"""torch-facing wrappers of the libvmk C-ABI: argument checks, output and workspace allocation, stream plumbing.

Every wrapper launches on `torch.cuda.current_stream()` of the inputs' device and returns without synchronising.
Arguments are checked in this order: types, dtypes and ranks, then shapes against each other, then that every
tensor is on a ROCm device, so a wrongly shaped tensor is refused before any GPU work.

Workspaces come from one cached byte buffer per device.  Calls that overlap on two streams of one device would
share it, so they must be ordered by the caller.  The buffer only grows, at least doubling each time, so a growing
workload reallocates O(log) times.  A buffer it outgrows is freed (after the device's queued work) unless a HIP graph
was captured while it was current: such a graph still addresses it, so it is kept alive until the process ends.
Growth is refused while the current stream is capturing (`reserve_workspace` beforehand, or one eager call of the
largest shape, avoids it).  After a call that failed at launch (return code 2) the buffer is set aside the same
way and the next call starts from a fresh zeroed one, since a call that stops half-way can leave the workspace head
(which must stay zero between calls) non-zero; a call refused on the host (code 1) launched nothing and keeps it.
"""
import ctypes

import torch

from . import lib

_ws = {}
_captured = set()      # devices whose current workspace was handed out during a HIP graph capture
_retired = []          # workspaces a captured graph may still address, kept alive until the process ends
_dev_ok = {}
HEAD_BYTES = 4 << 20   # VMK_WORKSPACE_HEAD of include/vmk.h: must be zero before a call, is zero after it
MIN_WORKSPACE = 1 << 20


def _alloc(nbytes, key):
    return torch.zeros(nbytes, dtype=torch.uint8, device=torch.device("cuda", key))


def _capturing():
    return torch.cuda.is_current_stream_capturing()


def _drain(key):
    torch.cuda.synchronize(key)


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


def _dev_index(device):
    dev = torch.device(device)
    return dev.index if dev.index is not None else torch.cuda.current_device()


def workspace(nbytes, device):
    """A cached uint8 buffer of at least `nbytes` on `device`, allocated zeroed (the head must start at zero)."""
    key = _dev_index(device)
    buf = _ws.get(key)
    capturing = _capturing()
    if buf is None or buf.numel() < nbytes:
        if capturing:
            raise lib.VmkError(f"the libvmk workspace would have to grow to {int(nbytes)} bytes during HIP graph "
                               "capture; call vmk.reserve_workspace (or the op once, eagerly) before capturing")
        size = max(int(nbytes), MIN_WORKSPACE)
        if buf is not None:
            size = max(size, 2 * buf.numel())
            _set_aside(key)
        buf = _alloc(size, key)
        _ws[key] = buf
    if capturing:
        _captured.add(key)
    return buf


def _set_aside(key):
    """Takes device `key`'s workspace out of use: kept alive until the process ends when a graph was captured over
    it, else released to torch's allocator once the work queued on the device (any stream) has finished."""
    buf = _ws.pop(key)
    if key in _captured:
        _captured.discard(key)
        _retired.append(buf)
        return
    try:
        _drain(key)
    except RuntimeError:            # the device reports an error: keep the buffer rather than risk a reuse race
        _retired.append(buf)


def reserve_workspace(nbytes, device="cuda"):
    """Grows the cached workspace of `device` to at least `nbytes` now (before a HIP graph capture)."""
    return workspace(nbytes, device)


def _launch(name, ws, *args):
    """Calls entry point `name`; after a launch or runtime failure the workspace `ws` is set aside before the error
    propagates (a refusal of the arguments launched nothing and leaves it in use)."""
    try:
        lib.call(name, *args)
    except lib.VmkError as e:
        key = ws.device.index
        if e.code != lib.REJECTED and _ws.get(key) is ws:
            _set_aside(key)
        raise


def _stream(t):
    return ctypes_ptr(torch.cuda.current_stream(t.device).cuda_stream)


def ctypes_ptr(x):
    return int(x)


def _need(t, name, dtype, ndim):
    """Type, dtype, rank and layout of one tensor argument (its device is checked later, by `_resident`)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _need_out(out, like):
    """A caller's output tensor must have the dtype and shape of `like` (the kernels write exactly that many rows)."""
    if out is None:
        return
    _need(out, "out", like.dtype, like.dim())
    if tuple(out.shape) != tuple(like.shape):
        raise ValueError(f"out {tuple(out.shape)}: expected {tuple(like.shape)}")


def _resident(**tensors):
    """Every given tensor (None skipped) is on the same ROCm device; then that device is checked once."""
    dev = None
    for name, t in tensors.items():
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a ROCm device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{name} is on {t.device}, the other arguments on {dev}")
    device_ok(dev)


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
    if tuple(words.shape) != (B, kd, (kd + 31) // 32):
        raise ValueError(f"bits shape {tuple(words.shape)} is not (B, kd, ceil(kd/32)) = {(B, kd, (kd + 31) // 32)}")
    _need_out(out, q)
    _resident(q=q, k=k, v=v, bits=words, out=out)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_spec_workspace_size(B, kd, Hq, Hkv, D, L)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported spec shape B={B} kd={kd} Hq={Hq} Hkv={Hkv} D={D} L={L}")
    ws = workspace(ws_n, q.device)
    _launch("vmk_spec_verify" + sfx, ws, q.data_ptr(), k.data_ptr(), v.data_ptr(), words.data_ptr(), out.data_ptr(),
            B, kd, Hq, Hkv, D, L, words.shape[2], ws.data_ptr(), ws.numel(), _stream(q))
    return out


def spec_verify_noalloc(q, k, v, words, out):
    """vmk_spec_verify_noalloc: spec_verify without a workspace (the library's static per-GPU scratch holds the
    partials), for callers that cannot allocate; fp16 only, `out` (B, kd, Hq, 128) fp16 given by the caller.  Calls
    that overlap on one GPU race on that scratch.  Shapes whose partials exceed vmk_spec_noalloc_max_bytes() are
    refused with VmkError."""
    _need(q, "q", torch.float16, 4)
    _need(k, "k", torch.float16, 4)
    _need(v, "v", torch.float16, 4)
    _need(words, "bits", torch.int32, 3)
    _need(out, "out", torch.float16, 4)
    B, kd, Hq, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    if tuple(k.shape) != (B, Hkv, L, D) or tuple(v.shape) != tuple(k.shape) or tuple(out.shape) != tuple(q.shape):
        raise ValueError(f"k/v/out shapes {tuple(k.shape)}/{tuple(v.shape)}/{tuple(out.shape)} do not match q "
                         f"{tuple(q.shape)}")
    if tuple(words.shape) != (B, kd, (kd + 31) // 32):
        raise ValueError(f"bits shape {tuple(words.shape)} is not (B, kd, ceil(kd/32)) = {(B, kd, (kd + 31) // 32)}")
    _resident(q=q, k=k, v=v, bits=words, out=out)
    with torch.cuda.device(q.device):           # the scratch of q's GPU, launched on that GPU's current stream
        lib.call("vmk_spec_verify_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), words.data_ptr(),
                 out.data_ptr(), B, kd, Hq, Hkv, D, L, words.shape[2], _stream(q))
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
    _need_out(out, q)
    _resident(q=q, k=k, v=v, lens=lens, out=out)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_decode_workspace_size(B, Hq, Hkv, D, L)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported decode shape B={B} Hq={Hq} Hkv={Hkv} D={D} L={L}")
    ws = workspace(ws_n, q.device)
    _launch("vmk_decode" + sfx, ws, q.data_ptr(), k.data_ptr(), v.data_ptr(), 0 if lens is None else lens.data_ptr(),
            out.data_ptr(), B, Hq, Hkv, D, L, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def decode_paged(q, k_pages, v_pages, page_table, lens=None, out=None, layout="HND"):
    """Single-token decode over a page pool: q (B, Hq, 128); k_pages/v_pages (num_pages, Hkv, page_size, 128) for
    layout "HND" or (num_pages, page_size, Hkv, 128) for "NHD", page_size a multiple of 32, all fp16 or all bf16;
    page_table (B, max_pages) int32; lens (B,) int32 or None (all max_pages * page_size).  Page ids outside
    [0, num_pages) are absent pages (left out).  Returns out (B, Hq, 128) of q's dtype."""
    if layout not in ("HND", "NHD"):
        raise ValueError(f"layout {layout!r}: expected 'HND' or 'NHD'")
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    for t, n in ((k_pages, "k_pages"), (v_pages, "v_pages")):
        _need(t, n, dt, 4)
    _need(page_table, "page_table", torch.int32, 2)
    B, Hq, D = q.shape
    if layout == "HND":
        num_pages, Hkv, ps = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
        want = (num_pages, Hkv, ps, D)
    else:
        num_pages, ps, Hkv = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
        want = (num_pages, ps, Hkv, D)
    if tuple(k_pages.shape) != want or tuple(v_pages.shape) != tuple(k_pages.shape):
        raise ValueError(f"k_pages {tuple(k_pages.shape)} / v_pages {tuple(v_pages.shape)}: expected {want} ({layout})")
    if page_table.shape[0] != B:
        raise ValueError("page_table must have B rows")
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
        if lens.shape[0] != B:
            raise ValueError("lens must have B entries")
    mp = page_table.shape[1]
    _need_out(out, q)
    _resident(q=q, k_pages=k_pages, v_pages=v_pages, page_table=page_table, lens=lens, out=out)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_decode_paged_workspace_size(B, Hq, Hkv, D, ps, mp)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported paged decode shape B={B} Hq={Hq} Hkv={Hkv} D={D} page_size={ps} "
                           f"max_pages={mp}")
    ws = workspace(ws_n, q.device)
    entry = "vmk_decode_paged" + ("_nhd" if layout == "NHD" else "") + sfx
    _launch(entry, ws, q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), page_table.data_ptr(),
            0 if lens is None else lens.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, num_pages, ps, mp,
            ws.data_ptr(), ws.numel(), _stream(q))
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
    _need_out(out, q)
    _resident(q=q, kp=kp, vp=vp, ks=ks, vs=vs, slens=slens, out=out)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_prefix_workspace_size(N, Hq, Hkv, D, P, S, 0 if slens is None else 1)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported prefix shape N={N} Hq={Hq} Hkv={Hkv} D={D} P={P} S={S}")
    ws = workspace(ws_n, q.device)
    _launch("vmk_prefix_decode" + sfx, ws, q.data_ptr(), kp.data_ptr(), vp.data_ptr(), ks.data_ptr(), vs.data_ptr(),
            0 if slens is None else slens.data_ptr(), out.data_ptr(), N, Hq, Hkv, D, P, S,
            0 if slens is None else 1, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def prefix_decode_paged(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None, out=None, layout="HND"):
    """Shared-prefix decode over a paged cache.  q (N, Hq, 128); k_pages/v_pages (num_pages, Hkv, page_size, 128)
    for layout "HND" or (num_pages, page_size, Hkv, 128) for "NHD", with page_size a multiple of 32, all fp16 or
    all bf16; prefix_pages (P / page_size,) int32; suffix_pages (N, max_sp) int32; slens (N,) int32 or None (full
    suffixes).  Page ids outside [0, num_pages) are absent pages (left out).  Returns out (N, Hq, 128) of q's
    dtype; both layouts give the same bits for the same logical cache."""
    if layout not in ("HND", "NHD"):
        raise ValueError(f"layout {layout!r}: expected 'HND' or 'NHD'")
    dt, sfx = _elem(q)
    _need(q, "q", dt, 3)
    for t, n in ((k_pages, "k_pages"), (v_pages, "v_pages")):
        _need(t, n, dt, 4)
    _need(prefix_pages, "prefix_pages", torch.int32, 1)
    _need(suffix_pages, "suffix_pages", torch.int32, 2)
    N, Hq, D = q.shape
    if layout == "HND":
        num_pages, Hkv, ps = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
        want = (num_pages, Hkv, ps, D)
    else:
        num_pages, ps, Hkv = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
        want = (num_pages, ps, Hkv, D)
    if tuple(k_pages.shape) != want or tuple(v_pages.shape) != tuple(k_pages.shape):
        raise ValueError(f"k_pages {tuple(k_pages.shape)} / v_pages {tuple(v_pages.shape)}: expected {want} ({layout})")
    if suffix_pages.shape[0] != N:
        raise ValueError("suffix_pages must have N rows")
    if slens is not None:
        _need(slens, "slens", torch.int32, 1)
        if slens.shape[0] != N:
            raise ValueError("slens must have N entries")
    P, max_sp = prefix_pages.shape[0] * ps, suffix_pages.shape[1]
    _need_out(out, q)
    _resident(q=q, k_pages=k_pages, v_pages=v_pages, prefix_pages=prefix_pages, suffix_pages=suffix_pages,
              slens=slens, out=out)
    if out is None:
        out = torch.empty_like(q)
    ws_n = lib.load().vmk_prefix_paged_workspace_size(N, Hq, Hkv, D, P, ps, max_sp)
    if ws_n == 0:
        raise lib.VmkError(f"unsupported paged prefix shape N={N} Hq={Hq} Hkv={Hkv} D={D} P={P} page_size={ps} "
                           f"max_suffix_pages={max_sp}")
    ws = workspace(ws_n, q.device)
    entry = "vmk_prefix_decode_paged" + ("_nhd" if layout == "NHD" else "") + sfx
    _launch(entry, ws, q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(),
            prefix_pages.data_ptr() if P else 0, suffix_pages.data_ptr() if max_sp else 0,
            0 if slens is None else slens.data_ptr(), out.data_ptr(), N, Hq, Hkv, D, num_pages, ps, P, max_sp,
            ws.data_ptr(), ws.numel(), _stream(q))
    return out


DSA_H, DSA_DK, DSA_DC, DSA_HI, DSA_DI, DSA_TOPK = 128, 576, 512, 64, 128, 2048


def _dsa_indexer_shapes(iq, ik, w, lens):
    """Checks of the indexer inputs; returns (B, L)."""
    dt, _ = _elem(iq)
    _need(iq, "iq", dt, 3)
    _need(ik, "ik", dt, 3)
    _need(w, "w", torch.float32, 2)
    B, L = ik.shape[0], ik.shape[1]
    if tuple(iq.shape) != (B, DSA_HI, DSA_DI) or tuple(ik.shape) != (B, L, DSA_DI) or tuple(w.shape) != (B, DSA_HI):
        raise ValueError(f"iq {tuple(iq.shape)}, ik {tuple(ik.shape)}, w {tuple(w.shape)}: expected (B,64,128), "
                         "(B,L,128), (B,64)")
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
        if lens.shape[0] != B:
            raise ValueError(f"lens has {lens.shape[0]} entries, expected B = {B}")
    return B, L


def _dsa_attention_shapes(q, kv, B):
    """Checks of the attention inputs against B; returns L."""
    dt, _ = _elem(q)
    _need(q, "q", dt, 3)
    _need(kv, "kv", dt, 3)
    if tuple(q.shape) != (B, DSA_H, DSA_DK) or kv.shape[0] != B or kv.shape[2] != DSA_DK:
        raise ValueError(f"q {tuple(q.shape)} / kv {tuple(kv.shape)}: expected (B,128,576) / (B,L,576), B = {B}")
    return kv.shape[1]


def _selection_shapes(idx, cnt, B):
    _need(idx, "idx", torch.int32, 2)
    _need(cnt, "cnt", torch.int32, 1)
    if tuple(idx.shape) != (B, DSA_TOPK) or tuple(cnt.shape) != (B,):
        raise ValueError(f"idx {tuple(idx.shape)} / cnt {tuple(cnt.shape)}: expected ({B}, 2048) / ({B},)")


def dsa_indexer_select(iq, ik, w, lens=None, idx=None, cnt=None):
    """Indexer scores + exact top-2048 per request; iq/ik both fp16 or both bf16, w fp32.  Returns idx (B, 2048)
    int32 (unordered, first cnt[b] valid) and cnt (B,) int32."""
    _, sfx = _elem(iq)
    B, L = _dsa_indexer_shapes(iq, ik, w, lens)
    if idx is not None or cnt is not None:
        if idx is None or cnt is None:
            raise ValueError("give both idx and cnt, or neither")
        _selection_shapes(idx, cnt, B)
    _resident(iq=iq, ik=ik, w=w, lens=lens, idx=idx, cnt=cnt)
    if idx is None:
        idx = torch.empty(B, DSA_TOPK, dtype=torch.int32, device=ik.device)
        cnt = torch.empty(B, dtype=torch.int32, device=ik.device)
    ws = workspace(lib.load().vmk_dsa_workspace_size(B, L), ik.device)
    _launch("vmk_dsa_indexer_select" + sfx, ws, iq.data_ptr(), ik.data_ptr(), w.data_ptr(),
            0 if lens is None else lens.data_ptr(), idx.data_ptr(), cnt.data_ptr(), B, L, ws.data_ptr(),
            ws.numel(), _stream(ik))
    return idx, cnt


def dsa_indexer(iq, ik, w, lens=None, scores=None):
    """Indexer scores alone: score[b, l] = sum_h w[b, h] * max(iq[b, h] . ik[b, l], 0) in fp32; iq/ik both fp16 or
    both bf16, w fp32.  Returns scores (B, L) float32; positions at or past lens[b] are left as they were."""
    _, sfx = _elem(iq)
    B, L = _dsa_indexer_shapes(iq, ik, w, lens)
    if scores is not None:
        _need(scores, "scores", torch.float32, 2)
        if tuple(scores.shape) != (B, L):
            raise ValueError(f"scores {tuple(scores.shape)}: expected ({B}, {L})")
    _resident(iq=iq, ik=ik, w=w, lens=lens, scores=scores)
    if scores is None:
        scores = torch.empty(B, L, dtype=torch.float32, device=ik.device)
    ws = workspace(lib.load().vmk_dsa_workspace_size(B, L), ik.device)
    _launch("vmk_dsa_indexer" + sfx, ws, iq.data_ptr(), ik.data_ptr(), w.data_ptr(),
            0 if lens is None else lens.data_ptr(), scores.data_ptr(), B, L, ws.data_ptr(), ws.numel(), _stream(ik))
    return scores


def dsa_topk(scores, lens=None, idx=None, cnt=None):
    """Exact top-2048 of given fp32 scores (B, L) per request, among the first lens[b] positions; the same picks in
    the same order as dsa_indexer_select for the same scores.  Returns idx (B, 2048) int32 and cnt (B,) int32."""
    _need(scores, "scores", torch.float32, 2)
    B, L = scores.shape
    if lens is not None:
        _need(lens, "lens", torch.int32, 1)
        if lens.shape[0] != B:
            raise ValueError(f"lens has {lens.shape[0]} entries, expected B = {B}")
    if idx is not None or cnt is not None:
        if idx is None or cnt is None:
            raise ValueError("give both idx and cnt, or neither")
        _selection_shapes(idx, cnt, B)
    _resident(scores=scores, lens=lens, idx=idx, cnt=cnt)
    if idx is None:
        idx = torch.empty(B, DSA_TOPK, dtype=torch.int32, device=scores.device)
        cnt = torch.empty(B, dtype=torch.int32, device=scores.device)
    ws = workspace(lib.load().vmk_dsa_workspace_size(B, L), scores.device)
    _launch("vmk_dsa_topk", ws, scores.data_ptr(), 0 if lens is None else lens.data_ptr(), idx.data_ptr(),
            cnt.data_ptr(), B, L, ws.data_ptr(), ws.numel(), _stream(scores))
    return idx, cnt


def dsa_sparse_mla(q, kv, idx, cnt, out=None):
    """Sparse absorbed-MLA attention of q (B,128,576) over rows kv[b, idx[b, :cnt[b]]], q/kv both fp16 or both bf16;
    idx (B, 2048) int32, cnt (B,) int32 (clamped to [0, 2048]; a request with cnt 0 gets NaN rows).  Returns
    (B,128,512) of q's dtype."""
    dt, sfx = _elem(q)
    _need(idx, "idx", torch.int32, 2)
    B = idx.shape[0]
    L = _dsa_attention_shapes(q, kv, B)
    _selection_shapes(idx, cnt, B)
    if out is not None:
        _need(out, "out", dt, 3)
        if tuple(out.shape) != (B, DSA_H, DSA_DC):
            raise ValueError(f"out {tuple(out.shape)}: expected ({B}, 128, 512)")
    _resident(q=q, kv=kv, idx=idx, cnt=cnt, out=out)
    if out is None:
        out = torch.empty(B, DSA_H, DSA_DC, dtype=dt, device=q.device)
    ws = workspace(lib.load().vmk_dsa_workspace_size(B, L), q.device)
    _launch("vmk_dsa_sparse_mla" + sfx, ws, q.data_ptr(), kv.data_ptr(), idx.data_ptr(), cnt.data_ptr(),
            out.data_ptr(), B, L, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def dsa_decode(q, kv, iq, ik, w, lens=None, out=None, idx=None, cnt=None, single=False):
    """Full DSA decode step (indexer -> top-2048 -> sparse MLA); q, kv, iq, ik all fp16 or all bf16, w fp32.
    Returns out (B,128,512) of q's dtype; the selected indices land in `idx`/`cnt` when given.  single=True runs
    the step as one kernel launch (vmk_dsa_decode_single: the same outputs bit for bit; a grid-barrier wait that
    gave up shows as cnt = -1)."""
    dt, sfx = _elem(q)
    B, L = _dsa_indexer_shapes(iq, ik, w, lens)
    if _dsa_attention_shapes(q, kv, B) != L:
        raise ValueError(f"kv has {kv.shape[1]} positions, ik {L}")
    if iq.dtype != dt:
        raise TypeError(f"iq/ik are {iq.dtype}, q/kv {dt}: all four must share one dtype")
    if out is not None:
        _need(out, "out", dt, 3)
        if tuple(out.shape) != (B, DSA_H, DSA_DC):
            raise ValueError(f"out {tuple(out.shape)}: expected ({B}, 128, 512)")
    if idx is not None or cnt is not None:
        if idx is None or cnt is None:
            raise ValueError("give both idx and cnt, or neither")
        _selection_shapes(idx, cnt, B)
    _resident(q=q, kv=kv, iq=iq, ik=ik, w=w, lens=lens, out=out, idx=idx, cnt=cnt)
    if out is None:
        out = torch.empty(B, DSA_H, DSA_DC, dtype=dt, device=q.device)
    if idx is None:
        idx = torch.empty(B, DSA_TOPK, dtype=torch.int32, device=q.device)
        cnt = torch.empty(B, dtype=torch.int32, device=q.device)
    ws = workspace(lib.load().vmk_dsa_workspace_size(B, L), q.device)
    _launch("vmk_dsa_decode" + ("_single" if single else "") + sfx, ws, q.data_ptr(), kv.data_ptr(), iq.data_ptr(),
            ik.data_ptr(), w.data_ptr(),
            0 if lens is None else lens.data_ptr(), out.data_ptr(), idx.data_ptr(), cnt.data_ptr(), B, L,
            ws.data_ptr(), ws.numel(), _stream(q))
    return out


# ---------------------------------------------------------------------------------------------- DSA projections
def dsa_project(x, pos, rope_cos, rope_sin, weights, kv, ik, q=None, iq=None, w=None):
    """The projections that make the DSA op's inputs for one new token per request (include/vmk.h,
    vmk_dsa_project): x (B, 7168) and the matrices of `weights` (a dict with the fields of vmk_dsa_project_weights)
    fp16 or bf16, norm weights fp32, pos (B,) int32, rope_cos/rope_sin (rows, 32) fp32.  Writes row pos[b] of the
    caches kv (B, L, 576) and ik (B, L, 128) (when 0 <= pos[b] < L) and returns q (B,128,576), iq (B,64,128) of x's
    dtype and w (B,64) fp32."""
    from .ops import dsa_project as op
    dt, sfx = _elem(x)
    _need(x, "x", dt, 2)
    B = x.shape[0]
    if x.shape[1] != op.DIM:
        raise ValueError(f"x {tuple(x.shape)}: expected (B, {op.DIM})")
    _need(pos, "pos", torch.int32, 1)
    if pos.shape[0] != B:
        raise ValueError(f"pos {tuple(pos.shape)}: expected ({B},)")
    _need(rope_cos, "rope_cos", torch.float32, 2)
    _need(rope_sin, "rope_sin", torch.float32, 2)
    if rope_cos.shape != rope_sin.shape or rope_cos.shape[1] != op.DR // 2 or rope_cos.shape[0] < 1:
        raise ValueError(f"rope tables {tuple(rope_cos.shape)}, {tuple(rope_sin.shape)}: expected (rows, 32) each")
    if not isinstance(weights, dict) or set(weights) != set(lib.PROJECT_WEIGHT_FIELDS):
        raise ValueError(f"weights must be a dict with exactly the keys {lib.PROJECT_WEIGHT_FIELDS}")
    for name, shape in op.WEIGHT_SHAPES.items():
        _need(weights[name], name, torch.float32 if name in op.NORMS else dt, len(shape))
        if tuple(weights[name].shape) != shape:
            raise ValueError(f"{name} {tuple(weights[name].shape)}: expected {shape}")
    _need(kv, "kv", dt, 3)
    _need(ik, "ik", dt, 3)
    L = kv.shape[1]
    if tuple(kv.shape) != (B, L, op.DC + op.DR) or tuple(ik.shape) != (B, L, op.DI):
        raise ValueError(f"kv {tuple(kv.shape)}, ik {tuple(ik.shape)}: expected ({B}, L, 576), ({B}, L, 128)")
    for name, t, shape, tdt in (("q", q, (B, op.H, op.DC + op.DR), dt), ("iq", iq, (B, op.HI, op.DI), dt),
                                ("w", w, (B, op.HI), torch.float32)):
        if t is not None:
            _need(t, name, tdt, len(shape))
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} {tuple(t.shape)}: expected {shape}")
    _resident(x=x, pos=pos, rope_cos=rope_cos, rope_sin=rope_sin, kv=kv, ik=ik, q=q, iq=iq, w=w, **weights)
    dev = x.device
    q = torch.empty(B, op.H, op.DC + op.DR, dtype=dt, device=dev) if q is None else q
    iq = torch.empty(B, op.HI, op.DI, dtype=dt, device=dev) if iq is None else iq
    w = torch.empty(B, op.HI, dtype=torch.float32, device=dev) if w is None else w
    wts = lib.DsaProjectWeights(*[weights[name].data_ptr() for name in lib.PROJECT_WEIGHT_FIELDS])
    ws = workspace(lib.load().vmk_dsa_project_workspace_size(B), dev)
    _launch("vmk_dsa_project" + sfx, ws, x.data_ptr(), pos.data_ptr(), rope_cos.data_ptr(), rope_sin.data_ptr(),
            rope_cos.shape[0], ctypes.addressof(wts), q.data_ptr(), iq.data_ptr(), w.data_ptr(), kv.data_ptr(),
            ik.data_ptr(), B, L, ws.data_ptr(), ws.numel(), _stream(x))
    return q, iq, w
