"""Paged single-token decode: the op contract (shapes, case lists, input generator, PyTorch standard op).

This build's decode op (vmk.ops.decode) with each request's cache held in a page pool, the way serving engines keep
KV caches.  The reference ships no kernel for it: its one paged variant is the shared-prefix kernel it leaves out of
the package (README.md:141-142).
    q: (B, Hq, D)                                   one query token per request
    k_pages, v_pages: (num_pages, Hkv, ps, D)       the page pool (HND), ps a multiple of 32, or (num_pages, ps, Hkv, D)
                                                    with layout "NHD"
    page_table: (B, max_pages) int32                each request's pages, in order
    lens: (B,) int32 or None                        positions in use (None: all max_pages * ps)
    layout: "HND", "NHD" or None (HND)
A page id outside [0, num_pages) is an absent page: its rows take no part in the softmax.  At most 16 query heads
per KV head.
"""
import numpy as np
import torch

from . import decode

NAME = "decode_paged"
HQ, HKV, D = decode.HQ, decode.HKV, decode.D
PS = 64                                                   # default page size
L1_SHAPE = dict(B=2, L=4096, ps=64)
# D1 on 64-row pages, and D2 on NHD pages.
CONFIGS = {"D1p": (dict(B=1, L=65536, ps=64), "randn"), "D2n": (dict(B=4, L=16384, ps=64, layout="NHD"), "randn")}
FUZZ = [(dict(B=1, L=32, ps=32), "randn"), (dict(B=3, L=77, ps=32), "randn"), (dict(B=2, L=4097, ps=64), "randn"),
        (dict(B=1, L=65536, ps=256), "randn"), (dict(B=5, L=300, ps=96), "large"), (dict(B=2, L=3000, ps=64), "needle"),
        (dict(B=2, L=3000, ps=64), "nan_inf"), (dict(B=2, L=3000, ps=64), "tiny"),
        (dict(B=4, L=1000, Hq=8, Hkv=8, ps=64), "randn"), (dict(B=2, L=2048, Hq=32, Hkv=2, ps=128), "randn"),
        (dict(B=7, L=33, ps=32), "randn"), (dict(B=3, L=5000, L_min=1, ps=64, absent=2), "randn")]
L3_CASES = [(dict(B=2, L=8192, ps=64), "randn"), (dict(B=1, L=32768, ps=128), "randn"),
            (dict(B=4, L=4096, ps=64), "large"), (dict(B=2, L=8192, ps=64), "needle"), (dict(B=8, L=2048, ps=32), "randn")]
EXTRA = [(dict(B=6, L=5000, L_min=1, ps=64, absent=2), "randn"), (dict(B=4, L=5000, L_min=1, ps=64, dtype="bf16"), "randn"),
         (dict(B=3, L=3000, ps=96, absent=1, layout="NHD"), "randn"),
         (dict(B=2, L=6000, L_min=1, ps=64, layout="NHD", dtype="bf16"), "randn")]
L4_CASES = [(dict(B=8, L=8192, ps=64), "randn"), (dict(B=6, L=5000, L_min=1, ps=64, absent=1), "randn"),
            (dict(B=4, L=4096, ps=64, layout="NHD"), "randn")]


def row_inputs(inp, i):
    """Request i alone: its query, page-table row and length, with the page pool unchanged."""
    out = dict(inp)
    for k in ("q", "page_table", "lens"):
        if inp.get(k) is not None:
            out[k] = inp[k][i:i + 1]
    return out


def to_nhd(pages):
    """The same page pool in the layout FlashInfer calls NHD: (num_pages, Hkv, ps, D) -> (num_pages, ps, Hkv, D)."""
    return pages.transpose(1, 2).contiguous()


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """The decode op's inputs for (B, L, L_min, Hq, Hkv, dtype, dist) and seed (vmk.ops.decode.make_inputs, same
    draws), scattered into a page pool.  A second generator, seeded with (seed, 1), then draws a permutation of the
    page ids (request b takes the ids b * max_pages ..) and shape["absent"] (default 0) pages inside the rows in use,
    marked absent (-1).  The pool holds 1/8 more pages than used; the spare pages are NaN, so a read of any page the
    table does not name shows in the output.  Table entries past a request's rows in use are -1.  When L is not a
    whole number of pages, lens = L is passed even without L_min."""
    ps = shape.get("ps", PS)
    B, L = shape["B"], shape["L"]
    base = {k: v for k, v in shape.items() if k not in ("ps", "absent", "layout")}
    c = decode.make_inputs(base, seed=seed, dist=dist)
    k, v = c["k"], c["v"]                                       # CPU (B, Hkv, L, D) of the op's dtype
    lens = None if c["lens"] is None else c["lens"].numpy()
    if lens is None and L % ps:
        lens = np.full((B,), L, np.int32)
    Hkv, d = k.shape[1], k.shape[3]
    mp = -(-L // ps)
    used = B * mp
    num_pages = used + used // 8 + 1
    rng = np.random.default_rng([seed, 1])
    table = rng.permutation(num_pages).astype(np.int32)[:used].reshape(B, mp).copy()
    kpool = torch.full((num_pages, Hkv, ps, d), float("nan"), dtype=k.dtype)
    vpool = torch.full((num_pages, Hkv, ps, d), float("nan"), dtype=k.dtype)
    for b in range(B):
        for j in range(mp):
            rows, page = min(ps, L - j * ps), int(table[b, j])
            kpool[page, :, :rows] = k[b, :, j * ps:j * ps + rows]
            vpool[page, :, :rows] = v[b, :, j * ps:j * ps + rows]
            kpool[page, :, rows:] = 0
            vpool[page, :, rows:] = 0
        n = L if lens is None else min(max(int(lens[b]), 1), L)
        table[b, -(-n // ps):] = -1                             # entries past the rows in use
    for _ in range(shape.get("absent", 0)):
        b = int(rng.integers(0, B))
        live = np.flatnonzero(table[b] >= 0)
        if live.size:
            table[b, int(rng.choice(live))] = -1
    t = lambda a: torch.from_numpy(a).to(device)
    out = dict(q=c["q"].to(device), k_pages=kpool.to(device), v_pages=vpool.to(device), page_table=t(table),
               lens=None if lens is None else t(lens))
    if shape.get("layout", "HND") == "NHD":
        out.update(k_pages=to_nhd(out["k_pages"]), v_pages=to_nhd(out["v_pages"]), layout="NHD")
    return out


def gather(k_pages, v_pages, page_table, lens=None, layout="HND"):
    """Dense caches k, v (B, Hkv, max_pages * ps, D) and a (B, 1, 1, max_pages * ps) bool mask of the rows present
    and in use (lens clamped to [1, max_pages * ps]).  Rows of absent pages are zeros and masked out."""
    if layout == "NHD":
        k_pages, v_pages = k_pages.transpose(1, 2), v_pages.transpose(1, 2)
    num_pages, Hkv, ps, d = k_pages.shape
    B, mp = page_table.shape
    dev = k_pages.device
    pt = page_table.to(dev).long()
    ok = (pt >= 0) & (pt < num_pages)
    k = k_pages[pt.clamp(0, num_pages - 1)].permute(0, 2, 1, 3, 4).reshape(B, Hkv, mp * ps, d)
    v = v_pages[pt.clamp(0, num_pages - 1)].permute(0, 2, 1, 3, 4).reshape(B, Hkv, mp * ps, d)
    L = mp * ps
    n = torch.full((B,), L, device=dev) if lens is None else lens.to(dev).long().clamp(1, L)
    m = ok.repeat_interleave(ps, dim=1) & (torch.arange(L, device=dev)[None, :] < n[:, None])
    z = torch.zeros((), dtype=k.dtype, device=dev)
    k = torch.where(m[:, None, :, None], k, z)
    v = torch.where(m[:, None, :, None], v, z)
    return k, v, m[:, None, None, :]


# ---------------------------------------------------------------- PyTorch standard op
def torch_sdpa(q, k_pages, v_pages, page_table, lens=None, layout="HND", **_):
    """Gather the pages into a dense cache, then SDPA with the presence mask (decode.torch_sdpa)."""
    import torch.nn.functional as F
    k, v, m = gather(k_pages, v_pages, page_table, lens, layout)
    return F.scaled_dot_product_attention(q[:, :, None, :], k, v, attn_mask=m, enable_gqa=True)[:, :, 0, :]


TORCH_REFS = dict(torch_sdpa=torch_sdpa)
L1_REF = "torch_sdpa"
L3_REF = "torch_sdpa"


def algorithmic_bytes(shape, lens=None):
    """q + the K/V rows in use + the page table + the fp16 output."""
    B, L, ps = shape["B"], shape["L"], shape.get("ps", PS)
    return decode.algorithmic_bytes({k: v for k, v in shape.items() if k not in ("ps", "absent", "layout")}, lens) + \
        4 * B * (-(-L // ps))


def flops(shape, lens=None):
    return decode.flops(shape, lens)


def softmax_scale(d=D):
    return decode.softmax_scale(d)
