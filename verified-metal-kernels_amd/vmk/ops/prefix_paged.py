"""Shared-prefix decode over a paged KV cache: the op contract (shapes, case lists, input generator, standard op).

The reference leaves the paged variant of its shared-prefix kernel out of the package (README.md:141-142; its one
measurement is cases/README.md:13).  This op is ops/prefix.py's attention with the keys and values held in a page
pool, in the layout FlashInfer calls HND:
    q: (N, Hq, D)                                   one decode token per request
    k_pages, v_pages: (num_pages, Hkv, ps, D)       the page pool (fp16 or bf16), ps (page size) a multiple of 32
    prefix_pages: (P / ps,) int32                   the shared prefix's pages, in order
    suffix_pages: (N, max_sp) int32                 each request's suffix pages, in order
    slens: (N,) int32 or None                       suffix rows in use (None: all max_sp * ps)
    layout: "HND", "NHD" or None (HND)              NHD pools are (num_pages, ps, Hkv, D)
A page id outside [0, num_pages) is an absent page: its rows take no part in the softmax.
"""
import math

import numpy as np
import torch

from . import prefix

NAME = "prefix_paged"
HQ, HKV, D = prefix.HQ, prefix.HKV, prefix.D
PS = 64                                                   # default page size
L1_SHAPE = dict(N=4, P=2048, S=256, ps=64)
BENCH_SHAPES = [dict(N=64, P=16384, S=2048, S_min=128, ps=64), dict(N=8, P=2048, S=256, ps=32)]
CONFIGS = {"P2": (dict(N=64, P=16384, S=2048, S_min=128, ps=64), "outlier"),
           "P2n": (dict(N=64, P=16384, S=2048, S_min=128, ps=64, layout="NHD"), "outlier")}   # P2 in NHD pages
FUZZ = [(dict(N=1, P=32, S=1, ps=32), "randn"), (dict(N=3, P=1024, S=77, ps=64), "randn"),
        (dict(N=5, P=4096, S=33, ps=128), "randn"), (dict(N=2, P=96, S=200, ps=96), "randn"),
        (dict(N=7, P=8192, S=700, S_min=1, ps=32), "randn"), (dict(N=4, P=2048, S=256, ps=256), "large"),
        (dict(N=4, P=2048, S=256, ps=64), "needle_prefix"), (dict(N=4, P=2048, S=256, ps=64), "needle_suffix"),
        (dict(N=4, P=2048, S=256, ps=64), "nan_inf"), (dict(N=4, P=2048, S=256, ps=64), "tiny"),
        (dict(N=6, P=3072, S=500, S_min=0, ps=64, absent=3), "randn"), (dict(N=3, P=0, S=300, ps=32), "randn")]
L3_CASES = [(dict(N=8, P=1024, S=128, ps=64), "randn"), (dict(N=8, P=32768, S=1024, ps=128), "randn"),
            (dict(N=16, P=4096, S=512, S_min=1, ps=32), "randn"), (dict(N=4, P=8192, S=512, ps=64), "needle_suffix"),
            (dict(N=64, P=16384, S=2048, S_min=128, ps=64), "outlier")]
EXTRA = [(dict(N=33, P=640, S=40, ps=32, absent=2), "randn"), (dict(N=20, P=40960, S=3000, S_min=1, ps=256), "randn"),
         (dict(N=6, P=1024, S=300, ps=64, dtype="bf16"), "randn"),
         (dict(N=7, P=2048, S=500, S_min=1, ps=128, absent=1, layout="NHD"), "randn")]
L4_CASES = [(dict(N=64, P=16384, S=2048, S_min=128, ps=64), "outlier"), (dict(N=8, P=2048, S=256, ps=32), "randn"),
            (dict(N=12, P=3072, S=2500, S_min=1, ps=128, absent=2), "randn"),
            (dict(N=16, P=4096, S=700, S_min=1, ps=64, layout="NHD"), "randn")]


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """The contiguous op's inputs for (N, P, S, S_min, dist) and seed (vmk.ops.prefix.make_inputs, same draws),
    scattered into a page pool.  A second generator, seeded with (seed, 1), then draws:
      * a random permutation of the page ids: the prefix takes the first P/ps ids, request n the next ceil(S/ps);
      * shape["absent"] (default 0) pages of the prefix and as many suffix pages inside the rows in use, marked
        absent (-1).
    The pool holds 1/8 more pages than used; the spare pages are NaN, so a read of any page the tables do not name
    shows in the output.  Table entries past a request's rows in use are -1.  When S is not a whole number of pages,
    slens = S is passed even without S_min (a suffix without slens fills all its pages).  With shape["layout"] =
    "NHD" the pools are returned as (num_pages, ps, Hkv, D) (to_nhd) and the dict carries layout="NHD"."""
    ps = shape.get("ps", PS)
    N, P, S = shape["N"], shape["P"], shape["S"]
    if P % ps:
        raise ValueError(f"P={P} is not a whole number of pages of {ps}")
    base = {k: v for k, v in shape.items() if k not in ("ps", "absent", "layout")}
    c = prefix.make_inputs(base, seed=seed, dist=dist)
    kp, vp, ks, vs = (c[k] for k in ("kp", "vp", "ks", "vs"))          # CPU tensors of the op's dtype
    slens = None if c["slens"] is None else c["slens"].numpy()
    Hkv, d = kp.shape[0], kp.shape[2]
    npp, nsp = P // ps, -(-S // ps)
    if slens is None and S % ps:                           # suffixes end inside their last page
        slens = np.full((N,), S, np.int32)
    used = npp + N * nsp
    num_pages = used + used // 8 + 1
    rng = np.random.default_rng([seed, 1])
    ids = rng.permutation(num_pages).astype(np.int32)
    kpool = torch.full((num_pages, Hkv, ps, d), float("nan"), dtype=kp.dtype)
    vpool = torch.full((num_pages, Hkv, ps, d), float("nan"), dtype=kp.dtype)
    pp = ids[:npp].copy()
    for i in range(npp):
        kpool[int(pp[i])] = kp[:, i * ps:(i + 1) * ps]
        vpool[int(pp[i])] = vp[:, i * ps:(i + 1) * ps]
    sp = ids[npp:used].reshape(N, nsp).copy()
    for n in range(N):
        for j in range(nsp):
            rows, page = min(ps, S - j * ps), int(sp[n, j])
            kpool[page, :, :rows] = ks[n, :, j * ps:j * ps + rows]
            vpool[page, :, :rows] = vs[n, :, j * ps:j * ps + rows]
            kpool[page, :, rows:] = 0
            vpool[page, :, rows:] = 0
        sn = S if slens is None else int(slens[n])
        sp[n, -(-sn // ps):] = -1                          # entries past the rows in use
    na = shape.get("absent", 0)
    if na:
        if npp:
            pp[rng.choice(npp, min(na, npp), replace=False)] = -1
        for _ in range(na):
            n = int(rng.integers(0, N))
            live = np.flatnonzero(sp[n] >= 0)
            if live.size:
                sp[n, int(rng.choice(live))] = -1
    t = lambda a: torch.from_numpy(a).to(device)
    out = dict(q=c["q"].to(device), k_pages=kpool.to(device), v_pages=vpool.to(device), prefix_pages=t(pp),
               suffix_pages=t(sp), slens=None if slens is None else t(slens))
    if shape.get("layout", "HND") == "NHD":
        out.update(k_pages=to_nhd(out["k_pages"]), v_pages=to_nhd(out["v_pages"]), layout="NHD")
    return out


def to_nhd(pages):
    """The same page pool in the layout FlashInfer calls NHD: (num_pages, Hkv, ps, D) -> (num_pages, ps, Hkv, D)."""
    return pages.transpose(1, 2).contiguous()


def gather(k_pages, v_pages, prefix_pages, suffix_pages, slens=None):
    """Dense per-request caches kf/vf (N, Hkv, P + S, D) with S = max_sp * ps, and a (N, 1, 1, P + S) bool mask of
    the rows present and in use.  Rows of absent pages and rows past slens are zeros and masked out."""
    num_pages, Hkv, ps, d = k_pages.shape
    N, max_sp = suffix_pages.shape
    dev = k_pages.device
    pp, sp = prefix_pages.to(dev).long(), suffix_pages.to(dev).long()
    ok_p = (pp >= 0) & (pp < num_pages)
    ok_s = (sp >= 0) & (sp < num_pages)
    kpre = k_pages[pp.clamp(0, num_pages - 1)].permute(1, 0, 2, 3).reshape(Hkv, -1, d)     # (Hkv, P, D)
    vpre = v_pages[pp.clamp(0, num_pages - 1)].permute(1, 0, 2, 3).reshape(Hkv, -1, d)
    ksuf = k_pages[sp.clamp(0, num_pages - 1)].permute(0, 2, 1, 3, 4).reshape(N, Hkv, -1, d)  # (N, Hkv, S, D)
    vsuf = v_pages[sp.clamp(0, num_pages - 1)].permute(0, 2, 1, 3, 4).reshape(N, Hkv, -1, d)
    P, S = kpre.shape[1], ksuf.shape[2]
    rows = torch.arange(S, device=dev)
    sn = torch.full((N,), S, device=dev) if slens is None else slens.to(dev).long().clamp(0, S)
    m_p = ok_p.repeat_interleave(ps)[None].expand(N, P)
    m_s = ok_s.repeat_interleave(ps, dim=1) & (rows[None, :] < sn[:, None])
    m = torch.cat([m_p, m_s], 1)
    kf = torch.cat([kpre[None].expand(N, -1, -1, -1), ksuf], 2)
    vf = torch.cat([vpre[None].expand(N, -1, -1, -1), vsuf], 2)
    z = torch.zeros((), dtype=kf.dtype, device=dev)
    kf = torch.where(m[:, None, :, None], kf, z)
    vf = torch.where(m[:, None, :, None], vf, z)
    return kf, vf, m[:, None, None, :]


def row_inputs(inp, i):
    """Request i alone: its query, suffix page row and length, with the page pool and prefix pages unchanged."""
    out = dict(inp)
    for k in ("q", "suffix_pages", "slens"):
        if inp.get(k) is not None:
            out[k] = inp[k][i:i + 1]
    return out


# ---------------------------------------------------------------- PyTorch standard op
def torch_naive(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None, layout="HND", **_):
    """Gather the pages into a dense per-request cache, then SDPA with the presence mask (prefix.torch_naive)."""
    import torch.nn.functional as F
    if layout == "NHD":
        k_pages, v_pages = k_pages.transpose(1, 2), v_pages.transpose(1, 2)
    kf, vf, m = gather(k_pages, v_pages, prefix_pages, suffix_pages, slens)
    return F.scaled_dot_product_attention(q[:, :, None, :], kf, vf, attn_mask=m, enable_gqa=True)[:, :, 0, :]


TORCH_REFS = dict(torch_naive=torch_naive)
L1_REF = "torch_naive"
L3_REF = "torch_naive"


def used_rows(shape, slens=None):
    N, S = shape["N"], shape["S"]
    return N * S if slens is None else int(np.asarray(slens).astype(np.int64).sum())


def algorithmic_bytes(shape, slens=None):
    """q + prefix K/V + the used suffix K/V rows + the page tables + the fp16 output."""
    N, P, S, ps = shape["N"], shape["P"], shape["S"], shape.get("ps", PS)
    tables = 4 * (P // ps + N * -(-S // ps))
    return prefix.algorithmic_bytes({k: v for k, v in shape.items() if k != "ps"}, slens) + tables


def flops(shape, slens=None):
    return prefix.flops(shape, slens)


def scale(d=D):
    return 1.0 / math.sqrt(d)
