"""GPU parity of the DSA kernels (libvmk through the C-ABI) against the float64 oracle, plus the exact top-k check."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import dsa

pytestmark = pytest.mark.gpu

CASES = [(s, d, 7 + i) for i, (s, d) in enumerate(dsa.FUZZ)] + [(s, d, 40 + i) for i, (s, d) in
                                                                enumerate(dsa.EXTRA)]
CASES += [(dict(B=2, L=8192), "randn", 100), (dict(B=2, L=8192), "needle", 3)]


@pytest.mark.parametrize("shape,dist,seed", CASES)
def test_dsa_parity(shape, dist, seed):
    import vmk
    print(f"dsa case {shape} {dist} seed={seed}", flush=True)
    inp = dsa.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    B = shape["B"]
    idx = torch.full((B, 2048), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    out = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp["lens"], idx=idx, cnt=cnt)
    torch.cuda.synchronize()
    s64, sel = oracle.dsa.ref_select64(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
    for b in range(B):
        n = shape["L"] if lens is None else int(lens[b])
        ok, det = oracle.dsa.topk_set_check(idx[b], int(cnt[b]), s64[b], n, bound[b])
        assert ok, (b, det)
        print(f"  request {b}: band {det.get('band', 0):.2e} boundary {det.get('boundary', 0)} "
              f"swapped {det.get('swapped', 0)}")
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.dsa.ref64(**inp, sel=sel)
    assert out.shape == tuple(r.shape) and out.dtype == inp["q"].dtype
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2
    # The attention workgroups' arrival counters (and the histograms) are back to zero after the call.
    from vmk import api
    assert int(api.workspace(0, "cuda")[: 4 << 20].count_nonzero().item()) == 0


def test_dsa_kernel_module_matches_entry_points():
    """The kernel(**inputs) module, the fused entry and the two-stage entries give the same output."""
    import vmk
    import dsa_mi355x
    inp = dsa.make_inputs(dict(B=3, L=9000), seed=5, dist="ragged", device="cuda")
    o1 = dsa_mi355x.kernel(**inp)
    idx, cnt = vmk.dsa_indexer_select(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    o2 = vmk.dsa_sparse_mla(inp["q"], inp["kv"], idx, cnt)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def tied_inputs(L, n_high, n_tied, seed):
    """DSA inputs whose indexer scores take three values: n_high positions at 2 s, n_tied at exactly s (identical
    ik rows give identical fp32 scores), the rest at 0 (ik = 0).  With n_high < 2048 < n_high + n_tied, the
    threshold bucket holds the n_tied exact ties, and the select must take the first 2048 - n_high of them in
    position order.  Returns (inputs, expected index set)."""
    B = 2
    inp = dsa.make_inputs(dict(B=B, L=L), seed=seed, dist="randn")
    rng = np.random.default_rng(seed + 1)
    ik = np.zeros((B, L, dsa.DI), dtype=np.float32)
    want = []
    for b in range(B):
        iq = inp["iq"][b].float().numpy()
        w = inp["w"][b].numpy()
        base = (iq * np.sign(w)[:, None]).mean(0) * 8.0
        s = float((w * np.maximum(iq.astype(np.float64) @ base.astype(np.float16).astype(np.float64), 0)).sum())
        assert s > 0
        perm = rng.permutation(L)
        high, tied = np.sort(perm[:n_high]), np.sort(perm[n_high:n_high + n_tied])
        ik[b, tied] = base
        ik[b, high] = 2.0 * base
        want.append(np.concatenate([high, tied[:dsa.TOPK - n_high]]))
    inp["ik"] = torch.from_numpy(ik).half()
    return inp, want


@pytest.mark.parametrize("L,n_high,n_tied", [(16384, 1000, 3000), (16384, 1000, 15384), (70000, 7, 50000)])
def test_dsa_select_exact_ties_broken_by_position(L, n_high, n_tied):
    """More than 4096 tied candidates take the select's global-memory walk; up to 4096 stay in LDS.  Either way the
    picks among equal scores are the lowest positions, and the attention over them matches float64."""
    import vmk
    print(f"dsa ties L={L} high={n_high} tied={n_tied}", flush=True)
    inp, want = tied_inputs(L, n_high, n_tied, seed=11)
    inp = {k: (v.cuda() if v is not None else None) for k, v in inp.items()}
    idx = torch.full((2, 2048), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    out = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], None, idx=idx, cnt=cnt)
    torch.cuda.synchronize()
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    s64, _ = oracle.dsa.ref_select64(inp["iq"], inp["ik"], inp["w"], None)
    bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], None)
    sel = []
    for b in range(2):
        assert cnt[b] == 2048
        ok, det = oracle.dsa.topk_set_check(idx[b], 2048, s64[b], L, bound[b])
        assert ok and det["boundary"] == n_tied, det
        assert np.array_equal(np.sort(idx[b]), np.sort(want[b]))
        sel.append(idx[b].astype(np.int64))
    r = oracle.dsa.ref64(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], sel=sel)
    em, _ = nerr(out.float().cpu().numpy(), r)
    assert em <= 1e-2
    again = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], None)
    torch.cuda.synchronize()
    assert torch.equal(out, again)                    # the histograms were left zero by the first call


def test_dsa_batch_above_64_keeps_histograms_outside_the_head():
    """B > 64 moves the per-request histograms out of the workspace head and zero-fills them first; two calls in a
    row must both select exactly."""
    import vmk
    shape = dict(B=65, L=2500)
    print(f"dsa {shape}", flush=True)
    for seed in (21, 22):
        inp = dsa.make_inputs(shape, seed=seed, dist="randn", device="cuda")
        idx = torch.full((65, 2048), -1, dtype=torch.int32, device="cuda")
        cnt = torch.full((65,), -1, dtype=torch.int32, device="cuda")
        out = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], None, idx=idx, cnt=cnt)
        torch.cuda.synchronize()
        s64, sel = oracle.dsa.ref_select64(inp["iq"], inp["ik"], inp["w"], None)
        bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], None)
        idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
        for b in range(65):
            ok, det = oracle.dsa.topk_set_check(idx[b], int(cnt[b]), s64[b], 2500, bound[b])
            assert ok, (seed, b, det)
        em, _ = nerr(out.float().cpu().numpy(), oracle.dsa.ref64(**inp, sel=sel))
        assert em <= 1e-2


@pytest.mark.parametrize("shape,dist,seed", [(dict(B=2, L=5003), "randn", 61), (dict(B=3, L=9000), "ragged", 62),
                                             (dict(B=4, L=65536), "randn", 0), (dict(B=1, L=1500), "randn", 63)])
def test_dsa_split_entries(shape, dist, seed):
    """llama.cpp's decomposition of the select: vmk_dsa_indexer's scores lie within the fp32 error bound of the
    float64 scores, vmk_dsa_topk picks exactly the top-2048 of the scores it is given (ties by position), and
    the two together give the fused entry's idx and cnt bit for bit."""
    import vmk
    print(f"dsa split entries {shape} {dist} seed={seed}", flush=True)
    inp = dsa.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    B, L = shape["B"], shape["L"]
    scores = vmk.dsa_indexer(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    idx, cnt = vmk.dsa_topk(scores, inp["lens"])
    idx2, cnt2 = vmk.dsa_indexer_select(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    torch.cuda.synchronize()
    assert torch.equal(cnt, cnt2) and torch.equal(idx, idx2)
    s32 = scores.cpu().numpy().astype(np.float64)
    s64 = oracle.dsa.scores64(inp["iq"], inp["ik"], inp["w"])
    bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    for b in range(B):
        n = L if lens is None else int(lens[b])
        assert np.abs(s32[b, :n] - s64[b, :n]).max() <= bound[b]
        k = min(n, 2048)
        assert cnt[b] == k
        want = np.argsort(-s32[b, :n], kind="stable")[:k]           # the fp32 top-k, ties taken by position
        assert np.array_equal(np.sort(idx[b, :k]), np.sort(want)), b


def test_dsa_topk_exact_on_tied_scores():
    """vmk_dsa_topk on scores with large exact ties (more than 4096 equal values at the threshold take the
    global-memory walk): the lowest positions of the tied value are taken."""
    import vmk
    rng = np.random.default_rng(71)
    B, L = 2, 20000
    s = rng.standard_normal((B, L)).astype(np.float32)
    s[0, rng.permutation(L)[:6000]] = 1.25                          # 6000 ties, above about 2000 positions
    s[1, rng.permutation(L)[:300]] = 1.25
    scores = torch.from_numpy(s).cuda()
    idx, cnt = vmk.dsa_topk(scores)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    for b in range(B):
        want = np.argsort(-s[b], kind="stable")[:2048]
        assert np.array_equal(np.sort(idx[b]), np.sort(want)), b


def test_dsa_sparse_mla_counts_outside_the_range():
    """Counts a caller passes to vmk_dsa_sparse_mla are clamped to [0, 2048]: 0 and a negative count give NaN rows
    (the softmax of no keys) without reading any partial, 3000 acts as 2048, and 100 attends over the first 100
    indices."""
    import vmk
    shape = dict(B=4, L=6000)
    print(f"dsa counts outside the range {shape}", flush=True)
    inp = dsa.make_inputs(shape, seed=81, dist="randn", device="cuda")
    idx, _ = vmk.dsa_indexer_select(inp["iq"], inp["ik"], inp["w"])
    cnt = torch.tensor([0, -5, 3000, 100], dtype=torch.int32, device="cuda")
    out = vmk.dsa_sparse_mla(inp["q"], inp["kv"], idx, cnt)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.isnan(o[0]).all() and np.isnan(o[1]).all()
    ix = idx.cpu().numpy().astype(np.int64)
    for b, k in ((2, 2048), (3, 100)):
        sel = [ix[i, :k] for i in range(4)]
        r = oracle.dsa.ref64(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], sel=sel)[b]
        assert np.isfinite(o[b]).all()
        em, _ = nerr(o[b], r)
        assert em <= 1e-2, (b, em)
