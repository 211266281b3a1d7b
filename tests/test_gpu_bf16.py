"""bf16 inputs on the GPU (the _bf16 entry points of libvmk) against the float64 oracle, which reads the same bf16
values.  The reference kernels read fp16 only (README.md:140).  Tolerance: the verifier's L2 bar (normalised max
error <= 1e-2 and the oracle's NaN/Inf pattern after rounding to bf16)."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import KEYS, decode, dsa, prefix, prefix_paged, spec

pytestmark = pytest.mark.gpu

CASES = [("spec", dict(B=4, L=32768, k=8, dtype="bf16"), "chain", 1),
         ("spec", dict(B=2, L=8192, k=64, dtype="bf16"), "tree_bd", 2),
         ("spec", dict(B=2, L=3000, k=8, dtype="bf16"), "large", 3),
         ("spec", dict(B=2, L=3000, k=8, dtype="bf16"), "nan_inf", 4),
         ("decode", dict(B=8, L=8192, dtype="bf16"), "randn", 5),
         ("decode", dict(B=6, L=5000, L_min=1, dtype="bf16"), "needle", 6),
         ("prefix", dict(N=64, P=16384, S=2048, S_min=128, dtype="bf16"), "outlier", 7),
         ("prefix", dict(N=8, P=2048, S=256, dtype="bf16"), "randn", 8),
         ("prefix", dict(N=20, P=5000, S=3000, S_min=1, dtype="bf16"), "tiny", 9),
         ("prefix", dict(N=4, P=8192, S=256, S_min=1, dtype="bf16"), "randn", 11),   # single-wave prefix units
         ("prefix_paged", dict(N=12, P=3072, S=700, S_min=1, ps=64, absent=2, dtype="bf16"), "randn", 10)]
OPS = {"spec": spec, "decode": decode, "prefix": prefix, "prefix_paged": prefix_paged, "dsa": dsa}


def kernel_of(opname):
    import decode_mi355x
    import dsa_mi355x
    import prefix_mi355x
    import prefix_paged_mi355x
    import spec_mi355x
    return {"spec": spec_mi355x, "decode": decode_mi355x, "prefix": prefix_mi355x,
            "prefix_paged": prefix_paged_mi355x, "dsa": dsa_mi355x}[opname].kernel


@pytest.mark.parametrize("opname,shape,dist,seed", CASES)
def test_bf16_parity(opname, shape, dist, seed):
    print(f"bf16 {opname} {shape} {dist} seed={seed}", flush=True)
    op = OPS[opname]
    inp = {k: v for k, v in op.make_inputs(shape, seed=seed, dist=dist, device="cuda").items() if k in KEYS[opname]}
    out = kernel_of(opname)(**inp)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    o = out.float().cpu().numpy().astype(np.float64)
    r = getattr(oracle, opname).ref64(**inp)
    assert same_pattern(o, r, "bf16"), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


DSA_CASES = [(dict(B=4, L=65536, dtype="bf16"), "randn", 11), (dict(B=3, L=9000, dtype="bf16"), "ragged", 12),
             (dict(B=2, L=8192, dtype="bf16"), "needle", 13), (dict(B=1, L=1500, dtype="bf16"), "randn", 14),
             (dict(B=2, L=6000, dtype="bf16"), "nan_inf", 15)]


@pytest.mark.parametrize("shape,dist,seed", DSA_CASES)
def test_bf16_dsa_parity(shape, dist, seed):
    """DSA decode on bf16 q, kv, iq, ik: the selected set passes the exact top-k check against float64 scores of the
    same bf16 values, and the output meets the L2 bar against the oracle over that set."""
    import vmk
    print(f"bf16 dsa {shape} {dist} seed={seed}", flush=True)
    inp = dsa.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    B = shape["B"]
    idx = torch.full((B, 2048), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    out = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp["lens"], idx=idx, cnt=cnt)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    s64, sel = oracle.dsa.ref_select64(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
    for b in range(B):
        n = shape["L"] if lens is None else int(lens[b])
        ok, det = oracle.dsa.topk_set_check(idx[b], int(cnt[b]), s64[b], n, bound[b])
        assert ok, (b, det)
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.dsa.ref64(**inp, sel=sel)
    assert same_pattern(o, r, "bf16"), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


def test_bf16_dsa_two_stage_equals_fused():
    """The indexer/select entry then the sparse-MLA entry give the bits of the fused bf16 entry."""
    import vmk
    inp = dsa.make_inputs(dict(B=3, L=9000, dtype="bf16"), seed=5, dist="ragged", device="cuda")
    o1 = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp["lens"])
    idx, cnt = vmk.dsa_indexer_select(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    o2 = vmk.dsa_sparse_mla(inp["q"], inp["kv"], idx, cnt)
    torch.cuda.synchronize()
    assert o1.dtype == o2.dtype == torch.bfloat16
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_bf16_rejects_mixed_dtypes():
    import vmk
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 8, 64, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(TypeError):
        vmk.decode(q, k, k)
    y = torch.zeros(1, 2100, 576, dtype=torch.bfloat16, device="cuda")
    iq = torch.zeros(1, 64, 128, dtype=torch.bfloat16, device="cuda")
    ik = torch.zeros(1, 2100, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(1, 64, device="cuda")
    with pytest.raises(TypeError):
        vmk.dsa_decode(y[:, :128].contiguous(), y.half(), iq, ik, w, None)
    with pytest.raises(TypeError):
        vmk.dsa_indexer_select(iq, ik.half(), w, None)


@pytest.mark.parametrize("opname,shape,dist", [("spec", dict(B=4, L=32768, k=8, dtype="bf16"), "chain"),
                                               ("prefix", dict(N=64, P=16384, S=2048, S_min=128, dtype="bf16"),
                                                "outlier"),
                                               ("decode", dict(B=5, L=3000, L_min=1, dtype="bf16"), "randn"),
                                               ("dsa", dict(B=4, L=16384, dtype="bf16"), "randn")])
def test_bf16_rows_alone_equal_batch(opname, shape, dist):
    """Batch invariance holds for bf16 as for fp16: the plans do not depend on the element type."""
    print(f"bf16 L4 {opname} {shape}", flush=True)
    op = OPS[opname]
    inp = {k: v for k, v in op.make_inputs(shape, seed=40, dist=dist, device="cuda").items() if k in KEYS[opname]}
    kern = kernel_of(opname)
    full = kern(**inp)
    torch.cuda.synchronize()
    for r in range(full.shape[0]):
        o = kern(**op.row_inputs(inp, r))
        torch.cuda.synchronize()
        assert torch.equal(full[r:r + 1].view(torch.int16), o.view(torch.int16)), r
