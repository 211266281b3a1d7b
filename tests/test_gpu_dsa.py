"""GPU parity of the DSA kernels (libvmk through the C-ABI) against the float64 oracle, plus the exact top-k check."""
import numpy as np
import pytest
import torch

import oracle
from judge import nerr, same_pattern
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
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
    for b in range(B):
        n = shape["L"] if lens is None else int(lens[b])
        ok, det = oracle.dsa.topk_set_check(idx[b], int(cnt[b]), s64[b], n)
        assert ok, (b, det)
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.dsa.ref64(**inp, sel=sel)
    assert out.shape == tuple(r.shape) and out.dtype == inp["q"].dtype
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


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
