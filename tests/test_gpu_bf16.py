"""bf16 inputs on the GPU (the _bf16 entry points of libvmk) against the float64 oracle, which reads the same bf16
values.  The reference kernels read fp16 only (README.md:140).  Tolerance: the verifier's L2 bar (normalised max
error <= 1e-2 and the oracle's NaN/Inf pattern after rounding to bf16)."""
import numpy as np
import pytest
import torch

import oracle
from judge import nerr, same_pattern
from vmk.ops import KEYS, decode, prefix, prefix_paged, spec

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
         ("prefix_paged", dict(N=12, P=3072, S=700, S_min=1, ps=64, absent=2, dtype="bf16"), "randn", 10)]
OPS = {"spec": spec, "decode": decode, "prefix": prefix, "prefix_paged": prefix_paged}


def kernel_of(opname):
    import decode_mi355x
    import prefix_mi355x
    import prefix_paged_mi355x
    import spec_mi355x
    return {"spec": spec_mi355x, "decode": decode_mi355x, "prefix": prefix_mi355x,
            "prefix_paged": prefix_paged_mi355x}[opname].kernel


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


def test_bf16_rejects_mixed_dtypes():
    import vmk
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 8, 64, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(TypeError):
        vmk.decode(q, k, k)


@pytest.mark.parametrize("opname,shape,dist", [("spec", dict(B=4, L=32768, k=8, dtype="bf16"), "chain"),
                                               ("prefix", dict(N=64, P=16384, S=2048, S_min=128, dtype="bf16"),
                                                "outlier"),
                                               ("decode", dict(B=5, L=3000, L_min=1, dtype="bf16"), "randn")])
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
