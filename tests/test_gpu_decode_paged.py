"""GPU parity of paged single-token decode (libvmk vmk_decode_paged / _nhd through the C-ABI).

With every page of the rows in use present, the paged kernel must give vmk_decode's bits on the gathered cache (the
plans, splits and tile order are the same, only the rows' addresses differ); with absent pages and NaN spare pages it
is checked against the float64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import decode, decode_paged

pytestmark = pytest.mark.gpu

SAME = [(dict(B=1, L=65536, ps=64), 1), (dict(B=4, L=16384, ps=64, layout="NHD"), 2),
        (dict(B=3, L=5000, L_min=1, ps=32), 3), (dict(B=8, L=8192, ps=256), 4),
        (dict(B=2, L=3000, L_min=1, ps=96, layout="NHD"), 5),
        (dict(B=5, L=4097, ps=64, dtype="bf16"), 6), (dict(B=2, L=2048, Hq=32, Hkv=2, ps=128, layout="NHD"), 7),
        (dict(B=6, L=77, ps=32), 8)]
ORACLE = [(dict(B=6, L=5000, L_min=1, ps=64, absent=3), "randn", 11),
          (dict(B=3, L=3000, ps=96, absent=2, layout="NHD"), "randn", 12),
          (dict(B=2, L=3000, ps=64), "nan_inf", 13), (dict(B=4, L=4096, ps=128), "large", 14),
          (dict(B=1, L=32, ps=32), "randn", 15)]


@pytest.mark.parametrize("shape,seed", SAME)
def test_paged_equals_contiguous_kernel(shape, seed):
    import vmk
    print(f"paged decode vs contiguous {shape} seed={seed}", flush=True)
    inp = decode_paged.make_inputs(shape, seed=seed, device="cuda")
    c = decode.make_inputs({k: v for k, v in shape.items() if k not in ("ps", "layout")}, seed=seed, device="cuda")
    ps = shape["ps"]
    Lp = inp["page_table"].shape[1] * ps
    pad = lambda t: torch.nn.functional.pad(t, (0, 0, 0, Lp - t.shape[2])).contiguous()
    a = vmk.decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["page_table"], inp["lens"],
                         layout=inp.get("layout", "HND"))
    b = vmk.decode(c["q"], pad(c["k"]), pad(c["v"]), inp["lens"])
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert not torch.isnan(a).any()                     # no spare (NaN) page was read


@pytest.mark.parametrize("shape,dist,seed", ORACLE)
def test_paged_parity_vs_oracle(shape, dist, seed):
    import decode_paged_mi355x
    print(f"paged decode vs oracle {shape} {dist} seed={seed}", flush=True)
    inp = decode_paged.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    out = decode_paged_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.decode_paged.ref64(**inp)
    assert same_pattern(o, r), (np.isnan(o).sum(), np.isnan(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


def test_all_pages_absent_rows_are_nan_like_the_oracle():
    import vmk
    inp = decode_paged.make_inputs(dict(B=3, L=200, ps=64), seed=17, device="cuda")
    inp["page_table"][1] = -1
    out = vmk.decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["page_table"], inp["lens"])
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.decode_paged.ref64(**inp)
    assert same_pattern(o, r) and np.isnan(o[1]).all() and not np.isnan(o[[0, 2]]).any()
