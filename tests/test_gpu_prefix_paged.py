"""GPU parity of the paged shared-prefix kernel (libvmk vmk_prefix_decode_paged through the C-ABI).

With every page present the paged kernel must give the contiguous kernel's bits on the same cache (the plans are the
same and a tile is the same 32 rows either way); with absent pages and NaN spare pages it is checked against the
float64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import prefix, prefix_paged

pytestmark = pytest.mark.gpu

SAME = [(dict(N=64, P=16384, S=2048, S_min=128, ps=64), "outlier", 1), (dict(N=8, P=2048, S=256, ps=32), "randn", 2),
        (dict(N=5, P=1024, S=77, ps=64), "randn", 3), (dict(N=4, P=384, S=300, ps=96), "randn", 4),
        (dict(N=3, P=0, S=300, ps=32), "randn", 5), (dict(N=6, P=4096, S=1000, ps=512), "randn", 6),
        (dict(N=20, P=40960, S=3000, S_min=1, ps=256), "randn", 7), (dict(N=40, P=2048, S=64, S_min=0, ps=32),
                                                                     "randn", 8),
        # single-wave prefix units (2 and 4 per workgroup)
        (dict(N=4, P=8192, S=256, S_min=1, ps=64), "randn", 9), (dict(N=1, P=65536, S=64, ps=128), "randn", 10)]
ORACLE = [(dict(N=6, P=3072, S=500, S_min=0, ps=64, absent=3), "randn", 11),
          (dict(N=33, P=640, S=40, ps=32, absent=2), "randn", 12),
          (dict(N=4, P=2048, S=256, ps=64), "nan_inf", 13), (dict(N=4, P=2048, S=256, ps=256), "large", 14),
          (dict(N=70, P=8192, S=700, S_min=1, ps=32, absent=4), "randn", 15),
          (dict(N=1, P=32, S=1, ps=32), "randn", 16)]


@pytest.mark.parametrize("shape,dist,seed", SAME)
def test_paged_equals_contiguous_kernel(shape, dist, seed):
    import vmk
    print(f"paged vs contiguous {shape} {dist} seed={seed}", flush=True)
    inp = prefix_paged.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    c = prefix.make_inputs({k: v for k, v in shape.items() if k != "ps"}, seed=seed, dist=dist, device="cuda")
    ps = shape["ps"]
    S = inp["suffix_pages"].shape[1] * ps
    pad = lambda t: torch.nn.functional.pad(t, (0, 0, 0, S - t.shape[2])).contiguous()
    slens = inp["slens"]
    a = vmk.prefix_decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["prefix_pages"], inp["suffix_pages"],
                                slens)
    b = vmk.prefix_decode(c["q"], c["kp"], c["vp"], pad(c["ks"]), pad(c["vs"]),
                          slens if slens is not None else None)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert not torch.isnan(a).any()                      # no spare (NaN) page was read


@pytest.mark.parametrize("shape,dist,seed", ORACLE)
def test_paged_parity_vs_oracle(shape, dist, seed):
    import prefix_paged_mi355x
    print(f"paged vs oracle {shape} {dist} seed={seed}", flush=True)
    inp = prefix_paged.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    out = prefix_paged_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.prefix_paged.ref64(**inp)
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind), (np.isnan(o).sum(), np.isnan(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


def test_paged_all_pages_absent_rows_are_nan_like_the_oracle():
    """A request whose every page is absent has no keys: 0/0 like the oracle's softmax over an empty set."""
    import vmk
    print("paged all-absent case", flush=True)
    inp = prefix_paged.make_inputs(dict(N=3, P=64, S=64, ps=32), seed=17, device="cuda")
    inp["prefix_pages"][:] = -1
    inp["suffix_pages"][1] = -1
    out = vmk.prefix_decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["prefix_pages"], inp["suffix_pages"],
                                  inp["slens"])
    torch.cuda.synchronize()
    r = oracle.prefix_paged.ref64(**inp)
    o = out.float().cpu().numpy().astype(np.float64)
    assert same_pattern(o, r) and np.isnan(o[1]).all() and not np.isnan(o[[0, 2]]).any()


# NHD pools: the HND pool transposed to (num_pages, ps, Hkv, D).  The plans and the arithmetic do not depend on the
# layout, so the output must be the HND call's bits; absent pages, NaN spare pages and partial last tiles included.
NHD = [SAME[0], SAME[1], SAME[3], SAME[4], SAME[5], SAME[8], SAME[9], ORACLE[0], ORACLE[2], ORACLE[4],
       (dict(N=6, P=1024, S=300, ps=64, dtype="bf16", absent=1), "randn", 18),
       # other head counts: rows 512 and 768 bytes apart, and Hkv = 1 (the two layouts coincide)
       (dict(N=2, P=1024, S=200, ps=64, Hq=32, Hkv=2), "randn", 20),
       (dict(N=5, P=384, S=130, S_min=1, ps=96, Hq=12, Hkv=3, absent=1), "randn", 21),
       (dict(N=3, P=512, S=100, ps=32, Hq=16, Hkv=1), "randn", 22)]


@pytest.mark.parametrize("shape,dist,seed", NHD)
def test_nhd_equals_hnd(shape, dist, seed):
    import vmk
    print(f"paged NHD vs HND {shape} {dist} seed={seed}", flush=True)
    inp = prefix_paged.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    args = (inp["prefix_pages"], inp["suffix_pages"], inp["slens"])
    a = vmk.prefix_decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], *args)
    kn, vn = prefix_paged.to_nhd(inp["k_pages"]), prefix_paged.to_nhd(inp["v_pages"])
    b = vmk.prefix_decode_paged(inp["q"], kn, vn, *args, layout="NHD")
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_nhd_parity_vs_oracle():
    """The NHD entry on its own against the float64 oracle (absent pages, ragged suffixes, NaN spare pages)."""
    import prefix_paged_mi355x
    shape = dict(N=9, P=2560, S=700, S_min=0, ps=128, absent=2)
    print(f"paged NHD vs oracle {shape}", flush=True)
    inp = prefix_paged.make_inputs(shape, seed=19, device="cuda")
    nhd = dict(inp, k_pages=prefix_paged.to_nhd(inp["k_pages"]), v_pages=prefix_paged.to_nhd(inp["v_pages"]))
    out = prefix_paged_mi355x.kernel(**nhd, layout="NHD")
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.prefix_paged.ref64(**inp)
    assert same_pattern(o, r)
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2
