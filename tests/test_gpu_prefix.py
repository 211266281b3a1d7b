"""GPU parity of the shared-prefix kernel (libvmk through the C-ABI) against the float64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import prefix

pytestmark = pytest.mark.gpu

CASES = [(s, d, 7 + i) for i, (s, d) in enumerate(prefix.FUZZ)] + [(s, d, 40 + i) for i, (s, d) in
                                                                   enumerate(prefix.EXTRA)]
CASES += [(dict(N=8, P=2048, S=256), "randn", 100), (dict(N=64, P=1000, S=300, S_min=1), "outlier", 101),
          # many rows per KV head with suffixes longer than one suffix item (separate merge launch), and with
          # empty suffixes (rows made of the prefix alone)
          (dict(N=20, P=3000, S=2500, S_min=1), "randn", 102), (dict(N=40, P=500, S=8, S_min=0), "randn", 103)]


@pytest.mark.parametrize("shape,dist,seed", CASES)
def test_prefix_parity(shape, dist, seed):
    import prefix_mi355x
    print(f"prefix case {shape} {dist} seed={seed}", flush=True)
    inp = prefix.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    out = prefix_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.prefix.ref64(**inp)
    assert out.shape == tuple(r.shape) and out.dtype == inp["q"].dtype
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


# More than 64 rows per KV head (prefix row blocks, then whole-suffix items that merge the prefix partials).
ROWS_CASES = [
    (dict(N=64, P=16384, S=2048, S_min=128), "outlier", 110),              # C2, the headline configuration
    (dict(N=32, P=16384, S=40, S_min=0), "randn", 111),                    # long prefix, short or empty suffixes
    (dict(N=100, P=3000, S=500, S_min=1, Hq=24, Hkv=8), "randn", 112),     # G = 3: requests straddle row blocks
    (dict(N=24, P=5000, S=700), "randn", 113),                             # equal suffix lengths
    (dict(N=40, P=4096, S=300, S_min=1, Hq=64, Hkv=8), "randn", 115),      # G = 8: the general merge
    (dict(N=40, P=65536, S=100, S_min=1), "randn", 116),                   # 64 prefix chunks: the general merge
]

# Other head counts, in the row-block path and the mixed launch.
HEADS_CASES = [
    (dict(N=10, P=3000, S=400, S_min=1, Hq=32, Hkv=1), "randn", 117),      # G = 32: two row blocks of 256 rows
    (dict(N=20, P=2500, S=300, Hq=32, Hkv=16), "randn", 118),              # G = 2, 40 rows (mixed launch)
    (dict(N=9, P=2048, S=300, S_min=1, Hq=8, Hkv=8), "randn", 119),        # G = 1, 9 rows
    (dict(N=3, P=4096, S=200, S_min=1, Hq=64, Hkv=4), "randn", 126),       # G = 16, 48 rows
]


# At most 32 rows per KV head and more mixed-launch items than CUs: the prefix runs as single-wave units, 2 or 4 per
# workgroup (the mixed launch's row blocks give the same bits; see the invariance test below).
UNITS_CASES = [
    (dict(N=4, P=4096, S=512), "randn", 120),                              # 2 units per workgroup
    (dict(N=4, P=8192, S=256, S_min=1), "outlier", 121),                   # ragged suffixes
    (dict(N=1, P=65536, S=100), "randn", 122),                             # 4 per workgroup, 64 chunks: general merge
    (dict(N=4, P=4096, S=300, S_min=1, Hq=64, Hkv=8), "randn", 123),       # G = 8: the general merge
    (dict(N=10, P=6000, S=200, Hq=24, Hkv=8), "randn", 124),               # G = 3, 30 rows, a partial last chunk
    (dict(N=8, P=3000, S=2500, S_min=1), "randn", 125),                    # suffixes of two chunks: combine launch
]


@pytest.mark.parametrize("shape,dist,seed", UNITS_CASES)
def test_prefix_units_parity(shape, dist, seed):
    test_prefix_parity(shape, dist, seed)


def _head_is_zero():
    from vmk import api
    ws = api.workspace(0, "cuda")
    return int(ws[: 4 << 20].count_nonzero().item()) == 0


@pytest.mark.parametrize("shape,dist,seed", ROWS_CASES)
def test_prefix_rows_parity(shape, dist, seed):
    test_prefix_parity(shape, dist, seed)
    assert _head_is_zero(), "the workspace head must be zero after every call"


@pytest.mark.parametrize("shape,dist,seed", HEADS_CASES)
def test_prefix_head_counts_parity(shape, dist, seed):
    test_prefix_parity(shape, dist, seed)
    assert _head_is_zero(), "the workspace head must be zero after every call"


def test_prefix_rows_empty_suffixes():
    """Every suffix empty: every row is the prefix alone."""
    import prefix_mi355x
    inp = prefix.make_inputs(dict(N=32, P=2000, S=64, S_min=0), seed=114, device="cuda")
    inp["slens"].zero_()
    out = prefix_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.prefix.ref64(**inp)
    em, _ = nerr(o, r)
    assert em <= 1e-2
    assert _head_is_zero()


def test_prefix_in_launch_merge_flag():
    """At most 128 rows per KV head with G <= 4 and one suffix chunk, the suffix workgroups wait (bounded) for their
    KV head's prefix partials inside the one launch.  A wait that gives up sets a sticky flag in the workspace head,
    and every later such call on that workspace writes NaN rows at once instead of waiting.  The flag is set here
    from the host (no wait is made to give up): the call writes NaN rows and the flag stays set (the arrival
    counters may be left behind too, as the suffix workgroups no longer wait for them); once the head is zeroed,
    the same call is exact again."""
    import prefix_mi355x
    from vmk import api
    # The flag word: workspace byte 2 MiB (the head's counter part) + 1.5 MiB (the prefix op's block), as in
    # vmk_prefix.hip (kPrefixSync).
    flag = (2 << 20) + (3 << 19)
    inp = prefix.make_inputs(dict(N=8, P=2048, S=256), seed=130, device="cuda")
    r = oracle.prefix.ref64(**inp)
    out = prefix_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    assert nerr(out.float().cpu().numpy().astype(np.float64), r)[0] <= 1e-2
    ws = api.workspace(0, "cuda")
    ws[flag:flag + 4] = torch.tensor([1, 0, 0, 0], dtype=torch.uint8, device="cuda")
    out = prefix_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    assert bool(torch.isnan(out.float()).all())
    assert int(ws[flag].item()) == 1, "the flag stays set"
    ws[: 4 << 20].zero_()
    out = prefix_mi355x.kernel(**inp)
    torch.cuda.synchronize()
    assert nerr(out.float().cpu().numpy().astype(np.float64), r)[0] <= 1e-2
    assert _head_is_zero()
