"""GPU parity of single-token decode (libvmk vmk_decode through the C-ABI) against the float64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import decode

pytestmark = pytest.mark.gpu

CASES = [(dict(B=1, L=1), "randn", 1), (dict(B=1, L=31), "randn", 2), (dict(B=3, L=77), "randn", 3),
         (dict(B=2, L=4097), "randn", 4), (dict(B=1, L=65536), "randn", 5), (dict(B=8, L=8192), "randn", 6),
         (dict(B=5, L=300), "large", 7), (dict(B=2, L=3000), "needle", 8), (dict(B=2, L=3000), "nan_inf", 9),
         (dict(B=2, L=3000), "tiny", 10), (dict(B=4, L=1000, Hq=8, Hkv=8), "randn", 11),
         (dict(B=2, L=2048, Hq=64, Hkv=2), "randn", 12), (dict(B=6, L=5000, L_min=1), "randn", 13),
         (dict(B=3, L=3000, L_min=1, Hq=24, Hkv=8), "randn", 21), (dict(B=2, L=4000, Hq=20, Hkv=4), "needle", 22),
         (dict(B=8, L=2048, L_min=1), "needle", 14), (dict(B=3, L=40000, L_min=30000), "randn", 15),
         (dict(B=4, L=16384), "randn", 16)]


def check(out, inp):
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.decode.ref64(**inp)
    assert out.shape == tuple(r.shape) and out.dtype == inp["q"].dtype
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2


@pytest.mark.parametrize("shape,dist,seed", CASES)
def test_decode_parity(shape, dist, seed):
    import decode_mi355x
    print(f"decode case {shape} {dist} seed={seed}", flush=True)
    inp = decode.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    check(decode_mi355x.kernel(**inp), inp)


def test_decode_lens_are_clamped():
    """lens <= 0 reads one position, lens > L reads all L (the oracle's clamp to [1, L])."""
    import vmk
    print("decode clamp case", flush=True)
    inp = decode.make_inputs(dict(B=4, L=500), seed=21, device="cuda")
    inp["lens"] = torch.tensor([0, -7, 501, 1 << 30], dtype=torch.int32, device="cuda")
    check(vmk.decode(inp["q"], inp["k"], inp["v"], inp["lens"]), inp)


def test_decode_positions_past_lens_are_not_read_into_the_result():
    """Garbage (NaN) past lens[b] leaves the output unchanged."""
    import vmk
    print("decode garbage-tail case", flush=True)
    inp = decode.make_inputs(dict(B=3, L=2000, L_min=1), seed=22, device="cuda")
    a = vmk.decode(inp["q"], inp["k"], inp["v"], inp["lens"]).clone()
    k, v = inp["k"].clone(), inp["v"].clone()
    for b, n in enumerate(inp["lens"].tolist()):
        k[b, :, n:] = float("nan")
        v[b, :, n:] = float("nan")
    c = vmk.decode(inp["q"], k, v, inp["lens"])
    torch.cuda.synchronize()
    assert torch.equal(a, c)


def test_decode_equals_spec_with_one_draft():
    """Decode over the full cache is spec verification with kd = 1 and the draft seeing itself, bit for bit."""
    import vmk
    print("decode vs spec kd=1", flush=True)
    inp = decode.make_inputs(dict(B=3, L=3001), seed=23, device="cuda")
    a = vmk.decode(inp["q"], inp["k"], inp["v"])
    bits = torch.ones(3, 1, 1, dtype=torch.int32, device="cuda")
    s = vmk.spec_verify(inp["q"][:, None].contiguous(), inp["k"], inp["v"], bits)[:, 0]
    torch.cuda.synchronize()
    assert torch.equal(a, s)
