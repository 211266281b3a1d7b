"""The single-launch DSA decode (vmk_dsa_decode_single through the C-ABI): parity with the float64 oracle and the
exact top-2048 check at C5 and at ragged, short and many-request shapes, bit-equality with the four-launch
vmk_dsa_decode, repeated calls on one workspace (the grid-barrier counters return to zero; a barrier that gave up
would show as cnt = -1) and HIP-graph replays."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr, same_nonfinite as same_pattern
from vmk.ops import dsa

pytestmark = pytest.mark.gpu


def run(inp, single):
    import vmk
    B = inp["q"].shape[0]
    idx = torch.full((B, 2048), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    out = vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp["lens"], idx=idx, cnt=cnt,
                         single=single)
    return out, idx, cnt


def check_oracle(inp, out, idx, cnt):
    B, L = inp["ik"].shape[:2]
    s64, sel = oracle.dsa.ref_select64(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    bound = oracle.dsa.score_error_bound(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy()
    lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
    for b in range(B):
        n = L if lens is None else int(lens[b])
        ok, det = oracle.dsa.topk_set_check(idx[b], int(cnt[b]), s64[b], n, bound[b])
        assert ok, (b, det)
    o = out.float().cpu().numpy().astype(np.float64)
    r = oracle.dsa.ref64(**inp, sel=sel)
    kind = "bf16" if out.dtype == torch.bfloat16 else "fp16"
    assert same_pattern(o, r, kind)
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}", flush=True)
    assert em <= 1e-2


CASES = [(dict(B=4, L=65536), "randn", 0),            # C5
         (dict(B=3, L=9000), "ragged", 5),            # ragged lens, some at most 2048
         (dict(B=2, L=1500), "randn", 6),             # every request below 2048 positions: no indexer phase
         (dict(B=65, L=4096), "randn", 8),            # histograms outside the workspace head; items > grid
         (dict(B=2, L=8192, dtype="bf16"), "randn", 9)]


@pytest.mark.parametrize("shape,dist,seed", CASES)
def test_single_launch_parity_and_bits(shape, dist, seed):
    print(f"dsa single {shape} {dist} seed={seed}", flush=True)
    inp = dsa.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    out1, idx1, cnt1 = run(inp, single=True)
    out4, idx4, cnt4 = run(inp, single=False)
    torch.cuda.synchronize()
    assert (cnt1 >= 0).all(), cnt1
    assert torch.equal(cnt1, cnt4) and torch.equal(idx1, idx4)
    assert torch.equal(out1.view(torch.int16), out4.view(torch.int16))
    if shape["B"] <= 8:
        check_oracle(inp, out1, idx1, cnt1)


def test_single_launch_repeated_calls_and_graph():
    """Calls back to back on one workspace, a larger and a smaller shape in turn, then a graph of three calls
    replayed with eager work in between: every call bit-equal to the four-launch result."""
    shapes = [(dict(B=4, L=65536), 0), (dict(B=2, L=20000), 1), (dict(B=4, L=65536), 2)]
    sets = [dsa.make_inputs(s, seed=sd, dist="randn", device="cuda") for s, sd in shapes]
    want = [run(i, single=False)[0].clone() for i in sets]
    for _ in range(2):
        for i, w in zip(sets, want):
            out, _, cnt = run(i, single=True)
            torch.cuda.synchronize()
            assert (cnt >= 0).all() and torch.equal(out.view(torch.int16), w.view(torch.int16))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in sets:
            run(i, single=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [run(i, single=True) for i in sets]
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for (out, _, cnt), w in zip(outs, want):
            assert (cnt >= 0).all() and torch.equal(out.view(torch.int16), w.view(torch.int16))
        run(sets[1], single=False)                   # eager work between replays
        torch.cuda.synchronize()
