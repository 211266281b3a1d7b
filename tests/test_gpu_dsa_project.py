"""GPU parity of the DSA projections (libvmk vmk_dsa_project through the C-ABI) against the float64 oracle, the cache
rows they write, and their outputs feeding the DSA decode op."""
import numpy as np
import pytest
import torch

import oracle
from judge import normalised_error as nerr
from vmk.ops import dsa, dsa_project as op

pytestmark = pytest.mark.gpu

# (shape, seed); 33 tokens span two 32-token tiles of every product.
CASES = [(dict(B=1, L=64), 0), (dict(B=4, L=4096), 1), (dict(B=33, L=100), 2), (dict(B=5, L=300, dtype="bf16"), 3)]
TOL = {"fp16": 4e-3, "bf16": 3e-2}


def project(inp):
    import vmk
    return vmk.dsa_project(inp["x"], inp["pos"], inp["rope_cos"], inp["rope_sin"], inp["weights"], inp["kv"],
                           inp["ik"])


def reference(inp, dtype):
    return oracle.dsa_project.ref64(inp["x"], inp["pos"], inp["rope_cos"], inp["rope_sin"], dtype=dtype,
                                    **inp["weights"])


@pytest.mark.parametrize("shape,seed", CASES)
def test_project_parity(shape, seed):
    print(f"dsa_project case {shape} seed={seed}", flush=True)
    dtype = shape.get("dtype", "fp16")
    inp = op.make_inputs(shape, seed=seed, device="cuda")
    inp["kv"].fill_(7.0)                                   # every row but the new one must keep this
    inp["ik"].fill_(-3.0)
    q, iq, w = project(inp)
    torch.cuda.synchronize()
    r = reference(inp, dtype)
    pos = inp["pos"].cpu().numpy()
    B = shape["B"]
    kv = inp["kv"].float().cpu().numpy()
    ik = inp["ik"].float().cpu().numpy()
    got = dict(q=q, iq=iq, w=w, kv_row=kv[np.arange(B), pos], ik_row=ik[np.arange(B), pos])
    for name, g in got.items():
        g = g.float().cpu().numpy() if isinstance(g, torch.Tensor) else g
        em, ea = nerr(g.astype(np.float64), r[name])
        print(f"  {name}: err max {em:.3e} mean {ea:.3e}")
        assert em <= TOL[dtype], name
    keep = np.ones(kv.shape[:2], bool)
    keep[np.arange(B), pos] = False
    assert (kv[keep] == 7.0).all() and (ik[keep] == -3.0).all()


def test_positions_outside_the_cache_write_no_row():
    """pos = L or -1: q, iq and w are still produced (RoPE from the clamped table row), no cache row is written."""
    inp = op.make_inputs(dict(B=3, L=50), seed=9, device="cuda")
    inp["pos"] = torch.tensor([50, -1, 10], dtype=torch.int32, device="cuda")
    inp["kv"].fill_(1.5)
    inp["ik"].fill_(2.5)
    q, iq, w = project(inp)
    torch.cuda.synchronize()
    r = reference(inp, "fp16")
    for name, g in dict(q=q, iq=iq, w=w).items():
        assert nerr(g.float().cpu().numpy().astype(np.float64), r[name])[0] <= TOL["fp16"], name
    kv, ik = inp["kv"].float().cpu(), inp["ik"].float().cpu()
    assert (kv[:2] == 1.5).all() and (ik[:2] == 2.5).all()            # requests 0 and 1: nothing written
    assert not (kv[2, 10] == 1.5).all() and (kv[2, :10] == 1.5).all() and (kv[2, 11:] == 1.5).all()


def test_projected_inputs_drive_the_dsa_op():
    """Caches with the new token's rows written by the projections, then the DSA decode op on the projected q, iq, w
    with lens = pos + 1: parity with the float64 DSA oracle on the same inputs, and the selection contains pos."""
    import vmk
    B, L = 2, 3000
    inp = op.make_inputs(dict(B=B, L=L), seed=11, device="cuda")
    rng = np.random.default_rng(12)
    inp["kv"].copy_(torch.from_numpy(rng.standard_normal((B, L, 576), dtype=np.float32)).half())
    inp["ik"].copy_(torch.from_numpy(rng.standard_normal((B, L, 128), dtype=np.float32)).half())
    inp["pos"] = torch.tensor([L - 1, 2500], dtype=torch.int32, device="cuda")
    q, iq, w = project(inp)
    lens = inp["pos"] + 1
    idx = torch.empty(B, 2048, dtype=torch.int32, device="cuda")
    cnt = torch.empty(B, dtype=torch.int32, device="cuda")
    out = vmk.dsa_decode(q, inp["kv"], iq, inp["ik"], w, lens, idx=idx, cnt=cnt)
    torch.cuda.synchronize()
    s64, sel = oracle.dsa.ref_select64(iq, inp["ik"], w, lens)
    bound = oracle.dsa.score_error_bound(iq, inp["ik"], w, lens)
    for b in range(B):
        ok, det = oracle.dsa.topk_set_check(idx[b].cpu().numpy(), int(cnt[b]), s64[b], int(lens[b]), bound[b])
        assert ok, (b, det)
    r = oracle.dsa.ref64(q, inp["kv"], iq, inp["ik"], w, lens, sel=sel)
    em, _ = nerr(out.float().cpu().numpy().astype(np.float64), r)
    print(f"  projected DSA decode: err max {em:.3e}")
    assert em <= 1e-2


def test_standard_op_matches_oracle():
    """The float32 PyTorch form the benchmark times against computes the same projections."""
    inp = op.make_inputs(dict(B=3, L=128), seed=13, device="cuda")
    q, iq, w, kv_row, ik_row = op.torch_ref(inp["x"], inp["pos"], inp["rope_cos"], inp["rope_sin"], inp["weights"])
    torch.cuda.synchronize()
    r = reference(inp, "fp16")
    for name, g in dict(q=q, iq=iq, w=w, kv_row=kv_row, ik_row=ik_row).items():
        assert nerr(g.float().cpu().numpy().astype(np.float64), r[name])[0] <= TOL["fp16"], name
