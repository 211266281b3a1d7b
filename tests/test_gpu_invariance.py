"""Row invariance on the GPU (the judge's fourth layer, ONE-PAGER.md:13-14): a batch row computed alone must have the
same output bits as in the batch.  The split plans of libvmk depend on per-row sizes only (P, S, G for prefix; L and
kd * G for spec and decode; L for DSA), never on the batch size."""
import numpy as np
import pytest
import torch

from vmk.ops import KEYS, decode, dsa, prefix, prefix_paged, spec

pytestmark = pytest.mark.gpu


def run(kernel, op, shape, dist, seed):
    inp = op.make_inputs(shape, seed=seed, dist=dist, device="cuda")
    inp = {k: inp.get(k) for k in KEYS[op.NAME]}
    full = kernel(**inp)
    torch.cuda.synchronize()
    full = full.cpu().numpy()
    bad = []
    for r in range(full.shape[0]):
        o = kernel(**op.row_inputs(inp, r))
        torch.cuda.synchronize()
        if not np.array_equal(full[r:r + 1].view(np.uint16), o.cpu().numpy().view(np.uint16)):
            bad.append(r)
    return bad


@pytest.mark.parametrize("shape,dist", [(dict(N=64, P=16384, S=2048, S_min=128), "outlier"),
                                        (dict(N=8, P=2048, S=256), "randn"),
                                        (dict(N=12, P=3000, S=2500, S_min=1), "randn"),
                                        # the batch runs single-wave prefix units, a request alone the row blocks
                                        (dict(N=8, P=3000, S=2500, S_min=1), "randn"),
                                        (dict(N=4, P=8192, S=256), "randn"),
                                        (dict(N=3, P=0, S=300), "randn"), (dict(N=5, P=700, S=0), "randn"),
                                        # 64-key chunks: the batch runs eight-wave row blocks, a request alone units
                                        (dict(N=64, P=2048, S=256), "randn")])
def test_prefix_rows_alone_equal_batch(shape, dist):
    import prefix_mi355x
    print(f"prefix L4 {shape} {dist}", flush=True)
    assert run(prefix_mi355x.kernel, prefix, shape, dist, 31) == []


@pytest.mark.parametrize("shape,dist", [(dict(B=4, L=32768, k=8), "chain"), (dict(B=2, L=8192, k=64), "tree_bd"),
                                        (dict(B=3, L=3000, k=20), "randn")])
def test_spec_rows_alone_equal_batch(shape, dist):
    import spec_mi355x
    print(f"spec L4 {shape} {dist}", flush=True)
    assert run(spec_mi355x.kernel, spec, shape, dist, 32) == []


@pytest.mark.parametrize("shape,dist", [(dict(B=8, L=8192), "randn"), (dict(B=5, L=3000, L_min=1), "needle")])
def test_decode_rows_alone_equal_batch(shape, dist):
    import decode_mi355x
    print(f"decode L4 {shape} {dist}", flush=True)
    assert run(decode_mi355x.kernel, decode, shape, dist, 33) == []


@pytest.mark.parametrize("shape,dist", [(dict(B=3, L=9000), "randn"), (dict(B=4, L=4100), "ragged")])
def test_dsa_rows_alone_equal_batch(shape, dist):
    import dsa_mi355x
    print(f"dsa L4 {shape} {dist}", flush=True)
    assert run(dsa_mi355x.kernel, dsa, shape, dist, 34) == []


@pytest.mark.parametrize("shape,dist", [(dict(N=64, P=16384, S=2048, S_min=128, ps=64), "outlier"),
                                        (dict(N=12, P=3072, S=2500, S_min=1, ps=128, absent=2), "randn")])
def test_prefix_paged_rows_alone_equal_batch(shape, dist):
    import prefix_paged_mi355x
    print(f"prefix_paged L4 {shape} {dist}", flush=True)
    assert run(prefix_paged_mi355x.kernel, prefix_paged, shape, dist, 35) == []
