"""GPU parity of the shared-prefix kernel (libvmk through the C-ABI) against the float64 oracle."""
import numpy as np
import pytest
import torch

import oracle
from judge import nerr, same_pattern
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
    assert out.shape == tuple(r.shape) and out.dtype == torch.float16
    assert same_pattern(o, r), (np.isnan(o).sum(), np.isnan(r).sum(), np.isinf(o).sum(), np.isinf(r).sum())
    em, ea = nerr(o, r)
    print(f"  err max {em:.3e} mean {ea:.3e}")
    assert em <= 1e-2
