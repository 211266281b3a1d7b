"""The committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py) against a fresh run of the
generators and the float64 oracle: every input's bytes (SHA-256), the oracle output's first 64 values and its 64
random projections, and the first values of the BASELINE configurations' inputs."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

GOLDEN = os.path.join(HERE, "golden")
META = json.load(open(os.path.join(GOLDEN, "cases.json")))


@pytest.mark.parametrize("opname", sorted(META))
def test_golden_cases(opname):
    fx = np.load(os.path.join(GOLDEN, f"{opname}.npz"))
    for i, c in enumerate(META[opname]):
        ins, out = make_golden.case_arrays(opname, c["shape"], c["dist"], c["seed"])
        assert {k: make_golden.digest(v) for k, v in ins.items()} == c["inputs"], (opname, i, c["shape"], c["dist"])
        assert int(np.isnan(out).sum()) == c["nan"] and int(np.isinf(out).sum()) == c["inf"], (opname, i)
        assert np.allclose(out.reshape(-1)[:64], fx[f"case{i}__head"], rtol=1e-12, atol=1e-14, equal_nan=True)
        p, q = make_golden.projections(out), fx[f"case{i}__proj"]
        assert np.allclose(p, q, rtol=1e-9, atol=1e-9 * max(1.0, float(np.abs(q).max()))), (opname, i)


def test_golden_config_heads():
    fx = np.load(os.path.join(GOLDEN, "configs.npz"))
    now = make_golden.config_heads()
    assert sorted(now) == sorted(fx.files)
    for k in fx.files:
        assert np.array_equal(now[k], fx[k]), k


def test_golden_checks_catch_a_changed_draw():
    """A generator that draws one value differently changes the digests."""
    from vmk.ops import spec
    c = META["spec"][0]
    a = spec.make_inputs(c["shape"], seed=c["seed"], dist=c["dist"])
    b = spec.make_inputs(c["shape"], seed=c["seed"] + 1, dist=c["dist"])
    assert make_golden.digest(make_golden.raw(a["q"])) == c["inputs"]["q"]
    assert make_golden.digest(make_golden.raw(b["q"])) != c["inputs"]["q"]
