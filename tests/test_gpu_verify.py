"""The verifier (tests/verify.py) on the GPU: every libvmk kernel module is CORRECT, and the calibration cheats are
REJECTED by the layer that is meant to catch them (README.md:109-112 of the reference; the L4 fixture is this
build's)."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
KDIR = os.path.join(os.path.dirname(HERE), "verified-metal-kernels_amd", "kernels")


def run_verify(path, tmp_path, *extra):
    out = tmp_path / "rep.json"
    print(f"verify {os.path.basename(path)} {' '.join(extra)}", flush=True)
    p = subprocess.run([sys.executable, os.path.join(HERE, "verify.py"), path, "--json", str(out), *extra],
                       capture_output=True, text=True, timeout=900)
    print(p.stdout[-3000:], p.stderr[-2000:], flush=True)
    assert out.exists(), p.stdout + p.stderr
    return p.returncode, json.load(open(out))


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["spec_mi355x.py", "prefix_mi355x.py", "dsa_mi355x.py", "decode_mi355x.py",
                                  "prefix_paged_mi355x.py"])
def test_kernel_module_is_correct(name, tmp_path):
    rc, rep = run_verify(os.path.join(KDIR, name), tmp_path)
    assert rep["verdict"] == "CORRECT" and rc == 0
    if name.startswith("dsa"):
        assert rep["TK_n"] == rep["L1_n"] + rep["L2_n"] + rep["L3_n"] + rep["X_n"]


@pytest.mark.timeout(900)
def test_spec_cheat_rejected_by_fuzzing(tmp_path):
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "spec_cheat_nomax.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    assert rep["L1_pass"] == rep["L1_n"]
    failed_l2 = [c["dist"] for c in rep["L2"] if not c["ok"]]
    assert "large" in failed_l2


@pytest.mark.timeout(900)
def test_prefix_cheat_rejected(tmp_path):
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "prefix_cheat_fp16.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    assert rep["L1_pass"] == rep["L1_n"]
    assert rep["L2_pass"] < rep["L2_n"] or rep["L3_pass"] < rep["L3_n"]


@pytest.mark.timeout(900)
def test_batch_dependent_decode_rejected_only_by_l4(tmp_path):
    """The L4 calibration fixture is exact on every call but cuts the keys into B + 1 chunks: every other layer
    accepts it and the row-invariance layer rejects it."""
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "decode_cheat_batch_split.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    for layer in ("L1", "L2", "L3", "X"):
        assert rep[f"{layer}_pass"] == rep[f"{layer}_n"], (layer, [c for c in rep[layer] if not c["ok"]])
    assert rep["L4_pass"] == 0
