"""The verifier (tests/verify.py) on the GPU: every libvmk kernel module is CORRECT on every layer, benchmark
configurations included, and each calibration fixture is REJECTED by the layer meant to catch it (the two cheats
as README.md:109-112 of the reference documents; the row-invariance fixture is this build's)."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
KDIR = os.path.join(os.path.dirname(HERE), "verified-metal-kernels_amd", "kernels")


def run_verify(path, tmp_path, *extra):
    out = tmp_path / "report.json"
    print(f"verify {os.path.basename(path)} {' '.join(extra)}", flush=True)
    p = subprocess.run([sys.executable, os.path.join(HERE, "verify.py"), path, "--json", str(out), *extra],
                       capture_output=True, text=True, timeout=1500)
    print(p.stdout[-4000:], p.stderr[-2000:], flush=True)
    assert out.exists(), p.stdout + p.stderr
    return p.returncode, json.load(open(out))


def counts(rep, layer):
    v = rep["layers"][layer]
    return v["passed"], v["total"]


@pytest.mark.timeout(1500)
@pytest.mark.parametrize("name,configs", [("spec_mi355x.py", {"C3", "C4"}), ("prefix_mi355x.py", {"C1", "C2", "C2b"}),
                                          ("dsa_mi355x.py", {"C5"}), ("decode_mi355x.py", {"D1", "D2", "D3"}),
                                          ("prefix_paged_mi355x.py", {"P2", "P2n"}),
                                          ("decode_paged_mi355x.py", {"D1p", "D2n"})])
def test_kernel_module_is_correct(name, configs, tmp_path):
    rc, rep = run_verify(os.path.join(KDIR, name), tmp_path)
    assert rep["verdict"] == "CORRECT" and rc == 0
    assert {c["label"] for c in rep["layers"]["CFG"]["cases"]} == configs
    if name.startswith("dsa"):
        scored = sum(rep["layers"][n]["total"] for n in ("L1", "L2", "L3", "X", "CFG"))
        assert rep["layers"]["TK"]["total"] == scored


@pytest.mark.timeout(900)
def test_spec_cheat_rejected_by_fuzzing(tmp_path):
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "spec_cheat_nomax.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    p, n = counts(rep, "L1")
    assert p == n
    assert "large" in [c["dist"] for c in rep["layers"]["L2"]["cases"] if not c["ok"]]


@pytest.mark.timeout(900)
def test_prefix_cheat_rejected(tmp_path):
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "prefix_cheat_fp16.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    p, n = counts(rep, "L1")
    assert p == n
    assert counts(rep, "L2")[0] < counts(rep, "L2")[1] or counts(rep, "L3")[0] < counts(rep, "L3")[1]


@pytest.mark.timeout(900)
def test_batch_dependent_decode_rejected_only_by_l4(tmp_path):
    """The row-invariance fixture is exact on every call but cuts the keys into B + 1 chunks: every other layer
    accepts it and the row-invariance layer rejects it."""
    rc, rep = run_verify(os.path.join(HERE, "wrong_kernels", "decode_cheat_batch_split.py"), tmp_path, "--skip-gate")
    assert rep["verdict"] == "REJECTED" and rc == 1
    for layer in ("L1", "L2", "L3", "X", "CFG"):
        p, n = counts(rep, layer)
        assert p == n, (layer, [c for c in rep["layers"][layer]["cases"] if not c["ok"]])
    assert counts(rep, "L4")[0] == 0
