"""CPU checks of the verifier's host logic: the static gate, the case lists, the error measures and the judge's
handling of a crashed child (forced on the CPU with fake outputs)."""
import json
import os

import numpy as np
import pytest

import verify
from judge import nerr, pattern
from vmk.ops import dsa, prefix, spec

HERE = os.path.dirname(os.path.abspath(__file__))
KDIR = os.path.join(os.path.dirname(HERE), "verified-metal-kernels_amd", "kernels")


@pytest.mark.parametrize("name", ["spec_mi355x.py", "prefix_mi355x.py", "dsa_mi355x.py", "decode_mi355x.py",
                                  "prefix_paged_mi355x.py"])
def test_gate_accepts_shipped_kernels(name):
    assert verify.gate(open(os.path.join(KDIR, name)).read()) == []


@pytest.mark.parametrize("src,needle", [
    ("import torch\ndef kernel(q):\n    return torch.nn.functional.scaled_dot_product_attention(q, q, q)\n", "scaled_dot"),
    ("import os\nimport vmk\ndef kernel(q):\n    return vmk.spec_verify(q)\n", "import os"),
    ("import torch\ndef kernel(q):\n    return q\n", "no call into vmk"),
    ("import vmk\ndef kernel(q):\n    return open('x')\n", "open"),
    ("import vmk, torch\ndef kernel(s):\n    return vmk.x(s.topk(3))\n", "topk"),
    ("import vmk\ndef kernel(q):\n    vmk.flag = 1\n    return vmk.f(q)\n", "assigning"),
    ("import vmk\ndef kern(q):\n    return vmk.f(q)\n", "def kernel"),
    ("import vmk\ndef kernel(q):\n    return vmk._lib\n", "attribute `._lib`"),
])
def test_gate_rejects(src, needle):
    errs = verify.gate(src)
    assert errs and any(needle in e for e in errs), errs


def test_case_lists_match_reference_counts():
    for op, (n1, n2, n3) in ((prefix, (5, 12, 5)), (spec, (5, 14, 5)), (dsa, (5, 12, 5))):
        c = verify.cases(op, extra=False)
        assert [sum(1 for x in c if x[0] == l) for l in ("L1", "L2", "L3")] == [n1, n2, n3]
        seeds = [x[4] for x in c]
        assert seeds[:5] == [100, 101, 102, 103, 104] and seeds[5] == 7 and seeds[-1] == 3


def test_nerr_and_pattern():
    r = np.array([0.5, -2.0, np.nan, np.inf])
    o = np.array([0.52, -2.0, np.nan, np.inf])
    em, ea = nerr(o, r)
    assert em == pytest.approx(0.01) and ea == pytest.approx(0.005)
    pn, pi = pattern(np.array([1e5, 7e4, np.nan]))           # 7e4 overflows fp16
    assert list(pi) == [True, True, False] and list(pn) == [False, False, True]
    assert nerr(np.array([np.nan]), np.array([1.0])) == (0.0, 0.0)


def test_judge_counts_a_crashed_child_as_failures(tmp_path):
    out = str(tmp_path / "outputs")
    meta = {"L1_0": dict(ok=False, error="RuntimeError: boom")}
    np.savez(out + ".npz")
    json.dump(meta, open(out + ".json", "w"))
    try:
        rep = verify.judge("spec", out)
    except Exception as e:  # torch.cuda may be unavailable on the CPU: only the error path is exercised
        pytest.skip(f"judge needs the GPU for the passing layers: {e}")
    assert rep["verdict"] == "REJECTED"


def test_missing_cases_are_failures_without_gpu(tmp_path, monkeypatch):
    """A child that saved nothing: every case is 'missing', which the judge reports without computing anything."""
    out = str(tmp_path / "outputs")
    np.savez(out + ".npz")
    json.dump({}, open(out + ".json", "w"))
    monkeypatch.setattr(verify, "cases", lambda op, extra=True: [("L1", 0, dict(B=1, L=8, k=8), "randn", 100)])
    rep = verify.judge("spec", out)
    assert rep["verdict"] == "REJECTED" and rep["L1_pass"] == 0 and "missing" in rep["L1"][0]["error"]


@pytest.mark.parametrize("opname", ["prefix", "spec", "dsa", "decode", "prefix_paged"])
def test_l4_row_inputs_slice_one_batch_row(opname):
    """row_inputs(i) is batch row i of every per-row input (CPU tensors, the smallest L4-like shape of each op)."""
    from vmk.ops import KEYS, load_op
    op = load_op(opname)
    shape, dist = {"prefix": (dict(N=3, P=40, S=9, S_min=1), "randn"), "spec": (dict(B=3, L=40, k=5), "randn"),
                   "dsa": (dict(B=3, L=300), "ragged"), "decode": (dict(B=3, L=50, L_min=1), "randn"),
                   "prefix_paged": (dict(N=3, P=64, S=40, S_min=1, ps=32), "randn")}[opname]
    inp = {k: v for k, v in op.make_inputs(shape, seed=1, dist=dist).items() if k in KEYS[opname]}
    assert op.L4_CASES
    for i in range(3):
        r = op.row_inputs(inp, i)
        assert set(r) == set(inp)
        for k, v in inp.items():
            if v is None:
                assert r[k] is None
            elif (opname, k) in (("prefix", "kp"), ("prefix", "vp"), ("prefix_paged", "k_pages"),
                                 ("prefix_paged", "v_pages"), ("prefix_paged", "prefix_pages")):
                assert r[k] is v                              # the shared prefix is not sliced
            else:
                assert r[k].shape[0] == 1 and (r[k][0] == v[i]).all()


def test_l4_judgement_flags_the_differing_rows():
    full = np.arange(24, dtype=np.float16).reshape(4, 6)
    rows = full.copy()
    meta = {"L4_0": dict(ok=True, n_out=1, n_rows=4)}
    assert verify.l4_case(meta, {"L4_0__full0": full, "L4_0__rows0": rows}, 0, {}, "randn")["ok"]
    rows[2, 3] = np.float16(-0.0) if full[2, 3] == 0 else -full[2, 3]
    c = verify.l4_case(meta, {"L4_0__full0": full, "L4_0__rows0": rows}, 0, {}, "randn")
    assert not c["ok"] and c["rows_differing"] == [2]
    nan = full.copy()
    nan[1, 1] = np.nan
    same = verify.l4_case(meta, {"L4_0__full0": nan, "L4_0__rows0": nan.copy()}, 0, {}, "randn")
    assert same["ok"]                                          # bit comparison: equal NaN bits are equal
    missing = verify.l4_case({}, {}, 0, {}, "randn")
    assert not missing["ok"] and "missing" in missing["error"]


def test_infer_op_takes_the_longest_op_name():
    assert verify.infer_op("x/prefix_paged_mi355x.py") == "prefix_paged"
    assert verify.infer_op("prefix_mi355x.py") == "prefix"
    assert verify.infer_op("kernel.py") is None
