"""CPU checks of the verifier: screening, the case plan, the scores, and a worker run end to end on the CPU with
stand-in kernel modules (one exact, one that raises on some cases, one that dies half-way through its plan)."""
import json
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import verify
from judge import nonfinite, normalised_error, rounding_of, same_nonfinite
from vmk.ops import dsa, prefix, spec

HERE = os.path.dirname(os.path.abspath(__file__))
KDIR = os.path.join(os.path.dirname(HERE), "verified-metal-kernels_amd", "kernels")
SHIPPED = ["spec_mi355x.py", "prefix_mi355x.py", "dsa_mi355x.py", "decode_mi355x.py", "prefix_paged_mi355x.py"]


@pytest.mark.parametrize("name", SHIPPED)
def test_screening_passes_the_shipped_modules(name):
    assert verify.screen(open(os.path.join(KDIR, name)).read()) == []


@pytest.mark.parametrize("src,needle", [
    ("import torch\ndef kernel(q):\n    return torch.nn.functional.scaled_dot_product_attention(q, q, q)\n",
     "scaled_dot_product_attention"),
    ("import os\nimport vmk\ndef kernel(q):\n    return vmk.spec_verify(q)\n", "import os"),
    ("import torch\ndef kernel(q):\n    return q\n", "never calls into vmk"),
    ("import vmk\ndef kernel(q):\n    return vmk\n", "never calls into vmk"),
    ("import vmk\ndef kernel(q):\n    return open('x')\n", "builtin `open`"),
    ("import vmk\ndef kernel(q):\n    print(q)\n    return vmk.f(q)\n", "builtin `print`"),
    ("import vmk\ndef kernel(q):\n    return vmk.f(getattr(q, 'x'))\n", "builtin `getattr`"),
    ("import vmk, torch\ndef kernel(s):\n    return vmk.x(s.topk(3))\n", "selection routine"),
    ("import vmk, torch\ndef kernel(s):\n    torch.manual_seed(0)\n    return vmk.x(s)\n", "global state"),
    ("import vmk, torch\ndef kernel(s):\n    return vmk.x(torch.jit.script(s))\n", "compiles code"),
    ("import vmk\ndef kernel(q):\n    vmk.flag = 1\n    return vmk.f(q)\n", "stores into"),
    ("import vmk\ndef kern(q):\n    return vmk.f(q)\n", "def kernel"),
    ("import vmk\ndef kernel(q):\n    return vmk._lib.f(q)\n", "private attribute `._lib`"),
    ("import vmk\ndef kernel(q):\n    return __builtins__\n", "dunder name"),
    ("from . import vmk\ndef kernel(q):\n    return vmk.f(q)\n", "from . import"),
    ("from torch.utils import cpp_extension\nimport vmk\ndef kernel(q):\n    return vmk.f(q)\n", "torch.utils"),
    ("import vmk\ndef kernel(q):\n    yield vmk.f(q)\n", "Yield"),
    ("import vmk\nX = 0\ndef kernel(q):\n    global X\n    return vmk.f(q)\n", "global"),
    ("def kernel(q:\n", "does not parse"),
])
def test_screening_refuses(src, needle):
    problems = verify.screen(src)
    assert problems and any(needle in p for p in problems), problems


def test_screening_size_limit():
    src = "import vmk\ndef kernel(q):\n    return vmk.f(q)\n" + "#" * verify.SIZE_LIMIT
    assert "larger than" in verify.screen(src)[0]


def test_plan_keeps_the_reference_case_lists_and_seeds():
    """5/12/5, 5/14/5, 5/12/5 cases in L1/L2/L3 (README.md:70-71 of the reference), seeds 100+i, 7+i and 3."""
    for op, (n1, n2, n3) in ((prefix, (5, 12, 5)), (spec, (5, 14, 5)), (dsa, (5, 12, 5))):
        cases = verify.plan(op, verify.LAYERS[:3])
        counts = [sum(c.layer == name for c in cases) for name in ("L1", "L2", "L3")]
        assert counts == [n1, n2, n3]
        assert [c.seed for c in cases if c.layer == "L1"] == [100, 101, 102, 103, 104]
        assert [c.seed for c in cases if c.layer == "L2"] == [7 + i for i in range(n2)]
        assert {c.seed for c in cases if c.layer == "L3"} == {3}
        assert [(c.shape, c.dist) for c in cases if c.layer == "L2"] == list(op.FUZZ)


def test_plan_holds_every_benchmark_configuration():
    labels = {c.label for op in (prefix, spec, dsa) for c in verify.plan(op) if c.layer == "CFG"}
    assert {"C1", "C2", "C3", "C4", "C5"} <= labels
    cfg = {c.label: c for c in verify.plan(spec) if c.layer == "CFG"}
    assert cfg["C4"].shape == dict(B=2, L=65536, k=64) and cfg["C4"].dist == "tree_bd" and cfg["C4"].seed == 0
    assert all(c.seed == 0 for op in (prefix, spec, dsa) for c in verify.plan(op) if c.layer == "CFG")
    assert [layer.rules for layer in verify.LAYERS if layer.name == "CFG"] == [("fuzz", "relative")]


def test_normalised_error_and_nonfinite():
    want = np.array([0.5, -2.0, np.nan, np.inf])
    got = np.array([0.52, -2.0, np.nan, np.inf])
    emax, emean = normalised_error(got, want)
    assert emax == pytest.approx(0.01) and emean == pytest.approx(0.005)
    assert normalised_error(np.array([np.nan]), np.array([1.0])) == (0.0, 0.0)
    assert normalised_error(np.array([3.0]), np.array([0.5]))[0] == pytest.approx(2.5)      # scale floor 1
    nan, inf = nonfinite(np.array([1e5, 7e4, np.nan, 6e4]))                                  # 7e4 overflows fp16
    assert list(inf) == [True, True, False, False] and list(nan) == [False, False, True, False]
    assert not nonfinite(np.array([1e5]), "fp32")[1][0]
    big = verify_bf16_edge = (2.0 - 2.0 ** -8) * 2.0 ** 127
    assert nonfinite(np.array([big]), "bf16")[1][0] and not nonfinite(np.array([big * 0.999]), "bf16")[1][0]
    assert same_nonfinite(np.array([np.inf, 1.0]), np.array([7e4, 2.0]))
    assert not same_nonfinite(np.array([np.inf, 1.0]), np.array([7e4, 2.0]), "fp32")
    assert [rounding_of(n) for n in ("torch.float16", "torch.bfloat16", "torch.float32")] == ["fp16", "bf16", "fp32"]
    del verify_bf16_edge


def test_unfinished_cases_are_failures(tmp_path):
    """Nothing in the output directory: every planned case is reported as failed, without computing anything."""
    case = verify.Case("L1", 0, dict(B=1, L=8, k=8), "randn", 100)
    rep = verify.assess("spec", str(tmp_path), device="cpu", cases=[case], row_cases=[])
    c = rep["layers"]["L1"]["cases"][0]
    assert rep["verdict"] == "REJECTED" and not c["ok"] and "did not finish" in c["error"]


def test_row_scoring_names_the_differing_rows():
    case = verify.Case("L4", 0, {}, "randn", 200)
    full = np.arange(24, dtype=np.float16).reshape(4, 6)
    as_bytes = lambda a: a.view(np.uint8).reshape(a.shape[0], -1)
    entry = dict(ok=True, rows=4, outputs=1)
    assert verify.score_rows(case, entry, dict(batch0=as_bytes(full), alone0=as_bytes(full.copy())))["ok"]
    alone = full.copy()
    alone[2, 3] = -alone[2, 3]
    r = verify.score_rows(case, entry, dict(batch0=as_bytes(full), alone0=as_bytes(alone)))
    assert not r["ok"] and r["first_differing"] == [2] and r["differing"] == 1
    nan = full.copy()
    nan[1, 1] = np.nan
    assert verify.score_rows(case, entry, dict(batch0=as_bytes(nan), alone0=as_bytes(nan.copy())))["ok"]
    assert "did not finish" in verify.score_rows(case, None, None)["error"]


def test_op_from_filename_takes_the_longest_op_name():
    assert verify.op_from_filename("x/prefix_paged_mi355x.py") == "prefix_paged"
    assert verify.op_from_filename("prefix_mi355x.py") == "prefix"
    assert verify.op_from_filename("kernel.py") is None


# ---------------------------------------------------------------------------------------- worker runs on the CPU
EXACT_SPEC = textwrap.dedent('''
    import math
    import torch

    def kernel(q, k, v, bits):
        """Float32 masked GQA attention, rounded to q's dtype."""
        B, kd, Hq, d = q.shape
        Hkv, L = k.shape[1], k.shape[2]
        G = Hq // Hkv
        qf = q.float().reshape(B, kd, Hkv, G, d).permute(0, 2, 1, 3, 4).reshape(B, Hkv, kd * G, d)
        s = torch.matmul(qf, k.float().transpose(-1, -2)) / math.sqrt(d)
        w = (bits.long() & 0xFFFFFFFF).reshape(B, kd, -1)
        j = torch.arange(kd)
        tail = ((w[:, :, j // 32] >> (j % 32)) & 1).bool()
        m = torch.cat([torch.ones(B, kd, L - kd, dtype=torch.bool), tail], -1).repeat_interleave(G, dim=1)
        s = s.masked_fill(~m[:, None], float("-inf"))
        o = torch.matmul(torch.softmax(s, -1), v.float())
        return o.reshape(B, Hkv, kd, G, d).permute(0, 2, 1, 3, 4).reshape(B, kd, Hq, d).to(q.dtype)
''')


def _tiny_plan():
    return [verify.Case("L1", 0, dict(B=1, L=40, k=4), "randn", 100),
            verify.Case("L2", 0, dict(B=2, L=33, k=5), "large", 7),
            verify.Case("L3", 0, dict(B=1, L=64, k=8), "randn", 3),
            verify.Case("X", 0, dict(B=1, L=70, k=40), "needle_masked", 50)]


def _rows():
    return [verify.Case("L4", 0, dict(B=3, L=50, k=3), "randn", 200)]


def _run_worker(tmp_path, src):
    path = tmp_path / "spec_stand_in.py"
    path.write_text(src)
    out = tmp_path / "out"
    out.mkdir()
    w = verify.Worker("spec", str(path), str(out), device="cpu")
    w.run(_tiny_plan(), _rows())
    return verify.assess("spec", str(out), device="cpu", cases=_tiny_plan(), row_cases=_rows())


def test_worker_and_scoring_accept_an_exact_module(tmp_path):
    rep = _run_worker(tmp_path, EXACT_SPEC)
    assert rep["verdict"] == "CORRECT", verify.render(rep)
    assert [rep["layers"][n]["passed"] for n in ("L1", "L2", "L3", "X", "L4")] == [1, 1, 1, 1, 1]


def test_a_case_that_raises_fails_alone(tmp_path):
    src = EXACT_SPEC + textwrap.dedent('''
        _kernel = kernel

        def kernel(q, k, v, bits):
            if q.shape[1] == 5:
                raise RuntimeError("planted failure")
            return _kernel(q, k, v, bits)
    ''')
    rep = _run_worker(tmp_path, src)
    assert rep["verdict"] == "REJECTED"
    l2 = rep["layers"]["L2"]["cases"][0]
    assert not l2["ok"] and "planted failure" in l2["error"]
    assert all(rep["layers"][n]["passed"] == 1 for n in ("L1", "L3", "X", "L4"))


def test_a_wrong_module_is_rejected_by_the_oracle_layers(tmp_path):
    """Scores multiplied by 2 (a planted mistake): close enough for no layer except the ones against float64."""
    rep = _run_worker(tmp_path, EXACT_SPEC.replace("/ math.sqrt(d)", "* 2 / math.sqrt(d)"))
    assert rep["verdict"] == "REJECTED"
    assert rep["layers"]["L3"]["passed"] == 0 and rep["layers"]["L4"]["passed"] == 1


def test_a_worker_that_dies_keeps_the_cases_it_finished(tmp_path):
    """The worker process exits abruptly on its third case: the first two are scored, the rest fail."""
    src = EXACT_SPEC + textwrap.dedent('''
        _kernel = kernel
        _calls = [0]

        def kernel(q, k, v, bits):
            _calls[0] += 1
            if _calls[0] == 3:
                import os
                os._exit(7)
            return _kernel(q, k, v, bits)
    ''')
    path = tmp_path / "spec_dies.py"
    path.write_text(src)
    out = tmp_path / "out"
    out.mkdir()
    driver = textwrap.dedent(f'''
        import sys
        sys.path[:0] = {sys.path!r}
        import verify
        from test_verify_cpu import _tiny_plan, _rows
        w = verify.Worker("spec", {str(path)!r}, {str(out)!r}, device="cpu")
        w.run(_tiny_plan(), _rows())
    ''')
    p = subprocess.run([sys.executable, "-c", driver], cwd=HERE, capture_output=True, text=True, timeout=300)
    assert p.returncode == 7, p.stderr[-2000:]
    lines = [json.loads(x) for x in open(out / "manifest.jsonl")]
    assert [x["key"] for x in lines] == ["L1-0", "L2-0"]
    rep = verify.assess("spec", str(out), device="cpu", cases=_tiny_plan(), row_cases=_rows())
    assert rep["layers"]["L1"]["passed"] == 1 and rep["layers"]["L2"]["passed"] == 1
    for name in ("L3", "X", "L4"):
        assert "did not finish" in rep["layers"][name]["cases"][0]["error"]
    assert rep["verdict"] == "REJECTED"


def test_command_line_refuses_unscreened_modules_without_running_them(tmp_path):
    bad = tmp_path / "spec_bad.py"
    bad.write_text("import os\ndef kernel(q, k, v, bits):\n    return os.getcwd()\n")
    p = subprocess.run([sys.executable, os.path.join(HERE, "verify.py"), str(bad)], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 1 and "refused" in p.stdout and "REJECTED" in p.stdout
    p = subprocess.run([sys.executable, os.path.join(HERE, "verify.py"), str(tmp_path / "nameless.py")],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2


@pytest.mark.parametrize("opname", ["prefix", "spec", "dsa", "decode", "prefix_paged"])
def test_row_inputs_slice_one_batch_row(opname):
    """row_inputs(i) is batch row i of every per-row input (CPU tensors, a small L4-like shape of each op)."""
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
