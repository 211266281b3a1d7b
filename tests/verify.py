"""Judge one kernel module of an op: is it CORRECT on every case of the op's case plan, or REJECTED?

    python tests/verify.py verified-metal-kernels_amd/kernels/spec_mi355x.py
    python tests/verify.py tests/wrong_kernels/spec_cheat_nomax.py --skip-gate
    python tests/verify.py some_module.py --op dsa --json report.json

A kernel module defines `kernel(**inputs)`, called with the op's keyword inputs (vmk.ops.KEYS; absent optional
inputs arrive as None).  The op is taken from the file name (`<op>_anything.py`) unless --op names it.

How a module is judged
----------------------
1. Screening.  Before anything runs, the module's source is parsed and screened (`screen`): imports, builtins and
   attributes must stay inside what a kernel module needs (torch tensors in, libvmk kernels, tensors out), and the
   module must call into vmk at least once.  --skip-gate turns the screening off; the calibration fixtures under
   tests/wrong_kernels/ are plain torch code and need it.
2. Running.  A worker process (this script with --worker) imports the module and runs it over the case plan.  Each
   finished case is written to disk at once: one .npz of outputs plus one line of a manifest.  A worker that dies
   or runs out of time therefore leaves every case it finished behind.
3. Scoring.  This process never imports the module.  It rebuilds each case's inputs from its seed, computes the
   float64 oracle and the torch standard op where the layer needs them, and scores what the worker left.  A case
   the worker did not finish is a failure.

The layers.  L1, L2 and L3 are the reference harness's (their case lists, seeds and thresholds follow
verify.py:48-53 and 160-241 of the reference); the others are this build's.
  L1   five seeds at the nominal shape; every output allclose (atol = rtol = 1e-2, NaN matching NaN) to the
       torch standard op L1_REF.
  L2   the op's FUZZ cases, seed 7 + i: NaN/Inf positions as in the float64 oracle rounded to the output type
       (for dist "nan_inf", the standard op L3_REF's positions are accepted too) and normalised max error <= 1e-2.
  L3   the op's L3_CASES, seed 3: max and mean normalised error each <= 2 * max(standard op's, 2^-11).
  X    the op's EXTRA cases (this build's extensions), seed 50 + i, scored like L2.
  CFG  the op's benchmark configurations (CONFIGS, seed 0 as in bench.py), scored like L2 and like L3.
  TK   (dsa, when the module also defines `select(iq, ik, w, lens)`) on every case above: the count is
       min(n, 2048), the positions are distinct and below n, and the set equals the float64 top-2048 except inside
       a band of twice the fp32 score error bound around the 2048th score (oracle.dsa.score_error_bound and
       topk_set_check).
  L4   the op's L4_CASES, seed 200 + i: each batch row run alone gives the same output bytes as in the batch.
The verdict is CORRECT when every case of every layer passes.  Exit status: 0 CORRECT, 1 REJECTED, 2 bad usage.
"""
import argparse
import ast
import builtins
import importlib
import importlib.util
import json
import os
import subprocess
import sys
import tempfile
import time
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for _p in (ROOT, os.path.join(ROOT, "verified-metal-kernels_amd"), HERE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

from judge import normalised_error, nonfinite, rounding_of  # noqa: E402
from vmk.ops import KEYS, load_op  # noqa: E402

ORACLES = {name: f"oracle.{name}" for name in KEYS}
FLOOR = 2.0 ** -11                                  # L3: the error a correct fp16 kernel may always have


# ============================================================================================ the case plan
@dataclass
class Case:
    layer: str
    n: int
    shape: dict
    dist: str
    seed: int
    label: str = ""

    @property
    def key(self):
        return f"{self.layer}-{self.n}"

    def describe(self):
        return dict(case=self.key, label=self.label, shape=self.shape, dist=self.dist, seed=self.seed)


@dataclass
class Layer:
    name: str
    title: str
    cases: object                     # op -> [(shape, dist, seed, label)]
    rules: tuple = ()                 # scoring rules applied to each case, all of which must pass


LAYERS = (
    Layer("L1", "standard op at the nominal shape",
          lambda op: [(op.L1_SHAPE, "randn", 100 + i, "") for i in range(5)], ("standard",)),
    Layer("L2", "fuzzed shapes and values vs float64",
          lambda op: [(s, d, 7 + i, "") for i, (s, d) in enumerate(op.FUZZ)], ("fuzz",)),
    Layer("L3", "error within 2x the standard op's",
          lambda op: [(s, d, 3, "") for s, d in op.L3_CASES], ("relative",)),
    Layer("X", "this build's extension cases",
          lambda op: [(s, d, 50 + i, "") for i, (s, d) in enumerate(getattr(op, "EXTRA", ()))], ("fuzz",)),
    Layer("CFG", "benchmark configurations (L2 and L3 rules)",
          lambda op: [(s, d, 0, name) for name, (s, d) in getattr(op, "CONFIGS", {}).items()],
          ("fuzz", "relative")),
)
ROW_LAYER = Layer("L4", "row alone = row in the batch",
                  lambda op: [(s, d, 200 + i, "") for i, (s, d) in enumerate(getattr(op, "L4_CASES", ()))])
TOPK_LAYER = "TK"
ALL_LAYERS = tuple(l.name for l in LAYERS) + (TOPK_LAYER, ROW_LAYER.name)


def plan(op, layers=LAYERS):
    """Every output case of the op, in the order the worker runs them."""
    out = []
    for layer in layers:
        out += [Case(layer.name, i, s, d, seed, label) for i, (s, d, seed, label) in enumerate(layer.cases(op))]
    return out


def row_plan(op):
    return [Case(ROW_LAYER.name, i, s, d, seed) for i, (s, d, seed, _) in enumerate(ROW_LAYER.cases(op))]


def kernel_inputs(opname, inputs):
    """The keyword inputs the op's kernel receives; optional ones the generator left out are None."""
    return {k: inputs.get(k) for k in KEYS[opname]}


# ============================================================================================ screening
SIZE_LIMIT = 200_000
IMPORT_ROOTS = {"torch", "math", "functools", "vmk"}
TORCH_SUBMODULES = {"torch.nn.functional"}
# Builtins a kernel module may name; any other builtin (open, exec, getattr, print, type, ...) is refused.
BUILTINS_ALLOWED = frozenset({
    "abs", "all", "any", "bool", "dict", "divmod", "enumerate", "float", "int", "isinstance", "len", "list", "max",
    "min", "pow", "range", "reversed", "round", "slice", "str", "sum", "tuple", "zip", "Exception", "RuntimeError",
    "TypeError", "ValueError", "IndexError", "KeyError", "NotImplementedError", "AssertionError"})
BUILTIN_NAMES = frozenset(dir(builtins))
# Attribute names refused anywhere, by the reason for refusing them.
ATTRIBUTES_REFUSED = {
    "reads or writes files, or starts processes": {
        "save", "load", "savez", "tofile", "fromfile", "from_file", "system", "popen", "spawn", "fork"},
    "changes global state or draws random numbers": {
        "manual_seed", "seed", "random", "rand", "randn", "randint", "set_default_device", "set_default_dtype",
        "set_rng_state", "distributed"},
    "is a standard attention, softmax or selection routine": {
        "scaled_dot_product_attention", "multi_head_attention_forward", "flash_attention", "softmax",
        "log_softmax", "topk", "sort", "argsort", "msort", "kthvalue"},
    "generates or compiles code at run time": {"cpp_extension", "load_inline", "cuda_kernel", "jit", "compile"},
}
_REFUSED = {a: why for why, names in ATTRIBUTES_REFUSED.items() for a in names}


class _Screen(ast.NodeVisitor):
    def __init__(self):
        self.problems = []
        self.calls_vmk = False

    def refuse(self, node, what):
        self.problems.append(f"line {getattr(node, 'lineno', '?')}: {what}")

    @staticmethod
    def _import_ok(name):
        root = name.split(".")[0]
        if root not in IMPORT_ROOTS:
            return False
        return name in (root,) or name in TORCH_SUBMODULES

    def visit_Import(self, node):
        for alias in node.names:
            if not self._import_ok(alias.name):
                self.refuse(node, f"`import {alias.name}` (modules allowed: {sorted(IMPORT_ROOTS)}, "
                                  f"{sorted(TORCH_SUBMODULES)})")

    def visit_ImportFrom(self, node):
        if node.level or not node.module or not self._import_ok(node.module):
            self.refuse(node, f"`from {'.' * node.level}{node.module or ''} import ...`")

    def visit_Name(self, node):
        if node.id.startswith("__"):
            self.refuse(node, f"dunder name `{node.id}`")
        elif node.id in BUILTIN_NAMES and node.id not in BUILTINS_ALLOWED:
            self.refuse(node, f"builtin `{node.id}` is not on the allowlist")
        self.generic_visit(node)

    def visit_Attribute(self, node):
        if isinstance(node.ctx, (ast.Store, ast.Del)):
            self.refuse(node, f"stores into or deletes the attribute `.{node.attr}`")
        if node.attr.startswith("_"):
            self.refuse(node, f"private attribute `.{node.attr}`")
        if node.attr in _REFUSED:
            self.refuse(node, f"`.{node.attr}` {_REFUSED[node.attr]}")
        self.generic_visit(node)

    def visit_Call(self, node):
        f = node.func
        while isinstance(f, ast.Attribute):
            if isinstance(f.value, ast.Name) and f.value.id == "vmk":
                self.calls_vmk = True
            f = f.value
        self.generic_visit(node)

    def _scope(self, node):
        self.refuse(node, f"`{type(node).__name__.lower()}` statement")

    visit_Global = visit_Nonlocal = _scope

    def _coroutine(self, node):
        self.refuse(node, f"{type(node).__name__} (no async code or generators)")
        self.generic_visit(node)

    visit_AsyncFunctionDef = visit_Await = visit_Yield = visit_YieldFrom = _coroutine


def screen(src):
    """Problems found in a kernel module's source; an empty list means it may run."""
    if len(src.encode()) > SIZE_LIMIT:
        return [f"the module is larger than {SIZE_LIMIT} bytes"]
    try:
        tree = ast.parse(src)
    except SyntaxError as e:
        return [f"does not parse: {e}"]
    s = _Screen()
    s.visit(tree)
    if not any(isinstance(n, ast.FunctionDef) and n.name == "kernel" for n in tree.body):
        s.problems.append("no top-level `def kernel(...)`")
    if not s.calls_vmk:
        s.problems.append("never calls into vmk: the libvmk kernels must do the work")
    return s.problems


# ============================================================================================ worker side
def _module(path):
    spec = importlib.util.spec_from_file_location("kernel_under_test", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _outputs(result):
    return list(result) if isinstance(result, (tuple, list)) else [result]


def _host(t):
    """An output on the host: bf16 widened to float32 (NumPy has no bf16), anything else as it is."""
    import torch
    return (t.float() if t.dtype == torch.bfloat16 else t).cpu().numpy()


def _bytes(t):
    """An output's raw bytes, row by row, on the host (the row-invariance layer compares bits)."""
    import torch
    return t.contiguous().view(torch.uint8).reshape(t.shape[0], -1).cpu().numpy()


class Worker:
    """Runs a kernel module over a case plan and writes each case as soon as it finishes."""

    def __init__(self, opname, module_path, outdir, device="cuda"):
        self.opname, self.outdir, self.device = opname, outdir, device
        self.op = load_op(opname)
        self.mod = _module(module_path)
        self.select = getattr(self.mod, "select", None) if opname == "dsa" else None
        self.manifest = open(os.path.join(outdir, "manifest.jsonl"), "a")

    def sync(self):
        import torch
        if self.device != "cpu":
            torch.cuda.synchronize()

    def inputs(self, case):
        return kernel_inputs(self.opname, self.op.make_inputs(case.shape, seed=case.seed, dist=case.dist,
                                                              device=self.device))

    def record(self, case, entry, arrays):
        if arrays:
            np.savez(os.path.join(self.outdir, case.key + ".npz"), **arrays)
        self.manifest.write(json.dumps(dict(key=case.key, **entry)) + "\n")
        self.manifest.flush()
        os.fsync(self.manifest.fileno())

    def run_case(self, case):
        inp = self.inputs(case)
        t0 = time.perf_counter()
        outs = _outputs(self.mod.kernel(**inp))
        self.sync()
        arrays = {f"out{j}": _host(o) for j, o in enumerate(outs)}
        entry = dict(ok=True, dtypes=[str(o.dtype) for o in outs], seconds=round(time.perf_counter() - t0, 3))
        if self.select is not None:
            idx, cnt = self.select(inp["iq"], inp["ik"], inp["w"], inp.get("lens"))
            self.sync()
            arrays.update(idx=idx.cpu().numpy(), cnt=cnt.cpu().numpy())
            entry["selection"] = True
        return entry, arrays

    def run_rows(self, case):
        inp = self.inputs(case)
        t0 = time.perf_counter()
        batch = _outputs(self.mod.kernel(**inp))
        self.sync()
        arrays = {f"batch{j}": _bytes(o) for j, o in enumerate(batch)}
        alone = [[] for _ in batch]
        nrows = batch[0].shape[0]
        for r in range(nrows):
            for j, o in enumerate(_outputs(self.mod.kernel(**self.op.row_inputs(inp, r)))):
                alone[j].append(_bytes(o))
            self.sync()
        arrays.update({f"alone{j}": np.concatenate(a) for j, a in enumerate(alone)})
        return dict(ok=True, rows=nrows, outputs=len(batch), seconds=round(time.perf_counter() - t0, 3)), arrays

    def run(self, cases, row_cases):
        for run_one, todo in ((self.run_case, cases), (self.run_rows, row_cases)):
            for case in todo:
                print(f"[worker] {case.key} {case.label} {case.shape} {case.dist}", flush=True)
                try:
                    entry, arrays = run_one(case)
                except Exception as e:             # the case fails; the plan goes on
                    entry, arrays = dict(ok=False, error=f"{type(e).__name__}: {str(e)[:1500]}"), {}
                self.record(case, entry, arrays)
                if self.device != "cpu":
                    import torch
                    torch.cuda.empty_cache()
        self.manifest.close()


def read_results(outdir):
    """key -> (manifest entry, arrays or None), for every case the worker finished."""
    done = {}
    path = os.path.join(outdir, "manifest.jsonl")
    if not os.path.exists(path):
        return done
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line:
                continue
            try:
                e = json.loads(line)
            except json.JSONDecodeError:           # a line cut short by a dying worker
                continue
            npz = os.path.join(outdir, e["key"] + ".npz")
            done[e["key"]] = (e, dict(np.load(npz)) if os.path.exists(npz) else None)
    return done


# ============================================================================================ scoring side
def _f64(x):
    import torch
    if isinstance(x, torch.Tensor):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


class Scorer:
    """Scores finished cases of one op; references are computed lazily, once per case."""

    def __init__(self, opname, device="cuda"):
        self.opname, self.device = opname, device
        self.op = load_op(opname)
        self.oracle = importlib.import_module(ORACLES[opname])
        self.std_l1 = getattr(self.op, self.op.L1_REF)
        self.std_l3 = getattr(self.op, self.op.L3_REF)
        self._last = None

    def sync(self):
        import torch
        if self.device != "cpu":
            torch.cuda.synchronize()

    def context(self, case):
        """The references of `case`; the last case's are kept, since the TK layer scores the same case next."""
        if self._last is None or self._last.case is not case:
            self._last = _Refs(self, case)
        return self._last

    # -- rules: each returns (ok, details)
    def rule_standard(self, refs, outs, dtypes):
        want = refs.standard(self.std_l1)
        if (msg := _shape_mismatch(outs, want)):
            return False, dict(error=msg)
        close = [bool(np.allclose(o, w, rtol=1e-2, atol=1e-2, equal_nan=True)) for o, w in zip(outs, want)]
        worst = max((float(np.nanmax(np.abs(o - w))) if o.size else 0.0) for o, w in zip(outs, want))
        return all(close), dict(max_abs_diff=worst)

    def rule_fuzz(self, refs, outs, dtypes):
        want = refs.oracle()
        if (msg := _shape_mismatch(outs, want)):
            return False, dict(error=msg)
        ok, det = True, dict(err_max=0.0, err_mean=0.0)
        for j, (o, w) in enumerate(zip(outs, want)):
            kind = rounding_of(dtypes[j])
            on, oi = nonfinite(o, kind)
            wn, wi = nonfinite(w, kind)
            same = np.array_equal(on, wn) and np.array_equal(oi, wi)
            if not same and refs.case.dist == "nan_inf":
                sn, si = nonfinite(refs.standard(self.std_l3)[j], kind)
                same = np.array_equal(on, sn) and np.array_equal(oi, si)
                det["nonfinite_matched"] = "standard op"
            if not same:
                det.setdefault("nonfinite_mismatch", []).append(
                    dict(output=j, nan=[int(on.sum()), int(wn.sum())], inf=[int(oi.sum()), int(wi.sum())]))
            emax, emean = normalised_error(o, w)
            det["err_max"], det["err_mean"] = max(det["err_max"], emax), max(det["err_mean"], emean)
            ok = ok and same and emax <= 1e-2
        return ok, det

    def rule_relative(self, refs, outs, dtypes):
        want = refs.oracle()
        if (msg := _shape_mismatch(outs, want)):
            return False, dict(error=msg)
        std = refs.standard(self.std_l3)
        ok, det = True, {}
        for j, (o, w, s) in enumerate(zip(outs, want, std)):
            kmax, kmean = normalised_error(o, w)
            smax, smean = normalised_error(s, w)
            okj = kmax <= 2 * max(smax, FLOOR) and kmean <= 2 * max(smean, FLOOR)
            det[f"out{j}"] = dict(kernel=[kmax, kmean], standard=[smax, smean])
            ok = ok and okj
        return ok, det

    def score(self, layer, case, entry, arrays):
        res = case.describe()
        if entry is None:
            return dict(res, ok=False, error="the worker did not finish this case")
        if not entry["ok"]:
            return dict(res, ok=False, error=entry["error"])
        outs = [arrays[f"out{j}"].astype(np.float64) for j in range(len(entry["dtypes"]))]
        refs = self.context(case)
        ok = True
        for rule in layer.rules:
            okr, det = getattr(self, "rule_" + rule)(refs, outs, entry["dtypes"])
            res[rule] = det
            ok = ok and okr
        res["ok"] = bool(ok)
        return res

    def score_selection(self, case, entry, arrays):
        """The TK layer for one case whose worker entry holds a selection."""
        res = case.describe()
        refs = self.context(case)
        s64, _ = refs.selection()
        i = refs.inputs
        bound = self.oracle.score_error_bound(i["iq"], i["ik"], i["w"], i.get("lens"))
        lens = i.get("lens")
        lens = None if lens is None else lens.cpu().numpy()
        per = []
        ok = True
        for b in range(s64.shape[0]):
            n = s64.shape[1] if lens is None else int(lens[b])
            okb, det = self.oracle.topk_set_check(arrays["idx"][b], int(arrays["cnt"][b]), s64[b], n, bound[b])
            ok = ok and okb
            per.append(det)
        res.update(ok=bool(ok), boundary=[d.get("boundary", 0) for d in per],
                   swapped=[d.get("swapped", 0) for d in per])
        if not ok:
            res["requests"] = per
        return res


class _Refs:
    """Inputs and references of one case, each built on first use."""

    def __init__(self, scorer, case):
        self.s, self.case = scorer, case
        self._inp, self._oracle, self._std, self._sel = None, None, {}, None

    @property
    def inputs(self):
        if self._inp is None:
            c = self.case
            self._inp = self.s.op.make_inputs(c.shape, seed=c.seed, dist=c.dist, device=self.s.device)
        return self._inp

    def standard(self, fn):
        if fn not in self._std:
            self._std[fn] = [_f64(x) for x in _outputs(fn(**self.inputs))]
            self.s.sync()
        return self._std[fn]

    def oracle(self):
        if self._oracle is None:
            self._oracle = [_f64(x) for x in _outputs(self.s.oracle.ref64(**kernel_inputs(self.s.opname,
                                                                                            self.inputs)))]
        return self._oracle

    def selection(self):
        if self._sel is None:
            i = self.inputs
            self._sel = self.s.oracle.ref_select64(i["iq"], i["ik"], i["w"], i.get("lens"))
        return self._sel


def _shape_mismatch(outs, want):
    got_s, want_s = [o.shape for o in outs], [w.shape for w in want]
    return None if got_s == want_s else f"the kernel returned shapes {got_s}; the reference has {want_s}"


def score_rows(case, entry, arrays):
    """The L4 layer for one case: rows of the batch output whose bytes differ from the same row computed alone."""
    res = case.describe()
    if entry is None:
        return dict(res, ok=False, error="the worker did not finish this case")
    if not entry["ok"]:
        return dict(res, ok=False, error=entry["error"])
    differ = set()
    for j in range(entry["outputs"]):
        a, b = arrays[f"batch{j}"], arrays[f"alone{j}"]
        if a.shape != b.shape:
            return dict(res, ok=False, error=f"output {j}: batch bytes {a.shape} vs rows alone {b.shape}")
        differ |= set(np.nonzero((a != b).any(axis=1))[0].tolist())
    return dict(res, ok=not differ, rows=entry["rows"], differing=len(differ), first_differing=sorted(differ)[:16])


def assess(opname, outdir, device="cuda", cases=None, row_cases=None):
    """The report of one worker run: every layer's cases, scored; the verdict."""
    import torch
    sc = Scorer(opname, device)
    cases = plan(sc.op) if cases is None else cases
    row_cases = row_plan(sc.op) if row_cases is None else row_cases
    done = read_results(outdir)
    layers = {name: [] for name in ALL_LAYERS}
    by_name = {l.name: l for l in LAYERS}
    for case in cases:
        entry, arrays = done.get(case.key, (None, None))
        layers[case.layer].append(sc.score(by_name[case.layer], case, entry, arrays))
        if entry is not None and entry.get("selection"):
            layers[TOPK_LAYER].append(sc.score_selection(case, entry, arrays))
        if device != "cpu":
            torch.cuda.empty_cache()
    for case in row_cases:
        entry, arrays = done.get(case.key, (None, None))
        layers[ROW_LAYER.name].append(score_rows(case, entry, arrays))
    titles = {l.name: l.title for l in LAYERS}
    titles.update({TOPK_LAYER: "top-2048 set vs float64", ROW_LAYER.name: ROW_LAYER.title})
    rep = dict(op=opname, layers={name: dict(title=titles[name], passed=sum(c["ok"] for c in cs), total=len(cs),
                                             cases=cs) for name, cs in layers.items()})
    rep["verdict"] = "CORRECT" if all(v["passed"] == v["total"] for v in rep["layers"].values()) else "REJECTED"
    if device != "cpu":
        rep["sdpa_backends"] = dict(flash=torch.backends.cuda.flash_sdp_enabled(),
                                    mem_efficient=torch.backends.cuda.mem_efficient_sdp_enabled(),
                                    math=torch.backends.cuda.math_sdp_enabled())
    return rep


def render(rep, show=8):
    """A short text form of a report: one line per layer, then the first failing cases."""
    lines = []
    for name, v in rep["layers"].items():
        if v["total"]:
            lines.append(f"  {name:<4}{v['passed']:>4}/{v['total']:<4} {v['title']}")
    lines.append(f"verdict: {rep['verdict']}")
    bad = [c for v in rep["layers"].values() for c in v["cases"] if not c["ok"]]
    for c in bad[:show]:
        brief = {k: v for k, v in c.items() if k not in ("ok", "requests")}
        lines.append("  failed " + json.dumps(brief, default=str)[:700])
    if len(bad) > show:
        lines.append(f"  (+{len(bad) - show} more failed cases)")
    return "\n".join(lines)


def op_from_filename(path):
    """The longest op name that the file's name starts with, followed by '_' (prefix_paged_x.py -> prefix_paged)."""
    stem = os.path.basename(path)
    names = [op for op in KEYS if stem.startswith(op + "_")]
    return max(names, key=len) if names else None


# ============================================================================================ command line
def run_worker(opname, module_path, outdir, timeout, device):
    """Starts the worker process and waits for it; returns its exit status, or 'timeout'."""
    cmd = [sys.executable, os.path.abspath(__file__), "--worker", opname, module_path, outdir, device]
    try:
        return subprocess.run(cmd, timeout=timeout).returncode
    except subprocess.TimeoutExpired:
        return "timeout"


def main(argv=None):
    argv = sys.argv[1:] if argv is None else list(argv)
    if argv[:1] == ["--worker"]:
        opname, module_path, outdir, device = argv[1:5]
        w = Worker(opname, module_path, outdir, device)
        w.run(plan(w.op), row_plan(w.op))
        return 0
    ap = argparse.ArgumentParser(description="Judge one kernel module (the module docstring explains the layers).")
    ap.add_argument("kernel", help="path of the kernel module (defines `kernel(...)`)")
    ap.add_argument("--op", choices=sorted(KEYS), help="the op; by default taken from the file name")
    ap.add_argument("--skip-gate", action="store_true", help="run without screening the source")
    ap.add_argument("--json", help="also write the full report to this file")
    ap.add_argument("--timeout", type=int, default=1800, help="seconds the worker process may run")
    ap.add_argument("--device", default="cuda", help=argparse.SUPPRESS)
    a = ap.parse_args(argv)
    opname = a.op or op_from_filename(a.kernel)
    if opname is None:
        print(f"{a.kernel}: no op name at the start of the file name; give --op", file=sys.stderr)
        return 2
    path = os.path.abspath(a.kernel)
    print(f"{a.kernel}  (op {opname})", flush=True)
    if a.skip_gate:
        print("screening: off (--skip-gate)")
    else:
        problems = screen(open(path).read())
        if problems:
            print("screening: refused, the module was not run")
            print("\n".join("  " + p for p in problems))
            print("verdict: REJECTED")
            return 1
        print("screening: passed")
    t0 = time.time()
    with tempfile.TemporaryDirectory() as td:
        status = run_worker(opname, path, td, a.timeout, a.device)
        rep = assess(opname, td, a.device)
    rep.update(kernel=a.kernel, worker_exit=status, seconds=round(time.time() - t0, 1))
    if status != 0:
        print(f"worker process ended with status {status}; unfinished cases count as failed")
    print(render(rep))
    print(f"({rep['seconds']} s)", flush=True)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rep, f, indent=1, default=str)
    return 0 if rep["verdict"] == "CORRECT" else 1


if __name__ == "__main__":
    sys.exit(main())
