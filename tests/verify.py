"""Three-layer verifier for one kernel module (the counterpart of the reference's verify.py, with a PyTorch-ROCm
adapter): the standard op of L1/L3 is a PyTorch SDPA composition on the GPU where the reference used MLX, and
L2/L3 keep judging against the NumPy float64 oracle.

    python tests/verify.py verified-metal-kernels_amd/kernels/spec_mi355x.py          # op from the file name
    python tests/verify.py tests/wrong_kernels/spec_cheat_nomax.py --skip-gate
    python tests/verify.py my_kernel.py --op dsa --json out.json

A kernel module has a top-level `def kernel(...)` taking the op's inputs as keyword arguments (vmk.ops.KEYS).

Steps (verify.py:10-24 of the reference):
  0. static gate (AST whitelist, before import): imports limited to torch, math, functools and the vmk package; no
     file/OS access, no reflection, no attribute stores, no standard attention/top-k/sort entry points, and at least
     one call into vmk (the libvmk kernels).  --skip-gate disables it (needed for tests/wrong_kernels/).
  1. the kernel is imported and run on every case in a CHILD process, which saves its raw outputs;
  2. the verdict is computed in THIS process, which never imports the kernel, by regenerating the same inputs:
     L1: 5 seeds at the nominal shape, allclose(atol=rtol=1e-2) against the PyTorch standard op;
     L2: fuzzing against the float64 oracle: NaN/Inf pattern equal to the oracle rounded to fp16 (for nan_inf
         inputs: equal to the standard op's pattern), normalised max error <= 1e-2;
     L3: max and mean error vs float64 <= 2 * max(standard op error, 2^-11).
  This build adds three judged groups outside the reference's counts: X (the op's EXTRA cases: ragged suffixes,
  K outliers, kd > 32 masks, ...) judged like L2; TK (dsa only, when the module exports `select`): the
  selected index set must equal the float64 top-2048 outside the boundary-tie band (oracle.dsa.topk_set_check);
  and L4 (the judge's fourth layer, ONE-PAGER.md:13-14, absent from the public verify.py): on the op's L4_CASES,
  every batch row computed alone (the op's `row_inputs`) must have the same output bits as in the batch.
  An exception on any case is a failure.  Verdict: CORRECT only if every case of every group passes.

Exit code: 0 = CORRECT, 1 = REJECTED, 2 = usage error.
"""
import argparse
import ast
import importlib.util
import json
import os
import subprocess
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "verified-metal-kernels_amd")
for _p in (ROOT, PKG, HERE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

from vmk.ops import KEYS, load_op  # noqa: E402

ORACLE = {"prefix": "oracle.prefix", "spec": "oracle.spec", "dsa": "oracle.dsa", "decode": "oracle.decode",
          "prefix_paged": "oracle.prefix_paged"}


def cand_inputs(opname, inp):
    return {k: inp.get(k) for k in KEYS[opname]}


def cases(op, extra=True):
    """Verification cases, identical in the child (kernel outputs) and the parent (judgement): verify.py:48-53."""
    out = [("L1", i, op.L1_SHAPE, "randn", 100 + i) for i in range(5)]
    out += [("L2", i, s, d, 7 + i) for i, (s, d) in enumerate(op.FUZZ)]
    out += [("L3", i, s, d, 3) for i, (s, d) in enumerate(op.L3_CASES)]
    if extra:
        out += [("X", i, s, d, 50 + i) for i, (s, d) in enumerate(getattr(op, "EXTRA", []))]
    return out


# ------------------------------------------------------------------------------------------------ static gate
ALLOWED_IMPORTS = {"torch", "math", "functools", "vmk"}
BANNED_NAMES = {"open", "exec", "eval", "compile", "__import__", "globals", "locals", "vars", "getattr", "setattr",
                "delattr", "input", "breakpoint", "help", "exit", "quit", "memoryview", "super", "classmethod",
                "staticmethod", "property", "type", "object", "dir", "id", "hash", "print"}
BANNED_ATTRS = {"save", "load", "manual_seed", "seed", "set_default_device", "set_default_dtype", "distributed",
                "random", "rand", "randn", "scaled_dot_product_attention", "softmax", "log_softmax", "topk", "sort",
                "argsort", "kthvalue", "msort", "multi_head_attention_forward", "flash_attention", "cuda_kernel",
                "load_inline", "cpp_extension", "system", "popen"}
MAX_BYTES = 200_000


def gate(src):
    """List of violations (empty = accepted); verify.py:57-108 with torch/vmk in place of mlx.core."""
    errs = []
    if len(src.encode()) > MAX_BYTES:
        return [f"module larger than {MAX_BYTES} bytes"]
    try:
        tree = ast.parse(src)
    except SyntaxError as e:
        return [f"SyntaxError: {e}"]
    if not any(isinstance(n, ast.FunctionDef) and n.name == "kernel" for n in tree.body):
        errs.append("no top-level `def kernel(...)`")
    uses_vmk = False
    for n in ast.walk(tree):
        if isinstance(n, ast.Import):
            for a in n.names:
                if a.name.split(".")[0] not in ALLOWED_IMPORTS or (a.name.startswith("torch.") and
                                                                     a.name != "torch.nn.functional"):
                    errs.append(f"line {n.lineno}: import {a.name} not allowed")
        elif isinstance(n, ast.ImportFrom):
            if not n.module or n.module.split(".")[0] not in ALLOWED_IMPORTS or n.level:
                errs.append(f"line {n.lineno}: from {n.module} import ... not allowed")
        elif isinstance(n, ast.Name):
            if n.id in BANNED_NAMES or n.id.startswith("__"):
                errs.append(f"line {n.lineno}: name `{n.id}` not allowed")
        elif isinstance(n, ast.Attribute):
            if isinstance(n.ctx, (ast.Store, ast.Del)):
                errs.append(f"line {n.lineno}: assigning/deleting attributes is not allowed")
            if n.attr.startswith("_"):
                errs.append(f"line {n.lineno}: attribute `.{n.attr}` not allowed")
            if n.attr in BANNED_ATTRS:
                errs.append(f"line {n.lineno}: `.{n.attr}` not allowed")
            if isinstance(n.value, ast.Name) and n.value.id == "vmk":
                uses_vmk = True
        elif isinstance(n, (ast.Global, ast.Nonlocal)):
            errs.append(f"line {n.lineno}: global/nonlocal not allowed")
        elif isinstance(n, (ast.AsyncFunctionDef, ast.Await, ast.Yield, ast.YieldFrom)):
            errs.append(f"line {n.lineno}: async/generators not allowed")
    if not uses_vmk:
        errs.append("no call into vmk found: the hot path must use the libvmk kernels")
    return errs


def import_module(path):
    s = importlib.util.spec_from_file_location("candidate_kernel", path)
    m = importlib.util.module_from_spec(s)
    s.loader.exec_module(m)
    return m


# ------------------------------------------------------------------------------------------------ child side
def as_tuple(o):
    return tuple(o) if isinstance(o, (tuple, list)) else (o,)


def child_outputs(opname, kernel_path, out):
    """The only function that imports the kernel.  Saves raw outputs (.npz) and per-case status (.json)."""
    import torch
    mod = import_module(kernel_path)
    fn = mod.kernel
    sel = getattr(mod, "select", None) if opname == "dsa" else None
    op = load_op(opname)
    arrays, meta = {}, {}
    for layer, i, shape, dist, seed in cases(op):
        key = f"{layer}_{i}"
        inp = cand_inputs(opname, op.make_inputs(shape, seed=seed, dist=dist, device="cuda"))
        t0 = time.time()
        try:
            o = as_tuple(fn(**inp))
            torch.cuda.synchronize()
            for j, a in enumerate(o):
                arrays[f"{key}__{j}"] = a.float().cpu().numpy() if a.dtype == torch.bfloat16 else a.cpu().numpy()
            meta[key] = dict(ok=True, n_out=len(o), dtypes=[str(a.dtype) for a in o], s=time.time() - t0)
            if sel is not None:
                idx, cnt = sel(inp["iq"], inp["ik"], inp["w"], inp.get("lens"))
                torch.cuda.synchronize()
                arrays[f"{key}__idx"], arrays[f"{key}__cnt"] = idx.cpu().numpy(), cnt.cpu().numpy()
                meta[key]["select"] = True
        except Exception as e:
            meta[key] = dict(ok=False, error=f"{type(e).__name__}: {str(e)[:1500]}")
        del inp
        torch.cuda.empty_cache()
    for i, (shape, dist) in enumerate(getattr(op, "L4_CASES", [])):
        key = f"L4_{i}"
        inp = cand_inputs(opname, op.make_inputs(shape, seed=200 + i, dist=dist, device="cuda"))
        t0 = time.time()
        try:
            full = as_tuple(fn(**inp))
            torch.cuda.synchronize()
            full = [a.cpu().numpy() for a in full]
            nrows = full[0].shape[0]
            rows = [[] for _ in full]
            for r in range(nrows):
                o = as_tuple(fn(**op.row_inputs(inp, r)))
                torch.cuda.synchronize()
                for j, a in enumerate(o):
                    rows[j].append(a.cpu().numpy())
            for j, a in enumerate(full):
                arrays[f"{key}__full{j}"] = a
                arrays[f"{key}__rows{j}"] = np.concatenate(rows[j])
            meta[key] = dict(ok=True, n_out=len(full), n_rows=nrows, s=time.time() - t0)
        except Exception as e:
            meta[key] = dict(ok=False, error=f"{type(e).__name__}: {str(e)[:1500]}")
        del inp
        torch.cuda.empty_cache()
    np.savez(out + ".npz", **arrays)
    json.dump(meta, open(out + ".json", "w"))


# ------------------------------------------------------------------------------------------------ parent side
from judge import kind_of, nerr, pattern  # noqa: E402


def to64(a):
    import torch
    if isinstance(a, torch.Tensor):
        a = a.detach().float().cpu().numpy()
    return np.asarray(a).astype(np.float64)


def judge(opname, outpath):
    """verify.py:174-241 of the reference, against the float64 oracle and the PyTorch standard op."""
    import importlib
    import torch
    op = load_op(opname)
    orc = importlib.import_module(ORACLE[opname])
    meta = json.load(open(outpath + ".json"))
    arrs = np.load(outpath + ".npz")
    std1, std3 = getattr(op, op.L1_REF), getattr(op, op.L3_REF)
    rep = dict(L1=[], L2=[], L3=[], X=[], TK=[])
    for layer, i, shape, dist, seed in cases(op):
        key = f"{layer}_{i}"
        case = dict(case=key, shape=shape, dist=dist)
        m = meta.get(key, dict(ok=False, error="missing (child crashed or timed out before this case)"))
        if not m["ok"]:
            case.update(ok=False, error=m["error"])
            rep[layer].append(case)
            continue
        inp = op.make_inputs(shape, seed=seed, dist=dist, device="cuda")
        outs = [arrs[f"{key}__{j}"].astype(np.float64) for j in range(m["n_out"])]
        if m.get("select"):
            s64, _ = orc.ref_select64(inp["iq"], inp["ik"], inp["w"], inp["lens"])
            idx, cnt = arrs[f"{key}__idx"], arrs[f"{key}__cnt"]
            lens = None if inp["lens"] is None else inp["lens"].cpu().numpy()
            tk_ok, det = True, []
            for b in range(s64.shape[0]):
                n = shape["L"] if lens is None else int(lens[b])
                okb, d = orc.topk_set_check(idx[b], int(cnt[b]), s64[b], n)
                tk_ok &= okb
                det.append(d)
            rep["TK"].append(dict(case=key, shape=shape, dist=dist, ok=bool(tk_ok), detail=det if not tk_ok else None))
        if layer == "L1":
            s = [to64(x) for x in as_tuple(std1(**inp))]
            torch.cuda.synchronize()
            if len(s) != len(outs) or any(a.shape != b.shape for a, b in zip(outs, s)):
                case.update(ok=False, error=f"output shapes {[a.shape for a in outs]} != expected {[b.shape for b in s]}")
            else:
                ok = all(np.allclose(a, b, atol=1e-2, rtol=1e-2, equal_nan=True) for a, b in zip(outs, s))
                case.update(ok=bool(ok), maxdiff=max(float(np.nanmax(np.abs(a - b))) if a.size else 0.0
                                                     for a, b in zip(outs, s)))
            rep[layer].append(case)
            continue
        r = [to64(x) for x in as_tuple(orc.ref64(**cand_inputs(opname, inp)))]
        if len(r) != len(outs) or any(a.shape != b.shape for a, b in zip(outs, r)):
            case.update(ok=False, error=f"output shapes {[a.shape for a in outs]} != expected {[b.shape for b in r]}")
            rep[layer].append(case)
            continue
        if layer in ("L2", "X"):
            pat_ok, emax, emean, s = True, 0.0, 0.0, None
            for j, (o, rr) in enumerate(zip(outs, r)):
                half = kind_of(m["dtypes"][j])
                pn, pi = pattern(o, half)
                rn, ri = pattern(rr, half)
                pj = bool((pn == rn).all() and (pi == ri).all())
                if not pj and dist == "nan_inf":
                    s = s or [to64(x) for x in as_tuple(std3(**inp))]
                    sn, si = pattern(s[j], half)
                    pj = bool((pn == sn).all() and (pi == si).all())
                    case["pattern_vs"] = "std_op"
                if not pj:
                    case.setdefault("pattern_detail", []).append(
                        dict(output=j, nan_got=int(pn.sum()), nan_exp=int(rn.sum()), inf_got=int(pi.sum()),
                             inf_exp=int(ri.sum())))
                em, ea = nerr(o, rr)
                pat_ok, emax, emean = pat_ok and pj, max(emax, em), max(emean, ea)
            case.update(ok=bool(pat_ok and emax <= 1e-2), pattern_ok=pat_ok, err_max=emax, err_mean=emean)
        else:
            s = [to64(x) for x in as_tuple(std3(**inp))]
            ok, worst = True, {}
            for j, (o, rr, ss) in enumerate(zip(outs, r, s)):
                em, ea = nerr(o, rr)
                sm, sa = nerr(ss, rr)
                tol = 2.0 ** -11
                okj = em <= 2 * max(sm, tol) and ea <= 2 * max(sa, tol)
                ok = ok and okj
                worst[f"out{j}"] = dict(err_max=em, err_mean=ea, std_err_max=sm, std_err_mean=sa)
            case.update(ok=bool(ok), errors=worst)
        rep[layer].append(case)
        del inp
        torch.cuda.empty_cache()
    rep["L4"] = [l4_case(meta, arrs, i, shape, dist) for i, (shape, dist) in enumerate(getattr(op, "L4_CASES", []))]
    for layer in LAYERS:
        rep[f"{layer}_pass"] = sum(c["ok"] for c in rep[layer])
        rep[f"{layer}_n"] = len(rep[layer])
    rep["verdict"] = "CORRECT" if all(rep[f"{l}_pass"] == rep[f"{l}_n"] for l in LAYERS) else "REJECTED"
    rep["sdpa_backends"] = dict(flash=torch.backends.cuda.flash_sdp_enabled(),
                                mem_efficient=torch.backends.cuda.mem_efficient_sdp_enabled(),
                                math=torch.backends.cuda.math_sdp_enabled())
    return rep


LAYERS = ("L1", "L2", "L3", "X", "TK", "L4")


def l4_case(meta, arrs, i, shape, dist):
    """Row invariance: each output row of the batch call must be bit-equal to the same row computed alone."""
    key = f"L4_{i}"
    case = dict(case=key, shape=shape, dist=dist)
    m = meta.get(key, dict(ok=False, error="missing (child crashed or timed out before this case)"))
    if not m["ok"]:
        case.update(ok=False, error=m["error"])
        return case
    bad = []
    for j in range(m["n_out"]):
        full, rows = arrs[f"{key}__full{j}"], arrs[f"{key}__rows{j}"]
        if full.shape != rows.shape or full.dtype != rows.dtype:
            case.update(ok=False,
                        error=f"output {j}: batch {full.shape} {full.dtype} vs rows {rows.shape} {rows.dtype}")
            return case
        fb = full.reshape(full.shape[0], -1).view(np.uint8)
        rb = rows.reshape(rows.shape[0], -1).view(np.uint8)
        bad += [r for r in range(full.shape[0]) if not np.array_equal(fb[r], rb[r]) and r not in bad]
    case.update(ok=not bad, n_rows=m["n_rows"], rows_differing=sorted(bad)[:16], n_differing=len(bad))
    return case


def summary(rep, max_fail=6):
    lines = [f"L1 (standard op, nominal shape)  {rep['L1_pass']}/{rep['L1_n']}",
             f"L2 (fuzzing vs float64)          {rep['L2_pass']}/{rep['L2_n']}",
             f"L3 (numerical error vs float64)  {rep['L3_pass']}/{rep['L3_n']}",
             f"X  (this build's extra cases)    {rep['X_pass']}/{rep['X_n']}"]
    if rep["TK_n"]:
        lines.append(f"TK (top-k set vs float64)        {rep['TK_pass']}/{rep['TK_n']}")
    if rep["L4_n"]:
        lines.append(f"L4 (row alone = row in batch)    {rep['L4_pass']}/{rep['L4_n']}")
    lines.append(f"=> {rep['verdict']}")
    fails = [c for l in LAYERS for c in rep[l] if not c["ok"]]
    for c in fails[:max_fail]:
        d = {k: v for k, v in c.items() if k != "ok"}
        if "error" in d:
            d["error"] = d["error"][:600]
        lines.append("  FAIL " + json.dumps(d, default=str))
    if len(fails) > max_fail:
        lines.append(f"  ... and {len(fails) - max_fail} more failing cases")
    return "\n".join(lines)


def infer_op(path):
    """The longest op name that the file name starts with (prefix_paged_x.py is prefix_paged, not prefix)."""
    base = os.path.basename(path)
    hits = [op for op in KEYS if base.startswith(op + "_")]
    return max(hits, key=len) if hits else None


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) > 0 and argv[0] == "--child":   # internal: verify.py --child OP KERNEL OUT
        child_outputs(argv[1], argv[2], argv[3])
        return 0
    ap = argparse.ArgumentParser(description="Three-layer verifier (see the module docstring).")
    ap.add_argument("kernel", help="path to the kernel module (a file with `def kernel(...)`)")
    ap.add_argument("--op", choices=sorted(KEYS), help="op name (default: inferred from the file name)")
    ap.add_argument("--skip-gate", action="store_true", help="do not apply the static gate (tests/wrong_kernels/)")
    ap.add_argument("--json", help="write the full report to this file")
    ap.add_argument("--timeout", type=int, default=1800, help="child process timeout in seconds")
    a = ap.parse_args(argv)
    opname = a.op or infer_op(a.kernel)
    if opname is None:
        print("cannot infer the op from the file name; pass --op", file=sys.stderr)
        return 2
    kpath = os.path.abspath(a.kernel)
    print(f"kernel: {a.kernel}   op: {opname}", flush=True)
    if a.skip_gate:
        print("static gate: SKIPPED (--skip-gate)")
    else:
        errs = gate(open(kpath).read())
        if errs:
            print("static gate: REJECTED\n  " + "\n  ".join(errs))
            print("=> REJECTED (static gate; the kernel was not imported)")
            return 1
        print("static gate: passed")
    t0 = time.time()
    with tempfile.TemporaryDirectory() as td:
        out = os.path.join(td, "outputs")
        try:
            p = subprocess.run([sys.executable, os.path.abspath(__file__), "--child", opname, kpath, out],
                               timeout=a.timeout)
            rc = p.returncode
        except subprocess.TimeoutExpired:
            rc = "timeout"
        if rc != 0 or not os.path.exists(out + ".json"):
            print(f"child process failed ({rc}) before saving its outputs\n=> REJECTED")
            return 1
        rep = judge(opname, out)
    rep.update(kernel=a.kernel, op=opname, seconds=round(time.time() - t0, 1))
    print(summary(rep))
    print(f"({rep['seconds']} s)", flush=True)
    if a.json:
        json.dump(rep, open(a.json, "w"), indent=1, default=str)
    return 0 if rep["verdict"] == "CORRECT" else 1


if __name__ == "__main__":
    sys.exit(main())
