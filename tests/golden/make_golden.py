"""Writes the golden fixtures of tests/golden/ (run from the repo root: python tests/golden/make_golden.py).

Provenance: the reference cannot run here (every ops/*.py imports mlx.core, which is absent, and no import of the
reference was attempted), and it commits no golden vectors.  These fixtures are therefore made by this build's own
restated generators (vmk.ops.*.make_inputs, following the reference's draw order, ops/*.py:15-50) and float64 oracle
(oracle/).  They pin both against later change: the bytes every (shape, dist, seed) produces, the oracle's outputs
on them, and the first elements of the BASELINE configurations' inputs.  tests/test_golden.py regenerates and
compares.

Files: cases.json lists per op the cases (shape, dist, seed) with the SHA-256 of every input's raw bytes (16-bit floats
as their bits); <op>.npz holds per case i the oracle output's first 64 values (case{i}__head) and its projections on
64 fixed random vectors (case{i}__proj, generator seed 12345), which pin the whole output at a few hundred bytes;
configs.npz holds the first 16 values of each input of C1..C5 (seed 0).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for _p in (ROOT, os.path.join(ROOT, "verified-metal-kernels_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

CASES = {
    "prefix": [(dict(N=3, P=40, S=9), d, 1) for d in ("randn", "large", "needle_prefix", "needle_suffix", "nan_inf",
                                                      "tiny", "outlier")]
    + [(dict(N=4, P=33, S=20, S_min=1), "randn", 2), (dict(N=2, P=1, S=1), "randn", 3)],
    "spec": [(dict(B=2, L=40, k=6), d, 1) for d in ("randn", "chain", "large", "needle_masked", "needle_boundary",
                                                    "nan_inf", "tiny")]
    + [(dict(B=1, L=80, k=40), "tree_bd", 2), (dict(B=1, L=70, k=33), "chain", 3)],
    "dsa": [(dict(B=2, L=300), d, 1) for d in ("randn", "large", "needle", "nan_inf", "tiny")]
    + [(dict(B=3, L=2100), "ragged", 2)],
    "decode": [(dict(B=3, L=50), d, 1) for d in ("randn", "large", "needle", "nan_inf", "tiny")]
    + [(dict(B=4, L=90, L_min=1), "randn", 2), (dict(B=2, L=60, dtype="bf16"), "randn", 3)],
    "prefix_paged": [(dict(N=3, P=64, S=40, S_min=1, ps=32), "randn", 1),
                     (dict(N=4, P=192, S=100, ps=64, absent=2), "randn", 2),
                     (dict(N=2, P=96, S=50, ps=96, dtype="bf16"), "nan_inf", 3)],
}
CONFIG_OPS = {"C1": "prefix", "C2": "prefix", "C3": "spec", "C4": "spec", "C5": "dsa"}


def raw(t):
    """Input tensor -> NumPy array; 16-bit floats as their raw bits (np.uint16), everything else as is."""
    import torch
    if t is None:
        return None
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def case_arrays(opname, shape, dist, seed):
    """{input name: array} and the oracle output of one case."""
    import oracle
    from vmk.ops import KEYS, OPS
    op = OPS[opname]
    inp = {k: v for k, v in op.make_inputs(shape, seed=seed, dist=dist).items() if k in KEYS[opname]}
    out = getattr(oracle, opname).ref64(**inp)
    return {k: raw(v) for k, v in inp.items() if v is not None}, np.asarray(out, dtype=np.float64)


def config_heads():
    """First 16 values (raw bits for 16-bit floats) of every input of C1..C5."""
    from vmk.ops import KEYS, OPS
    arrs = {}
    for name, opname in CONFIG_OPS.items():
        op = OPS[opname]
        shape, dist = op.CONFIGS[name]
        inp = op.make_inputs(shape, seed=0, dist=dist)
        for k in KEYS[opname]:
            if inp.get(k) is not None:
                arrs[f"{name}__{k}"] = raw(inp[k]).reshape(-1)[:16].copy()
        del inp
    return arrs


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def projections(out):
    """64 fixed random projections of the flattened output (NaN/Inf entries replaced by 0, counted separately)."""
    flat = np.nan_to_num(np.asarray(out, dtype=np.float64).reshape(-1), nan=0.0, posinf=0.0, neginf=0.0)
    w = np.random.default_rng(12345).standard_normal((64, flat.size))
    return w @ flat


def main():
    meta = {}
    for opname, cases in CASES.items():
        arrs, rows = {}, []
        for i, (shape, dist, seed) in enumerate(cases):
            ins, out = case_arrays(opname, shape, dist, seed)
            arrs[f"case{i}__head"] = out.reshape(-1)[:64].copy()
            arrs[f"case{i}__proj"] = projections(out)
            rows.append(dict(shape=shape, dist=dist, seed=seed, inputs={k: digest(v) for k, v in ins.items()},
                             nan=int(np.isnan(out).sum()), inf=int(np.isinf(out).sum())))
        np.savez_compressed(os.path.join(HERE, f"{opname}.npz"), **arrs)
        meta[opname] = rows
    np.savez_compressed(os.path.join(HERE, "configs.npz"), **config_heads())
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump(meta, f, indent=1)


if __name__ == "__main__":
    main()
