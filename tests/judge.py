"""Numerical scores of the verifier.

Two measures decide the fuzz and error layers (the reference harness defines them, verify.py:160-171):
  * the normalised error of an output against a float64 reference: over the entries finite in both, the absolute
    difference divided by max(1, largest |reference| among those entries), as a (max, mean) pair;
  * where an output holds NaN and Inf once rounded to the kernel's output type.  The reference rounds to fp16 or
    float32; rounding to bf16 is this build's addition, since its entry points also produce bf16.
"""
import numpy as np

# Round-to-nearest-even sends a float to bf16 infinity at and above the midpoint between bf16's largest finite
# value (2 - 2^-7) * 2^127 and 2^128, i.e. (2 - 2^-8) * 2^127.
BF16_INF_FROM = (2.0 - 2.0 ** -8) * 2.0 ** 127


def normalised_error(got, want):
    """(max, mean) normalised error of `got` against the reference `want`; (0.0, 0.0) when no entry is finite in
    both."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    both = np.isfinite(g) & np.isfinite(w)
    if not np.any(both):
        return 0.0, 0.0
    g, w = g[both], w[both]
    denom = np.maximum(1.0, np.abs(w).max())
    d = np.abs(g - w) / denom
    return float(d.max()), float(d.mean())


def rounding_of(dtype_name):
    """The output type an output's dtype name ('torch.float16', 'torch.bfloat16', 'torch.float32', ...) rounds
    to: 'fp16', 'bf16' or 'fp32'."""
    if "bfloat16" in dtype_name:
        return "bf16"
    if "float32" in dtype_name:
        return "fp32"
    return "fp16"


def nonfinite(a, kind="fp16"):
    """(nan mask, inf mask) of `a` after rounding to `kind` ('fp16', 'bf16' or 'fp32')."""
    x = np.asarray(a, dtype=np.float64)
    if kind == "bf16":
        with np.errstate(invalid="ignore"):
            return np.isnan(x), np.isinf(x) | (np.abs(x) >= BF16_INF_FROM)
    if kind not in ("fp16", "fp32"):
        raise ValueError(f"unknown rounding {kind!r}")
    with np.errstate(over="ignore", invalid="ignore"):
        r = x.astype(np.float16 if kind == "fp16" else np.float32)
    return np.isnan(r), np.isinf(r)


def same_nonfinite(a, b, kind="fp16"):
    """True when `a` and `b` have NaN at the same positions and Inf at the same positions after rounding."""
    an, ai = nonfinite(a, kind)
    bn, bi = nonfinite(b, kind)
    return bool(np.array_equal(an, bn) and np.array_equal(ai, bi))
