"""Error measures and NaN/Inf pattern of the three-layer verifier (verify.py:160-171 of the reference; bf16 outputs
are this build's)."""
import numpy as np


def nerr(o, r):
    """Normalised error over entries finite in both: |o - r| / max(1, max|r|); returns (max, mean)."""
    o = np.asarray(o, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    fin = np.isfinite(r) & np.isfinite(o)
    if not fin.any():
        return 0.0, 0.0
    scale = max(1.0, float(np.abs(r[fin]).max()))
    d = np.abs(o[fin] - r[fin]) / scale
    return float(d.max()), float(d.mean())


BF16_OVERFLOW = (2.0 - 2.0 ** -8) * 2.0 ** 127       # float values at or above this round to bf16 inf


def pattern(a, half=True):
    """NaN and Inf masks of `a` rounded to the output type: half=True (or "fp16") fp16, "bf16" bf16 (rounding to
    nearest even overflows at (2 - 2^-8) * 2^127), False (or "fp32") float32."""
    a = np.asarray(a, dtype=np.float64)
    if half == "bf16":
        with np.errstate(invalid="ignore"):
            return np.isnan(a), np.isinf(a) | (np.abs(a) >= BF16_OVERFLOW)
    a16 = a.astype(np.float16 if half in (True, "fp16") else np.float32)
    return np.isnan(a16), np.isinf(a16)


def kind_of(dtype_name):
    """pattern()'s rounding for an output dtype name such as 'torch.bfloat16'."""
    return "bf16" if "bfloat16" in dtype_name else ("fp32" if "float32" in dtype_name else "fp16")


def same_pattern(o, r, half=True):
    pn, pi = pattern(o, half)
    rn, ri = pattern(r, half)
    return bool((pn == rn).all() and (pi == ri).all())
