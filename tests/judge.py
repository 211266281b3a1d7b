"""Error measures and NaN/Inf pattern of the three-layer verifier (verify.py:160-171 of the reference)."""
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


def pattern(a, half=True):
    a16 = np.asarray(a).astype(np.float16 if half else np.float32)
    return np.isnan(a16), np.isinf(a16)


def same_pattern(o, r, half=True):
    pn, pi = pattern(o, half)
    rn, ri = pattern(r, half)
    return bool((pn == rn).all() and (pi == ri).all())
