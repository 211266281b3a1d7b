"""Shared helpers of the float64 oracle (test infrastructure only)."""
import numpy as np


def to64(x):
    """torch tensor / numpy array (any float dtype) -> float64 numpy, through float32 like the reference's
    `np.array(x.astype(mx.float32)).astype(np.float64)` (ops/prefix.py:58)."""
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x).astype(np.float32).astype(np.float64)


def toint(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def softmax_attend(s, v):
    """softmax over the last axis with the max subtracted, then p @ v, with the reference's NaN/Inf behaviour:
    a NaN score makes its row NaN, +inf - +inf gives NaN, a -inf (masked) score gives p = 0
    (ops/spec.py:77-81, ops/prefix.py:65-69)."""
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        return p @ v
