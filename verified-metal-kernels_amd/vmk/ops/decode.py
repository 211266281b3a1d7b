"""Single-token decode: the op contract (shapes, case lists, input generator, PyTorch standard op).

One query token per request attends to its whole cache (GQA).  The reference ships no kernel module for it; it
benchmarks this decode against llama.cpp with Llama-3-8B heads (llama_cpp/test-backend-ops.patch:79-83) and reports it
at parity (POST.md:42-46).  The shapes below are those cases; the case lists follow the other ops' layout.
    q: (B, Hq, D)   k, v: (B, Hkv, L, D)   lens: (B,) int32 positions in use, or None (all L)
"""
import math

import numpy as np
import torch

from .elem import cast16

NAME = "decode"
HQ, HKV, D = 32, 8, 128                                       # test-backend-ops.patch:79 (32 q heads, 8 kv, D 128)
L1_SHAPE = dict(B=2, L=4096)
BENCH_SHAPES = [dict(B=1, L=8192), dict(B=1, L=32768), dict(B=1, L=65536), dict(B=4, L=16384),
                dict(B=8, L=8192)]                            # test-backend-ops.patch:80
CONFIGS = {"D1": (dict(B=1, L=65536), "randn"), "D2": (dict(B=4, L=16384), "randn"),
           "D3": (dict(B=8, L=8192), "randn")}
FUZZ = [(dict(B=1, L=1), "randn"), (dict(B=3, L=77), "randn"), (dict(B=2, L=4097), "randn"),
        (dict(B=1, L=65536), "randn"), (dict(B=5, L=300), "large"), (dict(B=2, L=3000), "needle"),
        (dict(B=2, L=3000), "nan_inf"), (dict(B=2, L=3000), "tiny"), (dict(B=4, L=1000, Hq=8, Hkv=8), "randn"),
        (dict(B=2, L=2048, Hq=64, Hkv=2), "randn"), (dict(B=7, L=33), "randn"), (dict(B=1, L=31), "large")]
L3_CASES = [(dict(B=2, L=8192), "randn"), (dict(B=1, L=32768), "randn"), (dict(B=4, L=4096), "large"),
            (dict(B=2, L=8192), "needle"), (dict(B=8, L=2048), "randn")]
# This build's ragged extension: lens ~ U[L_min, L].
EXTRA = [(dict(B=6, L=5000, L_min=1), "randn"), (dict(B=8, L=2048, L_min=1), "needle"),
         (dict(B=3, L=40000, L_min=30000), "randn"), (dict(B=4, L=5000, L_min=1, dtype="bf16"), "randn")]
# Row invariance (L4): every request decoded alone (B = 1) must give the same bits as in the batch.
L4_CASES = [(dict(B=8, L=8192), "randn"), (dict(B=6, L=5000, L_min=1), "randn"), (dict(B=4, L=16384), "needle")]


def row_inputs(inp, i):
    """Request i alone."""
    return {k: (x[i:i + 1] if x is not None else None) for k, x in inp.items()}


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """Seeded inputs, in the other ops' style: q, k, v as float32 standard normals, then the lengths (when
    shape["L_min"] is given), then the dist recipe, then an fp16 cast on the host."""
    rng = np.random.default_rng(seed)
    B, L = shape["B"], shape["L"]
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    q = rng.standard_normal((B, Hq, d), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, L, d), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, L, d), dtype=np.float32)
    lens = rng.integers(shape["L_min"], L + 1, (B,)).astype(np.int32) if "L_min" in shape else None
    G = Hq // Hkv
    if dist == "large":
        q, k = q * 8.0, k * 8.0
    elif dist == "needle":            # one dominant key per (request, KV head), inside the positions in use
        for b in range(B):
            n = L if lens is None else int(lens[b])
            for h in range(Hkv):
                j = int(rng.integers(0, n))
                k[b, h, j] = q[b, h * G:(h + 1) * G].mean(0) * 6.0
                v[b, h, j] += 3.0
    elif dist == "nan_inf":
        k[0, 0, L // 2, 3] = np.nan
        v[B - 1, Hkv - 1, L // 3, 7] = np.inf
    elif dist == "tiny":
        q, k, v = q * 1e-4, k * 1e-4, v * 1e-6
    elif dist != "randn":
        raise ValueError(f"unknown dist {dist!r}")
    f = lambda a: cast16(a, shape.get("dtype", "fp16"), device)
    return dict(q=f(q), k=f(k), v=f(v), lens=None if lens is None else torch.from_numpy(lens).to(device))


def valid_mask(L, lens, device):
    """(B, 1, 1, L) bool: the first lens[b] positions (None when every position is in use)."""
    if lens is None:
        return None
    n = lens.to(device).long().clamp(1, L)
    return (torch.arange(L, device=device)[None, :] < n[:, None])[:, None, None, :]


# ---------------------------------------------------------------- PyTorch standard op
def torch_sdpa(q, k, v, lens=None, **_):
    import torch.nn.functional as F
    m = valid_mask(k.shape[2], lens, q.device)
    return F.scaled_dot_product_attention(q[:, :, None, :], k, v, attn_mask=m, enable_gqa=True)[:, :, 0, :]


TORCH_REFS = dict(torch_sdpa=torch_sdpa)
L1_REF = "torch_sdpa"
L3_REF = "torch_sdpa"


def used(shape, lens=None):
    B, L = shape["B"], shape["L"]
    return B * L if lens is None else int(np.clip(np.asarray(lens), 1, L).sum())


def algorithmic_bytes(shape, lens=None):
    """Bytes an ideal kernel moves: q + the K/V rows in use + the fp16 output."""
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    B = shape["B"]
    return 2 * B * Hq * d * 2 + used(shape, lens) * Hkv * d * 2 * 2


def flops(shape, lens=None):
    Hq, d = shape.get("Hq", HQ), shape.get("D", D)
    return 4.0 * used(shape, lens) * Hq * d


def softmax_scale(d=D):
    return 1.0 / math.sqrt(d)
