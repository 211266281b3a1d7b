"""DeepSeek Sparse Attention (DSA) decode: the op contract (shapes, case lists, input generator, PyTorch standard ops).

Per request b (one new token), DeepSeek-V3.2 shapes (ops/dsa.py:1-9):
  indexer: score[l] = sum_h w[h] * relu(iq[h] . ik[l])      (64 indexer heads x 128)
  select : idx = top-2048(score) over the valid positions (all of them when there are <= 2048)
  attend : absorbed MLA, 128 query heads over 576-dim latent rows (512 latent + 64 rope):
           out = softmax(q . kv[idx]^T * scale) @ kv[idx][:, :512],  scale = 1/sqrt(192)
Shapes: q (B,128,576) fp16, kv (B,L,576) fp16, iq (B,64,128) fp16, ik (B,L,128) fp16, w (B,64) fp32,
lens (B,) int32 or None  ->  out (B,128,512) fp16.  q, kv, iq, ik may all be bf16 instead (out is then bf16).
"""
import math

import numpy as np
import torch

from .elem import cast16

NAME = "dsa"
H, DC, DR, HI, DI, TOPK = 128, 512, 64, 64, 128, 2048          # ops/dsa.py:15
DK = DC + DR
SCALE = 1.0 / math.sqrt(128 + 64)                              # ops/dsa.py:17
L1_SHAPE = dict(B=2, L=8192)                                   # ops/dsa.py:18
BENCH_SHAPES = [dict(B=1, L=8192), dict(B=1, L=32768), dict(B=1, L=65536), dict(B=4, L=16384)]
CONFIGS = {"C5": (dict(B=4, L=65536), "randn")}                # BASELINE C5


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """Seeded inputs with the reference's draw order (ops/dsa.py:22-50): q, kv, iq, ik, w (scaled by
    HI^-1/2 * DI^-1/2), then the dist recipe; fp16 (or shape["dtype"] = "bf16") cast on the host, w stays float32, lens int32 or None."""
    rng = np.random.default_rng(seed)
    B, L = shape["B"], shape["L"]
    q = rng.standard_normal((B, H, DK), dtype=np.float32)
    kv = rng.standard_normal((B, L, DK), dtype=np.float32)
    iq = rng.standard_normal((B, HI, DI), dtype=np.float32)
    ik = rng.standard_normal((B, L, DI), dtype=np.float32)
    w = rng.standard_normal((B, HI), dtype=np.float32) * (HI ** -0.5 * DI ** -0.5)
    lens = None
    if dist == "large":
        q, kv = q * 6.0, kv * 6.0
    elif dist == "needle":  # one strongly-indexed position per request, also dominant in attention
        for b in range(B):
            p = rng.integers(0, L)
            ik[b, p] = (iq[b] * np.sign(w[b])[:, None]).mean(0) * 8.0
            kv[b, p, :] = q[b].mean(0) * 4.0
            kv[b, p, :DC] += 5.0
    elif dist == "ragged":
        lens = rng.integers(1, L + 1, (B,)).astype(np.int32)
        lens[0] = min(L, 1000)
        if B > 1:
            lens[1] = L
    elif dist == "nan_inf":
        kv[0, L // 2, 3] = np.nan  # may or may not be selected -> pattern must match the fp64 reference
    elif dist == "tiny":
        q, kv = q * 1e-3, kv * 1e-3
    elif dist != "randn":
        raise ValueError(f"unknown dist {dist!r}")
    f = lambda a: cast16(a, shape.get("dtype", "fp16"), device)
    return dict(q=f(q), kv=f(kv), iq=f(iq), ik=f(ik), w=torch.from_numpy(w).to(device),
                lens=None if lens is None else torch.from_numpy(lens).to(device))


# ---------------------------------------------------------------- PyTorch standard op (ops/dsa.py:116-134)
def torch_ref(q, kv, iq, ik, w, lens=None):
    """Indexer GEMM in the input dtype, ReLU, fp32 head-weighted sum, masked top-k, gather, SDPA."""
    import torch.nn.functional as F
    B, L = kv.shape[0], kv.shape[1]
    s = torch.relu(torch.matmul(iq, ik.transpose(1, 2).contiguous()))      # (B, HI, L)
    s = (s.float() * w[:, :, None]).sum(1)                                 # (B, L)
    if lens is not None:
        s = s.masked_fill(torch.arange(L, device=s.device)[None, :] >= lens[:, None], float("-inf"))
    m = None
    if L > TOPK:
        idx = torch.topk(s, TOPK, dim=-1).indices
        ks = torch.gather(kv, 1, idx[:, :, None].expand(-1, -1, DK))
        if lens is not None:
            m = (idx < lens[:, None])[:, None, None, :]
    else:
        ks = kv
        if lens is not None:
            m = (torch.arange(L, device=s.device)[None, :] < lens[:, None])[:, None, None, :]
    return F.scaled_dot_product_attention(q[:, :, None, :], ks[:, None], ks[:, None, :, :DC].contiguous(),
                                          attn_mask=m, scale=SCALE)[:, :, 0, :]


def torch_fp32_ref(q, kv, iq, ik, w, lens=None):
    """The same algorithm computed in float32, output cast to q's dtype (the L1 standard op, ops/dsa.py:150-153)."""
    f = lambda a: a.float()
    return torch_ref(f(q), f(kv), f(iq), f(ik), w, lens).to(q.dtype)


def chain_torch(out, kw):
    """Bench data dependency: next layer's absorbed query = [output (512) | this query's rope part (64)]
    (ops/dsa.py:145-147)."""
    return torch.cat([out, kw["q"][..., DC:]], dim=-1)


TORCH_REFS = dict(torch_ref=torch_ref)
L1_REF = "torch_fp32_ref"       # the reference's are mlx_fp32_ref / mlx_lm (ops/dsa.py:156-157)
L3_REF = "torch_ref"
FUZZ = [(dict(B=1, L=1), "randn"), (dict(B=1, L=2048), "randn"), (dict(B=1, L=2049), "randn"), (dict(B=2, L=5003), "randn"),
        (dict(B=1, L=131072), "randn"), (dict(B=3, L=9000), "ragged"), (dict(B=1, L=30), "randn"),
        (dict(B=2, L=6000), "large"), (dict(B=2, L=6000), "needle"), (dict(B=2, L=6000), "nan_inf"),
        (dict(B=2, L=6000), "tiny"), (dict(B=4, L=3000), "ragged")]                       # ops/dsa.py:158-161
L3_CASES = [(dict(B=1, L=1500), "randn"), (dict(B=1, L=8192), "randn"), (dict(B=1, L=65536), "randn"),
            (dict(B=2, L=8192), "large"), (dict(B=2, L=8192), "needle")]                  # ops/dsa.py:162-163
EXTRA = [(dict(B=5, L=4100), "ragged"), (dict(B=2, L=6000, dtype="bf16"), "randn"), (dict(B=65, L=2500), "randn")]
# Row invariance (L4): every request decoded alone (B = 1) must give the same bits as in the batch.
L4_CASES = [(dict(B=4, L=65536), "randn"), (dict(B=5, L=4100), "ragged"), (dict(B=3, L=2049), "randn")]


def row_inputs(inp, i):
    """Request i alone."""
    return {k: (x[i:i + 1] if x is not None else None) for k, x in inp.items()}


def algorithmic_bytes(shape, lens=None):
    """ik streamed once + only the selected kv rows + q, iq, w, fp16 output (the full kv cache is not counted)."""
    B, L = shape["B"], shape["L"]
    n = [L] * B if lens is None else [int(x) for x in np.asarray(lens)]
    sel = sum(min(x, TOPK) for x in n)
    return (sum(n) * DI * 2 + sel * DK * 2 + B * H * DK * 2 + B * HI * DI * 2 + B * HI * 4 + B * H * DC * 2)


def flops(shape, lens=None):
    B, L = shape["B"], shape["L"]
    n = [L] * B if lens is None else [int(x) for x in np.asarray(lens)]
    return sum(2 * HI * DI * x + 2 * H * min(x, TOPK) * (DK + DC) for x in n)
