"""DSA projections: the per-token products that make the DSA decode op's inputs (this build's neighbour of the
reference's DSA op, which leaves them outside the op: ops/dsa.py:8-9).

For one new token per request, DeepSeek-V3.2 dimensions (hidden 7168, q LoRA rank 1536, 128 MLA heads of 128 + 64,
latent 512, 64 indexer heads of 128): from the hidden state x (B, 7168) and the token positions pos (B,), compute
the op's q (B,128,576), iq (B,64,128), w (B,64) and write the new kv (576) and ik (128) cache rows at pos.  The
formulas are in include/vmk.h (vmk_dsa_project) and oracle/dsa_project.py.  Weights are random here (there is no
checkpoint): N(0, 1/fan_in) matrices, so every product has O(1) entries, and norm weights around 1.
"""
import numpy as np
import torch

from .elem import cast16

NAME = "dsa_project"
DIM, QL, H, DN, DR, DC, HI, DI = 7168, 1536, 128, 128, 64, 512, 64, 128
EPS = 1e-6
WEIGHT_SHAPES = dict(wq_a=(QL, DIM), q_norm=(QL,), wq_b=(H * (DN + DR), QL), w_uk=(H, DC, DN), wkv_a=(DC + DR, DIM),
                     kv_norm=(DC,), iwq_b=(HI * DI, QL), iwk=(DI, DIM), ik_norm_w=(DI,), ik_norm_b=(DI,),
                     iw=(HI, DIM))
NORMS = ("q_norm", "kv_norm", "ik_norm_w", "ik_norm_b")                # fp32; the matrices are 16-bit
# The benchmark line: a decode step of 4 requests (the C5 batch) over 65536-row caches.
CONFIGS = {"DP": (dict(B=4, L=65536), "randn")}


def make_weights(seed=0, dtype="fp16", device="cpu"):
    """Seeded random weights in the layout of vmk_dsa_project_weights (include/vmk.h)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in WEIGHT_SHAPES.items():
        if name in NORMS:
            base = 0.0 if name == "ik_norm_b" else 1.0
            out[name] = torch.from_numpy(base + 0.1 * rng.standard_normal(shape, dtype=np.float32)).to(device)
        else:
            fan_in = shape[-1]
            a = rng.standard_normal(shape, dtype=np.float32) * np.float32(fan_in ** -0.5)
            out[name] = cast16(a, dtype, device)
    return out


def rope_tables(rows, base=10000.0):
    """Standard RoPE tables (rows, 32): angle p * base^(-2i/64) for pair i (the op takes any table)."""
    inv = base ** (-np.arange(0, DR, 2, dtype=np.float64) / DR)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    return torch.from_numpy(np.cos(ang).astype(np.float32)), torch.from_numpy(np.sin(ang).astype(np.float32))


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """x (B, 7168), pos (B,) in [0, L), RoPE tables of L rows, zeroed kv (B, L, 576) / ik (B, L, 128) caches and the
    weights (seed + 1).  `dist` must be "randn" (the only input distribution)."""
    if dist != "randn":
        raise ValueError(f"unknown dist {dist!r}")
    rng = np.random.default_rng(seed)
    B, L = shape["B"], shape["L"]
    dtype = shape.get("dtype", "fp16")
    x = cast16(rng.standard_normal((B, DIM), dtype=np.float32), dtype, device)
    pos = torch.from_numpy(rng.integers(0, L, (B,)).astype(np.int32)).to(device)
    cos, sin = rope_tables(L)
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    return dict(x=x, pos=pos, rope_cos=cos.to(device), rope_sin=sin.to(device),
                kv=torch.zeros(B, L, DC + DR, dtype=dt, device=device),
                ik=torch.zeros(B, L, DI, dtype=dt, device=device),
                weights=make_weights(seed + 1, dtype, device))


def _rms(v, w):
    return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + EPS) * w


def _rope(v, c, s):
    x0, x1 = v[..., 0::2], v[..., 1::2]
    return torch.stack([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1).flatten(-2)


def _rope_half(v, c, s):
    n = v.shape[-1] // 2
    x0, x1 = v[..., :n], v[..., n:]
    return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1)


def torch_ref(x, pos, rope_cos, rope_sin, weights, kv=None, ik=None):
    """The projections as PyTorch ops, the standard op the benchmark times against: the products in x's 16-bit type
    (F.linear, fp32 accumulation), norms and RoPE in float32, the absorbed product as one batched matmul over the
    heads.  Returns q, iq, w, kv_row, ik_row."""
    W = weights
    dt = x.dtype
    lin = torch.nn.functional.linear
    p = pos.long().clamp(0, rope_cos.shape[0] - 1)
    c, s = rope_cos[p], rope_sin[p]
    cq = _rms(lin(x, W["wq_a"]).float(), W["q_norm"]).to(dt)
    yq = lin(cq, W["wq_b"]).view(-1, H, DN + DR)
    nope_t = yq[..., :DN].permute(1, 2, 0).contiguous()                      # (H, DN, B)
    q_lat = torch.bmm(W["w_uk"], nope_t).permute(2, 0, 1)                   # (B, H, DC)
    q = torch.cat([q_lat.float(), _rope(yq[..., DN:].float(), c[:, None], s[:, None])], -1)
    kvx = lin(x, W["wkv_a"]).float()
    kv_row = torch.cat([_rms(kvx[:, :DC], W["kv_norm"]), _rope(kvx[:, DC:], c, s)], -1)
    yi = lin(cq, W["iwq_b"]).view(-1, HI, DI).float()
    iq = torch.cat([_rope_half(yi[..., :DR], c[:, None], s[:, None]), yi[..., DR:]], -1)
    ikv = torch.nn.functional.layer_norm(lin(x, W["iwk"]).float(), (DI,), W["ik_norm_w"], W["ik_norm_b"], EPS)
    ik_row = torch.cat([_rope_half(ikv[:, :DR], c, s), ikv[:, DR:]], -1)
    w = lin(x, W["iw"]).float() * (HI ** -0.5 * DI ** -0.5)
    return q.to(dt), iq.to(dt), w, kv_row.to(dt), ik_row.to(dt)


TORCH_REFS = dict(torch_ref=torch_ref)


def weight_bytes(dtype="fp16"):
    """Bytes of every weight the op reads once per call (the matrices 2 bytes per element, norms 4)."""
    return sum(int(np.prod(s)) * (4 if n in NORMS else 2) for n, s in WEIGHT_SHAPES.items())


def algorithmic_bytes(shape):
    """Weights once, plus the tokens' inputs and outputs: x, pos, q, iq, w, the two cache rows."""
    B = shape["B"]
    return weight_bytes() + B * (DIM * 2 + 4 + H * (DC + DR) * 2 + HI * DI * 2 + HI * 4 + (DC + DR) * 2 + DI * 2)


def flops(shape):
    """Multiply-adds of the five products (2 flops each)."""
    B = shape["B"]
    macs = DIM * (QL + DC + DR + DI + HI) + QL * (H * (DN + DR) + HI * DI) + H * DN * DC
    return 2 * B * macs
