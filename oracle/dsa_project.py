"""Float64 oracle of the DSA projections (test infrastructure only; see oracle/__init__.py).

The reference leaves the projections that produce its DSA op's inputs outside the op (ops/dsa.py:8-9, "as in
llama.cpp's LIGHTNING_INDEXER + TOP_K + FLASH_ATTN_EXT decomposition"); this build defines them after
DeepSeek-V3.2's published attention block for one new token per request (MLA in absorbed form plus the lightning
indexer), with the shapes the op consumes (ops/dsa.py:7: q (B,128,576), iq (B,64,128), w (B,64), kv rows of 576,
ik rows of 128) and its softmax scale 1/sqrt(128 + 64) (ops/dsa.py:17) implied by q's 128 + 64 dims.

Per request b, hidden state x (7168), position p:
  cq  = rmsnorm(x Wq_a^T) * q_norm                   (1536), rounded to the 16-bit input type
  q_h = cq Wq_b^T, head h = [nope (128) | pe (64)]   (128 heads x 192)
  q   = [round16(nope_h) W_uk[h]^T (512) | rope(pe_h, p) (64)]      W_uk given as (128, 512, 128): [h][c][d]
  kv row p = [rmsnorm(kv_c) * kv_norm (512) | rope(k_pe, p) (64)],  [kv_c | k_pe] = x Wkv_a^T
  iq_j = cq Wiq_b^T, head j = [rope_half(pe_j, p) (64) | nope_j (64)]   (64 heads x 128)
  ik row p = layernorm(x Wik^T) * ik_w + ik_b, then rope_half on its first 64 dims
  w   = (x Wiw^T) * 64^-1/2 * 128^-1/2                 (the op's "pre-scaled" w, ops/dsa.py:7, 28)
RMSNorm and LayerNorm use eps = 1e-6.  MLA's RoPE (q's and the kv row's rope parts) rotates interleaved pairs
(x[2i], x[2i+1]) by the table row p: (x0 c - x1 s, x0 s + x1 c) with c = cos[p, i], s = sin[p, i].  The indexer's
RoPE (iq's and the ik row's first 64 dims) is not interleaved: it rotates the pairs (x[i], x[i+32]) by the same
entries, as DeepSeek-V3.2's inference code applies it in the indexer (apply_rotary_emb with interleaved=False).  DeepSeek's indexer also applies a Hadamard rotation
to iq and ik before quantising them to fp8; the rotation is orthonormal, so it leaves every iq . ik product (and the
op's scores) unchanged, and this fp16/bf16 contract has no quantisation, so it is left out.
"""
import numpy as np

from .common import to64, toint

DIM, QL, H, DN, DR, DC, HI, DI = 7168, 1536, 128, 128, 64, 512, 64, 128
EPS = 1e-6


def round16(a, dtype):
    """Round float64 values to the 16-bit type (fp16 or bf16, round to nearest even) and back to float64."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))
    return t.to(torch.bfloat16 if dtype == "bf16" else torch.float16).to(torch.float64).numpy()


def rmsnorm(v, weight, eps=EPS):
    """v / sqrt(mean(v^2) + eps) * weight over the last axis."""
    return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps) * weight


def layernorm(v, weight, bias, eps=EPS):
    """(v - mean) / sqrt(var + eps) * weight + bias over the last axis (biased variance)."""
    m = v.mean(axis=-1, keepdims=True)
    var = ((v - m) ** 2).mean(axis=-1, keepdims=True)
    return (v - m) / np.sqrt(var + eps) * weight + bias


def rope(v, c, s):
    """Rotate the interleaved pairs of v (..., 2n) by per-pair cos/sin c, s (..., n)."""
    x0, x1 = v[..., 0::2], v[..., 1::2]
    out = np.empty_like(v)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def rope_half(v, c, s):
    """Rotate the pairs (v[i], v[i + n]) of v (..., 2n), the two halves, by per-pair cos/sin c, s (..., n)."""
    n = v.shape[-1] // 2
    x0, x1 = v[..., :n], v[..., n:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


W_SCALE = HI ** -0.5 * DI ** -0.5


def split_q(yq):
    """MLA head of 192 from Wq_b's rows: (nope (128), pe (64))."""
    return yq[..., :DN], yq[..., DN:]


def split_iq(yi):
    """Indexer head of 128 from Wiq_b's rows: (pe (64), nope (64))."""
    return yi[..., :DR], yi[..., DR:]


def absorb(nope, w_uk):
    """q_lat[b, h, c] = sum_d nope[b, h, d] W_uk[h][c][d]: the nope query through the key half of Wkv_b."""
    return np.einsum("bhd,hcd->bhc", nope, w_uk)


def ref64(x, pos, cos, sin, wq_a, q_norm, wq_b, w_uk, wkv_a, kv_norm, iwq_b, iwk, ik_norm_w, ik_norm_b, iw,
          dtype="fp16"):
    """Returns dict(q (B,128,576), iq (B,64,128), w (B,64), kv_row (B,576), ik_row (B,128)) in float64.  The
    positions index the RoPE tables (clamped into them); the 16-bit roundings of cq and of q's nope part are the
    op's own (its second and absorbed products take 16-bit operands)."""
    x = to64(x)
    p = np.clip(toint(pos).astype(np.int64), 0, len(cos) - 1)
    c, s = to64(cos)[p], to64(sin)[p]                                    # (B, 32)
    cq = round16(rmsnorm(x @ to64(wq_a).T, to64(q_norm)), dtype)
    nope, pe = split_q((cq @ to64(wq_b).T).reshape(-1, H, DN + DR))
    q = np.concatenate([absorb(round16(nope, dtype), to64(w_uk)), rope(pe, c[:, None], s[:, None])], axis=-1)
    kvx = x @ to64(wkv_a).T
    kv_row = np.concatenate([rmsnorm(kvx[:, :DC], to64(kv_norm)), rope(kvx[:, DC:], c, s)], axis=-1)
    ipe, inope = split_iq((cq @ to64(iwq_b).T).reshape(-1, HI, DI))
    iq = np.concatenate([rope_half(ipe, c[:, None], s[:, None]), inope], axis=-1)
    ikv = layernorm(x @ to64(iwk).T, to64(ik_norm_w), to64(ik_norm_b))
    ik_row = np.concatenate([rope_half(ikv[:, :DR], c, s), ikv[:, DR:]], axis=-1)
    w = (x @ to64(iw).T) * W_SCALE
    return dict(q=q, iq=iq, w=w, kv_row=kv_row, ik_row=ik_row)
