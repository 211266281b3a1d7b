"""Speculative verification: the op contract (shapes, case lists, input generator, PyTorch standard ops).

kd draft tokens (a chain or a tree) are verified in one pass against a cache of L tokens whose last kd positions are
the drafts themselves (ops/spec.py:1-3).
    q: (B, kd, Hq, D)   k, v: (B, Hkv, L, D)   bits: (B, kd) int32, or (B, kd, W) int32 words when kd > 32
Bit j of draft i's mask (word j // 32, bit j % 32) says that draft i may attend draft j (its ancestors and itself).
The (B, kd) form is the reference contract; the word form is this build's extension for kd up to 64 and beyond.
"""
import math

import numpy as np
import torch

from .elem import cast16

NAME = "spec"
HQ, HKV, D = 32, 8, 128                                                   # ops/spec.py:8
L1_SHAPE = dict(B=2, L=4096, k=8)                                         # ops/spec.py:9
BENCH_SHAPES = [dict(B=1, L=8192, k=8), dict(B=1, L=32768, k=8), dict(B=4, L=16384, k=4), dict(B=1, L=32768, k=16)]
# Headline configurations of this build (BASELINE C3, C4).  L counts the drafts, as in the reference.
CONFIGS = {"C3": (dict(B=4, L=32768, k=8), "chain"),
           "C4": (dict(B=2, L=65536, k=64), "tree_bd")}


def n_words(kd):
    return (kd + 31) // 32


def chain_bits(kd):
    """Draft i sees drafts 0..i (ops/spec.py:14-15); returned as (kd, W) uint32 words."""
    w = np.zeros((kd, n_words(kd)), dtype=np.uint64)
    for i in range(kd):
        for j in range(i + 1):
            w[i, j // 32] |= np.uint64(1) << np.uint64(j % 32)
    return w.astype(np.uint32)


def _bits_from_parents(par):
    kd = len(par)
    w = np.zeros((kd, n_words(kd)), dtype=np.uint32)
    for i in range(kd):
        w[i, i // 32] |= np.uint32(1 << (i % 32))
        if par[i] >= 0:
            w[i] |= w[par[i]]
    return w


def tree_bits(kd, rng):
    """Random tree: parent of node i uniform in [0, i) (ops/spec.py:18-25); (kd, W) uint32 words."""
    par = [-1] + [int(rng.integers(0, i)) for i in range(1, kd)]
    return _bits_from_parents(par)


def tree_bits_bounded(kd, rng, max_children=4, max_depth=8):
    """Random tree with at most `max_children` children per node and at most `max_depth` levels (root = level 1).
    Node i's parent is drawn uniformly among the nodes j < i that still have room, so parents precede children."""
    par, depth, nchild = [-1], [1], [0]
    for i in range(1, kd):
        cand = [j for j in range(i) if nchild[j] < max_children and depth[j] < max_depth]
        p = cand[int(rng.integers(0, len(cand)))]
        par.append(p)
        depth.append(depth[p] + 1)
        nchild.append(0)
        nchild[p] += 1
    return _bits_from_parents(par)


def words_to_int32(words, kd):
    """(B, kd, W) uint32 -> the reference's (B, kd) int32 when kd <= 32, else (B, kd, W) int32."""
    w = words.view(np.int32)
    return w[..., 0].copy() if kd <= 32 else w.copy()


def make_inputs(shape, seed=0, dist="randn", device="cpu"):
    """Seeded inputs with the reference's draw order (ops/spec.py:28-56): q, k, v, then the masks batch by batch
    (a tree draws kd-1 integers per batch; a chain draws nothing), then the dist recipe, then the fp16 cast.
    Extra dist "tree_bd": tree with branching <= 4 and depth <= 8 (this build's C4 configuration)."""
    rng = np.random.default_rng(seed)
    B, L, kd = shape["B"], shape["L"], shape["k"]
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    q = rng.standard_normal((B, kd, Hq, d), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, L, d), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, L, d), dtype=np.float32)
    if dist == "chain":
        words = np.stack([chain_bits(kd) for _ in range(B)])
    elif dist == "tree_bd":
        words = np.stack([tree_bits_bounded(kd, rng) for _ in range(B)])
    else:
        words = np.stack([tree_bits(kd, rng) for _ in range(B)])
    G = Hq // Hkv
    if dist == "large":
        q, k = q * 8.0, k * 8.0
    elif dist == "needle_masked":  # dominant key planted on a draft that row 0 must NOT see
        for b in range(B):
            j = kd - 1
            if (int(words[b, 0, j // 32]) >> (j % 32)) & 1 == 0:
                for h in range(Hkv):
                    k[b, h, L - kd + j] = q[b, 0, h * G:(h + 1) * G].mean(0) * 8.0
                    v[b, h, L - kd + j] += 50.0
    elif dist == "needle_boundary":  # dominant key just before the draft boundary
        for b in range(B):
            for h in range(Hkv):
                k[b, h, L - kd - 1] = q[b, :, h * G:(h + 1) * G].mean((0, 1)) * 6.0
    elif dist == "nan_inf":
        k[0, 0, L // 2, 3] = np.nan
    elif dist == "tiny":
        q, k, v = q * 1e-4, k * 1e-4, v * 1e-6
    elif dist not in ("randn", "chain", "tree_bd"):
        raise ValueError(f"unknown dist {dist!r}")
    f = lambda a: cast16(a, shape.get("dtype", "fp16"), device)
    return dict(q=f(q), k=f(k), v=f(v), bits=torch.from_numpy(words_to_int32(words, kd)).to(device))


def mask_words(bits, kd):
    """Any accepted `bits` layout -> (B, kd, W) int32 words."""
    if bits.dim() == 2:
        return bits.reshape(bits.shape[0], kd, 1)
    return bits


def draft_mask(bits, L, kd):
    """(B, kd, L) bool: every context position, then bit j of draft i's words for draft position L-kd+j
    (the torch form of ops/spec.py:277-282)."""
    w = mask_words(bits, kd).long() & 0xFFFFFFFF
    j = torch.arange(kd, device=bits.device)
    tail = ((w[:, :, j // 32] >> (j % 32)) & 1).bool()                          # (B, kd, kd)
    head = torch.ones(w.shape[0], kd, L - kd, dtype=torch.bool, device=bits.device)
    return torch.cat([head, tail], -1)


# ---------------------------------------------------------------- PyTorch standard ops (ops/spec.py:285-299)
def torch_sdpa(q, k, v, bits):
    import torch.nn.functional as F
    m = draft_mask(bits, k.shape[2], q.shape[1])[:, None]
    return F.scaled_dot_product_attention(q.transpose(1, 2), k, v, attn_mask=m, enable_gqa=True).transpose(1, 2)


def torch_sdpa_fold(q, k, v, bits):
    import torch.nn.functional as F
    B, kd, Hq, d = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qf = q.reshape(B, kd, Hkv, G, d).permute(0, 2, 1, 3, 4).reshape(B, Hkv, kd * G, d)
    m = draft_mask(bits, L, kd).repeat_interleave(G, dim=1)[:, None]
    o = F.scaled_dot_product_attention(qf, k, v, attn_mask=m)
    return o.reshape(B, Hkv, kd, G, d).permute(0, 2, 1, 3, 4).reshape(B, kd, Hq, d)


TORCH_REFS = dict(torch_sdpa=torch_sdpa, torch_sdpa_fold=torch_sdpa_fold)

L1_REF = "torch_sdpa"            # the reference's is mlx_sdpa (ops/spec.py:151-152)
L3_REF = "torch_sdpa"
FUZZ = [(dict(B=1, L=8, k=8), "randn"), (dict(B=1, L=9, k=1), "randn"), (dict(B=2, L=4097, k=8), "randn"),
        (dict(B=1, L=100000, k=16), "randn"), (dict(B=3, L=777, k=5), "randn"), (dict(B=1, L=4096, k=31), "randn"),
        (dict(B=2, L=3000, k=8), "chain"), (dict(B=2, L=3000, k=8), "large"), (dict(B=2, L=3000, k=8), "needle_masked"),
        (dict(B=2, L=3000, k=8), "needle_boundary"), (dict(B=2, L=3000, k=8), "nan_inf"), (dict(B=2, L=3000, k=8), "tiny"),
        (dict(B=8, L=2049, k=4), "randn"), (dict(B=1, L=31, k=31), "needle_masked")]     # ops/spec.py:153-157
L3_CASES = [(dict(B=1, L=1024, k=8), "randn"), (dict(B=1, L=32768, k=8), "randn"), (dict(B=1, L=65536, k=16), "randn"),
            (dict(B=2, L=8192, k=8), "large"), (dict(B=2, L=8192, k=8), "needle_boundary")]  # ops/spec.py:158-159
# Cases this build adds for kd > 32 (multi-word masks) and the bounded tree; judged like L2.
EXTRA = [(dict(B=2, L=4096, k=64), "tree_bd"), (dict(B=1, L=70, k=64), "needle_masked"),
         (dict(B=1, L=5000, k=33), "randn"), (dict(B=2, L=3000, k=64), "chain"),
         (dict(B=2, L=4096, k=8, dtype="bf16"), "chain"), (dict(B=1, L=3000, k=64, dtype="bf16"), "tree_bd")]
# Row invariance (L4): every batch entry verified alone (B = 1) must give the same bits as in the batch.
L4_CASES = [(dict(B=4, L=32768, k=8), "chain"), (dict(B=2, L=65536, k=64), "tree_bd"),
            (dict(B=3, L=5000, k=5), "randn"), (dict(B=5, L=777, k=33), "randn")]


def row_inputs(inp, i):
    """Batch entry i alone."""
    return {k: (x[i:i + 1] if x is not None else None) for k, x in inp.items()}


def algorithmic_bytes(shape):
    B, L, kd = shape["B"], shape["L"], shape["k"]
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    return 2 * B * kd * Hq * d * 2 + 2 * B * Hkv * L * d * 2 + B * kd * n_words(kd) * 4


def flops(shape):
    B, L, kd = shape["B"], shape["L"], shape["k"]
    Hq, d = shape.get("Hq", HQ), shape.get("D", D)
    return 4 * B * kd * Hq * L * d


def scale(d=D):
    return 1.0 / math.sqrt(d)
