"""Shared-prefix decode: the op contract (shapes, case lists, input generator, PyTorch standard ops).

N requests share a P-token prefix; request n also owns an S_n-token suffix and issues one decode token.
    q: (N, Hq, D)   kp, vp: (Hkv, P, D)   ks, vs: (N, Hkv, S, D)   slens: (N,) int32 or None   -> out (N, Hq, D) fp16
With `slens`, request n attends to its first slens[n] suffix rows only (ks/vs are padded to S = max slens);
`slens=None` means every request uses all S rows, which is the reference contract (ops/prefix.py:1-4, 15-44).

The float64 reference lives in the repo's `oracle/` package (test infrastructure); this module is what both the
kernel side and the verifier share.
"""
import math

import numpy as np
import torch

from .elem import cast16

NAME = "prefix"
HQ, HKV, D = 32, 8, 128                                  # ops/prefix.py:10
L1_SHAPE = dict(N=4, P=2048, S=256)                      # ops/prefix.py:11
BENCH_SHAPES = [dict(N=8, P=8192, S=512), dict(N=16, P=16384, S=1024), dict(N=32, P=4096, S=256)]  # :12
# Headline configurations of this build (BASELINE C1, C2).  S_min turns on ragged suffixes U[S_min, S].
CONFIGS = {"C1": (dict(N=8, P=2048, S=256), "randn"),
           "C2": (dict(N=64, P=16384, S=2048, S_min=128), "outlier"),
           "C2b": (dict(N=64, P=16384, S=2048, S_min=128, dtype="bf16"), "outlier")}   # C2 with bf16 inputs


def make_inputs(shape, seed=0, dist="randn", with_ref_layouts=False, device="cpu"):
    """Seeded inputs with the reference's draw order (ops/prefix.py:15-44): q, kp, vp, ks, vs as float32 standard
    normals, then the dist recipe, then an fp16 cast on the host.

    Extensions, drawn only after every reference draw so the reference cases are unchanged:
      * shape["S_min"]: ragged suffix lengths slens ~ U[S_min, S] (int32), drawn right after vs;
      * dist "outlier": 1 % of the entries of kp and ks (a fresh uniform draw each) scaled x20.
    """
    rng = np.random.default_rng(seed)
    N, P, S = shape["N"], shape["P"], shape["S"]
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    q = rng.standard_normal((N, Hq, d), dtype=np.float32)
    kp = rng.standard_normal((Hkv, P, d), dtype=np.float32)
    vp = rng.standard_normal((Hkv, P, d), dtype=np.float32)
    ks = rng.standard_normal((N, Hkv, S, d), dtype=np.float32)
    vs = rng.standard_normal((N, Hkv, S, d), dtype=np.float32)
    slens = None
    if "S_min" in shape:
        slens = rng.integers(shape["S_min"], S + 1, (N,)).astype(np.int32)
    G = Hq // Hkv
    if dist == "large":
        q, kp, ks = q * 8, kp * 8, ks * 8
    elif dist == "needle_prefix":
        for h in range(Hkv):
            kp[h, rng.integers(0, P)] = q[:, h * G:(h + 1) * G].mean((0, 1)) * 6.0
    elif dist == "needle_suffix":
        for n in range(N):
            for h in range(Hkv):
                ks[n, h, rng.integers(0, S)] = q[n, h * G:(h + 1) * G].mean(0) * 6.0
                vs[n, h] += 3.0
    elif dist == "nan_inf":
        ks[N - 1, 0, S - 1, 0] = np.nan
        vp[1, P // 2, 7] = np.inf
    elif dist == "tiny":
        q, kp, vp, ks, vs = q * 1e-4, kp * 1e-4, vp * 1e-6, ks * 1e-4, vs * 1e-6
    elif dist == "outlier":
        kp[rng.random(kp.shape) < 0.01] *= 20.0
        ks[rng.random(ks.shape) < 0.01] *= 20.0
    elif dist != "randn":
        raise ValueError(f"unknown dist {dist!r}")
    f = lambda a: cast16(a, shape.get("dtype", "fp16"), device)
    out = dict(q=f(q), kp=f(kp), vp=f(vp), ks=f(ks), vs=f(vs),
               slens=None if slens is None else torch.from_numpy(slens).to(device))
    if with_ref_layouts:
        out.update(build_layouts(out["kp"], out["vp"], out["ks"], out["vs"]))
    return out


def build_layouts(kp, vp, ks, vs):
    """Per-request full cache kf/vf (N, Hkv, P+S, D) with the prefix broadcast, and the unified cache
    ku/vu (1, Hkv, P+N*S, D) (ops/prefix.py:47-54).  Used by the standard ops only."""
    N = ks.shape[0]
    kf = torch.cat([kp[None].expand((N,) + tuple(kp.shape)), ks], dim=2)
    vf = torch.cat([vp[None].expand((N,) + tuple(vp.shape)), vs], dim=2)
    ku = torch.cat([kp] + [ks[n] for n in range(N)], dim=1)[None]
    vu = torch.cat([vp] + [vs[n] for n in range(N)], dim=1)[None]
    return dict(kf=kf, vf=vf, ku=ku, vu=vu)


def valid_mask(P, S, slens, device):
    """(N, 1, 1, P+S) bool: every prefix position plus the first slens[n] suffix rows (None when not ragged)."""
    if slens is None:
        return None
    c = torch.arange(P + S, device=device)[None, :]
    return (c < P + slens.to(device).long()[:, None])[:, None, None, :]


# ---------------------------------------------------------------- PyTorch standard ops (ops/prefix.py:121-138)
def torch_naive(q, kf=None, vf=None, kp=None, vp=None, ks=None, vs=None, slens=None, **_):
    """Non-sharing engine: every request reads the whole prefix (ops/prefix.py:121-123).  Builds kf/vf when they
    are not supplied; ragged suffixes are masked."""
    import torch.nn.functional as F
    if kf is None:
        lay = build_layouts(kp, vp, ks, vs)
        kf, vf = lay["kf"], lay["vf"]
    P = kf.shape[2] - (ks.shape[2] if ks is not None else 0)
    m = None if slens is None else valid_mask(P, ks.shape[2], slens, q.device)
    return F.scaled_dot_product_attention(q[:, :, None, :], kf, vf, attn_mask=m, enable_gqa=True)[:, :, 0, :]


def torch_unified(q, ku=None, vu=None, kp=None, vp=None, ks=None, vs=None, slens=None, **_):
    """Unified cache plus a per-request mask: prefix read once per KV head, N*G rows (ops/prefix.py:126-138)."""
    import torch.nn.functional as F
    if ku is None:
        lay = build_layouts(kp, vp, ks, vs)
        ku, vu = lay["ku"], lay["vu"]
    N, Hq, d = q.shape
    Hkv = ku.shape[1]
    G = Hq // Hkv
    S = ks.shape[2]
    P = ku.shape[2] - N * S
    r = torch.arange(N * G, device=q.device)[:, None] // G
    c = torch.arange(P + N * S, device=q.device)[None, :]
    sl = S if slens is None else slens.to(q.device).long().repeat_interleave(G)[:, None]
    m = (c < P) | ((c >= P + r * S) & (c < P + r * S + sl))
    qf = q.reshape(N, Hkv, G, d).permute(1, 0, 2, 3).reshape(1, Hkv, N * G, d)
    o = F.scaled_dot_product_attention(qf, ku, vu, attn_mask=m)
    return o.reshape(Hkv, N, G, d).permute(1, 0, 2, 3).reshape(N, Hq, d)


TORCH_REFS = dict(torch_naive=torch_naive, torch_unified=torch_unified)

L1_REF = "torch_naive"          # the reference's L1/L3 standard op is mlx_naive (ops/prefix.py:145-146)
L3_REF = "torch_naive"
FUZZ = [(dict(N=1, P=1, S=1), "randn"), (dict(N=3, P=1000, S=77), "randn"), (dict(N=5, P=4097, S=33), "randn"),
        (dict(N=2, P=65536, S=4096), "randn"), (dict(N=33, P=300, S=10), "randn"), (dict(N=64, P=2048, S=64), "randn"),
        (dict(N=4, P=3000, S=200), "large"), (dict(N=4, P=3000, S=200), "needle_prefix"),
        (dict(N=4, P=3000, S=200), "needle_suffix"), (dict(N=4, P=3000, S=200), "nan_inf"),
        (dict(N=4, P=3000, S=200), "tiny"), (dict(N=7, P=8, S=1), "randn")]          # ops/prefix.py:147-151
L3_CASES = [(dict(N=8, P=1024, S=128), "randn"), (dict(N=8, P=32768, S=1024), "randn"),
            (dict(N=4, P=8192, S=512), "large"), (dict(N=4, P=8192, S=512), "needle_prefix"),
            (dict(N=4, P=8192, S=512), "needle_suffix")]                                # ops/prefix.py:152-153
# Cases this build adds for its own extensions (ragged suffixes, K outliers); judged like L2.
EXTRA = [(dict(N=5, P=700, S=300, S_min=1), "randn"), (dict(N=16, P=2048, S=512, S_min=128), "outlier"),
         (dict(N=3, P=1, S=64, S_min=1), "randn"), (dict(N=8, P=2048, S=256, S_min=1, dtype="bf16"), "randn"),
         (dict(N=64, P=4096, S=512, S_min=128, dtype="bf16"), "outlier")]
# Row invariance (L4, ONE-PAGER.md:13-14): every request computed alone (N = 1) must give the same bits as in the
# batch.  The C2 and C1 shapes, a prefix of many chunks with suffixes split over two chunks, and odd sizes.
L4_CASES = [(dict(N=64, P=16384, S=2048, S_min=128), "outlier"), (dict(N=8, P=2048, S=256), "randn"),
            (dict(N=20, P=40000, S=3000, S_min=1), "randn"), (dict(N=33, P=300, S=10), "randn"),
            # 64-key prefix chunks: the batch runs eight-wave row blocks, each request alone single-wave units
            (dict(N=64, P=2048, S=256), "randn")]


def row_inputs(inp, i):
    """Request i alone: its query, suffix rows and length, with the shared prefix unchanged."""
    out = dict(inp)
    for k in ("q", "ks", "vs", "slens"):
        if inp.get(k) is not None:
            out[k] = inp[k][i:i + 1]
    return out


def algorithmic_bytes(shape, slens=None):
    """Bytes an ideal kernel moves: q + prefix K/V + the used suffix K/V rows + the fp16 output."""
    N, P, S = shape["N"], shape["P"], shape["S"]
    Hq, Hkv, d = shape.get("Hq", HQ), shape.get("Hkv", HKV), shape.get("D", D)
    sum_s = N * S if slens is None else int(np.asarray(slens).astype(np.int64).sum())
    return 2 * N * Hq * d * 2 + 2 * Hkv * P * d * 2 + 2 * Hkv * sum_s * d * 2


def flops(shape, slens=None):
    N, P, S = shape["N"], shape["P"], shape["S"]
    Hq, d = shape.get("Hq", HQ), shape.get("D", D)
    sum_s = N * S if slens is None else int(np.asarray(slens).astype(np.int64).sum())
    return 4 * Hq * d * (N * P + sum_s)


def scale(d=D):
    return 1.0 / math.sqrt(d)
