"""Pins the float64 oracle of the DSA projections (oracle/dsa_project.py) without the reference (which has none).

Independent checks: PyTorch's float64 rms_norm and layer_norm (library routines); both RoPE forms against complex
multiplication as DeepSeek-V3.2's apply_rotary_emb states them (MLA: the interleaved pairs viewed as complex
numbers; the indexer, interleaved=False: the 64 dims viewed as (2, 32), transposed into pairs, rotated, and the real
and imaginary parts written back as the two halves); two closed forms of the whole op (a zero hidden
state, where only the LayerNorm bias survives, and 0/1 selection weights, where every output is a known coordinate of
x, so the head layouts, the absorbed product's orientation, the normed and rotated slices and the w scale are all
fixed); and the scale structure (RMSNorm/LayerNorm outputs do not change when x doubles, the raw k_pe and w do).
Every check is also run against a planted mistake in the oracle and must reject it.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dsa_project as odp
from vmk.ops import dsa_project as op

H, DN, DR, DC, HI, DI, QL, DIM = odp.H, odp.DN, odp.DR, odp.DC, odp.HI, odp.DI, odp.QL, odp.DIM


def rope_complex(v, c, s):
    """Interleaved-pair RoPE as complex multiplication by c + i s: v (..., 2n), c and s (..., n)."""
    z = torch.view_as_complex(torch.from_numpy(np.ascontiguousarray(v, dtype=np.float64)).reshape(*v.shape[:-1], -1, 2))
    r = torch.complex(torch.from_numpy(np.asarray(c, np.float64)), torch.from_numpy(np.asarray(s, np.float64)))
    return torch.view_as_real(z * r).reshape(v.shape).numpy()


def rope_complex_halves(v, c, s):
    """Non-interleaved RoPE the way DeepSeek-V3.2 writes it: view (..., 2, n), transpose to (..., n, 2), rotate as
    complex numbers, then [real parts | imaginary parts]."""
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float64))
    n = v.shape[-1] // 2
    z = torch.view_as_complex(t.reshape(*v.shape[:-1], 2, n).transpose(-1, -2).contiguous())
    r = torch.complex(torch.from_numpy(np.asarray(c, np.float64)), torch.from_numpy(np.asarray(s, np.float64)))
    y = torch.view_as_real(z * r).reshape(v.shape)
    return torch.cat([y[..., 0::2], y[..., 1::2]], -1).numpy()


def tables(rows):
    theta = np.arange(rows, dtype=np.float64)[:, None] * 0.1 * np.arange(1, 33, dtype=np.float64)[None, :]
    return theta, np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


# ------------------------------------------------------------------------------------------------------- checks
def norms_vs_torch(o):
    rng = np.random.default_rng(0)
    v = rng.standard_normal((3, 512))
    wt, bias = 1 + 0.1 * rng.standard_normal(512), 0.1 * rng.standard_normal(512)
    t = lambda a: torch.from_numpy(a)
    rms = F.rms_norm(t(v), (512,), t(wt), eps=o.EPS).numpy()
    ln = F.layer_norm(t(v), (512,), t(wt), t(bias), eps=o.EPS).numpy()
    return np.allclose(o.rmsnorm(v, wt), rms, rtol=1e-12, atol=1e-12) and \
        np.allclose(o.layernorm(v, wt, bias), ln, rtol=1e-12, atol=1e-12)


def rope_vs_complex(o):
    rng = np.random.default_rng(1)
    v = rng.standard_normal((5, 64))
    theta = rng.uniform(-4, 4, (5, 32))
    c, s = np.cos(theta), np.sin(theta)
    return np.allclose(o.rope(v, c, s), rope_complex(v, c, s), atol=1e-12) and \
        np.allclose(o.rope_half(v, c, s), rope_complex_halves(v, c, s), atol=1e-12)


def rope_forms_differ(o):
    """A closed form that tells the two pairings apart: v = e_1 (the second dim) rotated by a quarter turn of pair 0
    and no turn elsewhere.  Interleaved pairs (v0, v1) give -e_0; halves leave e_1 in place (its pair is (v1, v33),
    not turned)."""
    v = np.zeros((1, 64))
    v[0, 1] = 1.0
    c, s = np.ones((1, 32)), np.zeros((1, 32))
    c[0, 0], s[0, 0] = 0.0, 1.0
    e0, e1 = np.eye(64)[0:1], np.eye(64)[1:2]
    return np.allclose(o.rope(v, c, s), -e0, atol=1e-15) and np.allclose(o.rope_half(v, c, s), e1, atol=1e-15)


_RANDOM = {}


def random_weights():
    """Full-size seeded weights (fp16), generated once."""
    if not _RANDOM:
        _RANDOM.update(op.make_weights(seed=3))
    return _RANDOM


def run(o, x, pos, weights, rows=64):
    _, cos, sin = tables(rows)
    return o.ref64(x, pos, cos, sin, **weights)


def zero_input(o):
    """x = 0: every product is 0, so q, iq, w and the kv row are 0 and the ik row is the LayerNorm bias (its first
    64 dims rotated)."""
    W = random_weights()
    pos = np.array([5, 17], dtype=np.int32)
    r = run(o, np.zeros((2, DIM), dtype=np.float32), pos, W)
    _, cos, sin = tables(64)
    bias = W["ik_norm_b"].double().numpy()
    want_ik = np.concatenate([rope_complex_halves(np.tile(bias[:DR], (2, 1)), cos[pos], sin[pos]),
                              np.tile(bias[DR:], (2, 1))], -1)
    zero = all(np.array_equal(r[k], np.zeros_like(r[k])) for k in ("q", "iq", "w", "kv_row"))
    return zero and np.allclose(r["ik_row"], want_ik, atol=1e-12)


def scale_structure(o):
    """x -> 2x: the RMSNorm/LayerNorm-fed outputs (q, iq, kv_c, ik) stay, k_pe and w double.  "Stay" allows 1e-3 of
    the output's magnitude: eps moves the normed values by ~1e-6, which can flip the fp16 rounding of a few cq and
    nope entries by one unit (measured: q 6.8e-4 of 4.8), far below the factor 2 a misplaced norm would give."""
    W = random_weights()
    x = np.random.default_rng(2).standard_normal((2, DIM)).astype(np.float16).astype(np.float32)
    pos = np.array([1, 40], dtype=np.int32)
    a, b = run(o, x, pos, W), run(o, 2 * x, pos, W)
    same = lambda u, v: np.abs(u - v).max() <= 1e-3 * max(1.0, np.abs(u).max())
    return (same(a["q"], b["q"]) and same(a["iq"], b["iq"]) and same(a["kv_row"][:, :DC], b["kv_row"][:, :DC])
            and same(a["ik_row"], b["ik_row"]) and np.allclose(2 * a["kv_row"][:, DC:], b["kv_row"][:, DC:])
            and np.allclose(2 * a["w"], b["w"]))


def selection_weights():
    """0/1 weights that copy coordinates: Wq_a takes x[:1536], Wkv_a x[1536:2112], Wik x[2112:2240], Wiw x[3000:3064];
    Wq_b row r takes cq[7 r mod 1536], Wiq_b row r takes cq[3 r mod 1536]; W_uk[h][c][d] = 1 for c = 4 d + h mod 4;
    q_norm, kv_norm and ik_norm_w are 1, ik_norm_b is 0.25."""
    f = np.float16
    wq_a = np.zeros((QL, DIM), f)
    wq_a[np.arange(QL), np.arange(QL)] = 1
    wq_b = np.zeros((H * (DN + DR), QL), f)
    r = np.arange(H * (DN + DR))
    wq_b[r, (7 * r) % QL] = 1
    w_uk = np.zeros((H, DC, DN), f)
    for h in range(H):
        w_uk[h, 4 * np.arange(DN) + h % 4, np.arange(DN)] = 1
    wkv_a = np.zeros((DC + DR, DIM), f)
    wkv_a[np.arange(DC + DR), QL + np.arange(DC + DR)] = 1
    iwq_b = np.zeros((HI * DI, QL), f)
    r = np.arange(HI * DI)
    iwq_b[r, (3 * r) % QL] = 1
    iwk = np.zeros((DI, DIM), f)
    iwk[np.arange(DI), 2112 + np.arange(DI)] = 1
    iw = np.zeros((HI, DIM), f)
    iw[np.arange(HI), 3000 + np.arange(HI)] = 1
    one = lambda n: np.ones(n, np.float32)
    return dict(wq_a=wq_a, q_norm=one(QL), wq_b=wq_b, w_uk=w_uk, wkv_a=wkv_a, kv_norm=one(DC), iwq_b=iwq_b, iwk=iwk,
                ik_norm_w=one(DI), ik_norm_b=np.full(DI, 0.25, np.float32), iw=iw)


def selection_closed_form(o):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, DIM)).astype(np.float16).astype(np.float64)
    pos = np.array([3, 50], dtype=np.int32)
    _, cos, sin = tables(64)
    c, s = cos[pos], sin[pos]                                        # (2, 32), the tables the op reads
    ch, sh = np.repeat(c[:, None], H, 1), np.repeat(s[:, None], H, 1)
    ci, si = np.repeat(c[:, None], HI, 1), np.repeat(s[:, None], HI, 1)
    r = run(o, x, pos, selection_weights())
    eps = odp.EPS
    r16 = lambda a: a.astype(np.float16).astype(np.float64)
    cq = r16(x[:, :QL] / np.sqrt((x[:, :QL] ** 2).mean(-1, keepdims=True) + eps))
    yq = cq[:, (7 * np.arange(H * (DN + DR))) % QL].reshape(2, H, DN + DR)
    q_lat = np.zeros((2, H, DC))
    for h in range(H):
        q_lat[:, h, 4 * np.arange(DN) + h % 4] = r16(yq[:, h, :DN])
    q = np.concatenate([q_lat, rope_complex(yq[:, :, DN:], ch, sh)], -1)
    kvc = x[:, QL:QL + DC]
    kv = np.concatenate([kvc / np.sqrt((kvc ** 2).mean(-1, keepdims=True) + eps),
                         rope_complex(x[:, QL + DC:QL + DC + DR], c, s)], -1)
    yi = cq[:, (3 * np.arange(HI * DI)) % QL].reshape(2, HI, DI)
    iq = np.concatenate([rope_complex_halves(yi[..., :DR], ci, si), yi[..., DR:]], -1)
    v = x[:, 2112:2112 + DI]
    ln = (v - v.mean(-1, keepdims=True)) / np.sqrt(v.var(-1, keepdims=True) + eps) + 0.25
    ik = np.concatenate([rope_complex_halves(ln[:, :DR], c, s), ln[:, DR:]], -1)
    w = x[:, 3000:3000 + HI] / np.sqrt(HI * DI)
    close = lambda a, b: np.allclose(a, b, rtol=1e-9, atol=1e-9)
    return close(r["q"], q) and close(r["kv_row"], kv) and close(r["iq"], iq) and close(r["ik_row"], ik) and \
        close(r["w"], w)


CHECKS = [norms_vs_torch, rope_vs_complex, rope_forms_differ, zero_input, scale_structure, selection_closed_form]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    assert check(odp)


# ----------------------------------------------------------------------------------------------- planted mistakes
_layernorm = odp.layernorm                                             # the original, for the mutants that wrap it


def _rope_halves(v, c, s):
    n = v.shape[-1] // 2
    return np.concatenate([v[..., :n] * c - v[..., n:] * s, v[..., :n] * s + v[..., n:] * c], -1)


MUTANTS = {
    "MLA rope on halves, not interleaved pairs": dict(rope=_rope_halves),
    "indexer rope on interleaved pairs, not halves": dict(rope_half=odp.rope),
    "rmsnorm without eps": dict(rmsnorm=lambda v, w, eps=0.0: v / np.sqrt(np.mean(v * v, -1, keepdims=True)) * w),
    "layernorm without bias": dict(layernorm=lambda v, w, b, eps=odp.EPS: _layernorm(v, w, 0 * b, eps)),
    "layernorm with the unbiased variance": dict(
        layernorm=lambda v, w, b, eps=odp.EPS: (v - v.mean(-1, keepdims=True)) /
        np.sqrt(v.var(-1, ddof=1, keepdims=True) + eps) * w + b),
    "q head as pe, nope": dict(split_q=lambda y: (y[..., DR:], y[..., :DR])),
    "iq head as nope, pe": dict(split_iq=lambda y: (y[..., DI - DR:], y[..., :DI - DR])),
    "absorb with the heads reversed": dict(absorb=lambda n, w: np.einsum("bhd,hcd->bhc", n, w[::-1])),
    "w not pre-scaled": dict(W_SCALE=1.0),
}


@pytest.mark.parametrize("kind", list(MUTANTS))
def test_checks_catch_planted_mistakes(kind, monkeypatch):
    for name, value in MUTANTS[kind].items():
        monkeypatch.setattr(odp, name, value)
    assert not all(check(odp) for check in CHECKS), kind
