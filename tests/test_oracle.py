"""Pins the float64 oracle (oracle/) without importing the reference.

Each check compares the oracle against something independent of its own formula: PyTorch's float64 SDPA on the CPU
(a library routine), closed forms, the cascade/LSE identity, the prefix<->spec equivalence and brute-force sorting.
Every check is also run against a planted mistake in a copy of the oracle (dropped max subtraction, dropped scale,
GQA heads grouped the wrong way, mask bits reversed, off-by-one top-k, ...) and must reject it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import decode as odecode, dsa as odsa, prefix as oprefix, prefix_paged as opaged, spec as ospec
from oracle.common import softmax_attend, to64
from vmk.ops import decode, dsa, prefix, prefix_paged, spec


def t64(x):
    return torch.from_numpy(to64(x))


# ------------------------------------------------------------------------------------------- independent checks
def prefix_vs_torch(ref, shape, seed=0, dist="randn"):
    inp = prefix.make_inputs(shape, seed=seed, dist=dist)
    q, kp, vp, ks, vs, sl = (inp[k] for k in ("q", "kp", "vp", "ks", "vs", "slens"))
    lay = prefix.build_layouts(t64(kp), t64(vp), t64(ks), t64(vs))
    m = prefix.valid_mask(kp.shape[1], ks.shape[2], sl, "cpu")
    o = F.scaled_dot_product_attention(t64(q)[:, :, None], lay["kf"], lay["vf"], attn_mask=m, enable_gqa=True)[:, :, 0]
    r = ref(**inp)
    return np.allclose(r, o.numpy(), rtol=1e-9, atol=1e-9, equal_nan=True)


def spec_vs_torch(ref, shape, seed=0, dist="randn"):
    inp = spec.make_inputs(shape, seed=seed, dist=dist)
    q, k, v, bits = inp["q"], inp["k"], inp["v"], inp["bits"]
    m = spec.draft_mask(bits, k.shape[2], q.shape[1])[:, None]
    o = F.scaled_dot_product_attention(t64(q).transpose(1, 2), t64(k), t64(v), attn_mask=m, enable_gqa=True)
    r = ref(**inp)
    return np.allclose(r, o.transpose(1, 2).numpy(), rtol=1e-9, atol=1e-9, equal_nan=True)


def dsa_vs_torch(ref, shape, seed=0, dist="randn"):
    inp = dsa.make_inputs(shape, seed=seed, dist=dist)
    _, sel = odsa.ref_select64(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    kv = t64(inp["kv"])
    outs = []
    for b in range(kv.shape[0]):
        ks = kv[b, torch.from_numpy(np.asarray(sel[b]))]
        o = F.scaled_dot_product_attention(t64(inp["q"])[b][None, :, None], ks[None, None], ks[None, None, :, :512],
                                           scale=dsa.SCALE)
        outs.append(o[0, :, 0])
    r = ref(**inp, sel=sel)
    return np.allclose(r, torch.stack(outs).numpy(), rtol=1e-9, atol=1e-9, equal_nan=True)


def select_vs_sort(sel_fn, shape, seed=0, dist="randn"):
    """Brute force: the selected set must be exactly the positions of the 2048 largest scores (no ties in float64
    for random inputs), or every valid position when there are <= 2048."""
    inp = dsa.make_inputs(shape, seed=seed, dist=dist)
    s, sel = sel_fn(inp["iq"], inp["ik"], inp["w"], inp["lens"])
    B, L = s.shape
    lens = inp["lens"]
    for b in range(B):
        n = L if lens is None else int(lens[b])
        want = np.arange(n) if n <= 2048 else np.sort(np.argsort(-s[b, :n], kind="stable")[:2048])
        if not np.array_equal(np.sort(np.asarray(sel[b])), want):
            return False
    return True


def scores_brute(sel_fn, shape, seed=0):
    """Scores against a pure-Python triple loop on a few positions."""
    inp = dsa.make_inputs(shape, seed=seed)
    s, _ = sel_fn(inp["iq"], inp["ik"], inp["w"], None)
    iq, ik, w = to64(inp["iq"]), to64(inp["ik"]), inp["w"].double().numpy()
    for b in range(s.shape[0]):
        for l in (0, s.shape[1] // 2, s.shape[1] - 1):
            acc = 0.0
            for h in range(iq.shape[1]):
                dot = sum(float(iq[b, h, d]) * float(ik[b, l, d]) for d in range(iq.shape[2]))
                acc += float(w[b, h]) * max(dot, 0.0)
            if abs(acc - s[b, l]) > 1e-9 * max(1.0, abs(acc)):
                return False
    return True


def prefix_as_spec(ref_prefix, ref_spec, shape, seed=0):
    """Prefix(N, P, S) equals spec with B=N, one draft per request, cache = [prefix ; suffix]: the draft is the
    last suffix row and sees itself (bit 0)."""
    inp = prefix.make_inputs(shape, seed=seed)
    q, kp, vp, ks, vs = (inp[k] for k in ("q", "kp", "vp", "ks", "vs"))
    N = q.shape[0]
    k = torch.cat([kp[None].expand(N, -1, -1, -1), ks], 2)
    v = torch.cat([vp[None].expand(N, -1, -1, -1), vs], 2)
    bits = torch.ones(N, 1, dtype=torch.int32)
    r1 = ref_prefix(**inp)
    r2 = ref_spec(q[:, None], k, v, bits)[:, 0]
    return np.allclose(r1, r2, rtol=1e-12, atol=1e-12)


def cascade_identity(ref, shape, seed=0):
    """LSE merge of prefix-only and suffix-only attention equals the oracle's full softmax."""
    inp = prefix.make_inputs(shape, seed=seed)
    q, kp, vp, ks, vs = (to64(inp[k]) for k in ("q", "kp", "vp", "ks", "vs"))
    N, Hq, d = q.shape
    Hkv = kp.shape[0]
    G = Hq // Hkv
    qg = q.reshape(N, Hkv, G, d)
    s1 = np.einsum("nhgd,hld->nhgl", qg, kp) / math.sqrt(d)
    s2 = np.einsum("nhgd,nhld->nhgl", qg, ks) / math.sqrt(d)
    m1, m2 = s1.max(-1, keepdims=True), s2.max(-1, keepdims=True)
    p1, p2 = np.exp(s1 - m1), np.exp(s2 - m2)
    o1, o2 = np.einsum("nhgl,hld->nhgd", p1, vp), np.einsum("nhgl,nhld->nhgd", p2, vs)
    m = np.maximum(m1, m2)
    a, b = np.exp(m1 - m), np.exp(m2 - m)
    o = (o1 * a + o2 * b) / (p1.sum(-1, keepdims=True) * a + p2.sum(-1, keepdims=True) * b)
    return np.allclose(ref(**inp), o.reshape(N, Hq, d), rtol=1e-10, atol=1e-12)


def spec_closed_forms(ref, seed=0):
    """q = 0: uniform attention, i.e. the mean of V over the allowed keys; constant V rows give that constant;
    a row that sees a single key returns that key's V row."""
    shape = dict(B=2, L=40, k=6)
    inp = spec.make_inputs(shape, seed=seed)
    q0 = torch.zeros_like(inp["q"])
    o = ref(q0, inp["k"], inp["v"], inp["bits"])
    a = ospec.allowed(inp["bits"], 40, 6)                                # (B, kd, L)
    v = to64(inp["v"])                                                   # (B, Hkv, L, D)
    want = np.einsum("bil,bhld->bihd", a.astype(np.float64), v) / a.sum(-1)[:, :, None, None]
    want = np.repeat(want, 4, axis=2)                                    # heads h*G+g share KV head h
    ok = np.allclose(o, want, rtol=1e-12, atol=1e-12)
    vc = torch.full_like(inp["v"], 0.375)
    ok &= np.allclose(ref(inp["q"], inp["k"], vc, inp["bits"]), 0.375, rtol=0, atol=1e-12)
    one = spec.make_inputs(dict(B=1, L=1, k=1), seed=seed)
    ok &= np.allclose(ref(**one)[0, 0], np.repeat(to64(one["v"])[0, :, 0], 4, axis=0), rtol=0, atol=0)
    return bool(ok)


def chain_is_causal(ref, seed=0):
    """Chain row i equals causal attention over the context and drafts 0..i (torch's is_causal on the tail)."""
    shape = dict(B=2, L=50, k=7)
    inp = spec.make_inputs(shape, seed=seed, dist="chain")
    q, k, v = (t64(inp[x]) for x in ("q", "k", "v"))
    L, kd = 50, 7
    m = torch.ones(kd, L, dtype=torch.bool)
    m[:, L - kd:] = torch.ones(kd, kd, dtype=torch.bool).tril()
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k, v, attn_mask=m, enable_gqa=True).transpose(1, 2)
    return np.allclose(ref(**inp), o.numpy(), rtol=1e-10, atol=1e-12)


def key_permutation(ref, shape, seed=0):
    inp = prefix.make_inputs(shape, seed=seed)
    perm = torch.from_numpy(np.random.default_rng(1).permutation(shape["P"]))
    inp2 = dict(inp, kp=inp["kp"][:, perm], vp=inp["vp"][:, perm])
    return np.allclose(ref(**inp), ref(**inp2), rtol=1e-10, atol=1e-12)


def no_overflow_large(ref):
    """Scores of several hundred (q x40 on top of the `large` recipe) must give a finite output: a softmax without
    the max subtraction overflows even in float64."""
    inp = spec.make_inputs(dict(B=1, L=300, k=4), seed=3, dist="large")
    inp["q"] = inp["q"] * 40
    return bool(np.isfinite(ref(**inp)).all())


# ------------------------------------------------------------------------------------------- planted mistakes
def _attend_nomax(s, v):
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        p = np.exp(s)
        return (p / p.sum(-1, keepdims=True)) @ v


def prefix_mutant(kind):
    def ref(q, kp, vp, ks, vs, slens=None, **_):
        q, kp, vp, ks, vs = (to64(x) for x in (q, kp, vp, ks, vs))
        N, Hq, d = q.shape
        Hkv = kp.shape[0]
        G = Hq // Hkv
        out = np.empty((N, Hkv, G, d))
        for n in range(N):
            sn = ks.shape[2] if slens is None else int(slens[n])
            if kind == "ragged_ignored":
                sn = ks.shape[2]
            k = np.concatenate([kp, ks[n, :, :sn]], 1)
            v = np.concatenate([vp, vs[n, :, :sn]], 1)
            qn = q[n].reshape(Hkv, G, d)
            if kind == "gqa_transposed":
                qn = q[n].reshape(G, Hkv, d).transpose(1, 0, 2)
            sc = 1.0 if kind == "no_scale" else 1 / math.sqrt(d)
            s = qn @ k.transpose(0, 2, 1) * sc
            if kind == "prefix_only":
                s[..., kp.shape[1]:] = -np.inf
            out[n] = (_attend_nomax if kind == "no_max" else softmax_attend)(s, v)
        return out.reshape(N, Hq, d)
    return ref


def spec_mutant(kind):
    def ref(q, k, v, bits):
        q, k, v = (to64(x) for x in (q, k, v))
        B, kd, Hq, d = q.shape
        Hkv, L = k.shape[1], k.shape[2]
        G = Hq // Hkv
        a = ospec.allowed(bits, L, kd)
        if kind == "bits_reversed":
            a[:, :, L - kd:] = a[:, :, L - kd:][:, :, ::-1]
        if kind == "mask_shifted":
            a[:, :, L - kd - 1:L - 1] = a[:, :, L - kd:].copy()
            a[:, :, L - 1] = True
        s = np.einsum("bihgd,bhld->bihgl", q.reshape(B, kd, Hkv, G, d), k) / math.sqrt(d)
        s = np.where(a[:, :, None, None, :], s, -np.inf)
        f = _attend_nomax if kind == "no_max" else softmax_attend
        o = np.stack([np.stack([f(s[b, :, h], v[b, h]) for h in range(Hkv)], 1) for b in range(B)])
        return o.reshape(B, kd, Hq, d)
    return ref


def select_mutant(kind):
    def sel_fn(iq, ik, w, lens=None):
        s = odsa.scores64(iq, ik, w)
        if kind == "no_relu":
            iq64, ik64 = to64(iq), to64(ik)
            s = ((iq64 @ ik64.transpose(0, 2, 1)) * np.asarray(w, dtype=np.float64)[:, :, None]).sum(1)
        if kind == "unweighted":
            s = np.maximum(to64(iq) @ to64(ik).transpose(0, 2, 1), 0).sum(1)
        B, L = s.shape
        sel = []
        for b in range(B):
            n = L if lens is None else int(lens[b])
            if kind == "lens_ignored":
                n = L
            if n <= 2048:
                sel.append(np.arange(n))
            elif kind == "off_by_one":
                sel.append(np.argpartition(-s[b, :n], 2048)[1:2049])
            elif kind == "smallest":
                sel.append(np.argpartition(s[b, :n], 2047)[:2048])
            else:
                sel.append(np.argpartition(-s[b, :n], 2047)[:2048])
        return s, sel
    return sel_fn


def dsa_mutant(kind):
    def ref(q, kv, iq, ik, w, lens=None, sel=None):
        q, kv = to64(q), to64(kv)
        out = np.zeros((q.shape[0], 128, 512))
        for b in range(q.shape[0]):
            ks = kv[b, sel[b]]
            if kind == "nope_only":
                s = q[b, :, :512] @ ks[:, :512].T * odsa.SCALE
            elif kind == "scale_128":
                s = q[b] @ ks.T / math.sqrt(128)
            else:
                s = q[b] @ ks.T * odsa.SCALE
            out[b] = softmax_attend(s, ks[:, 64:] if kind == "value_rope_side" else ks[:, :512])
        return out
    return ref


# ------------------------------------------------------------------------------------------- tests
PREFIX_SHAPES = [dict(N=3, P=70, S=9), dict(N=2, P=1, S=1), dict(N=4, P=33, S=20, S_min=1)]


@pytest.mark.parametrize("shape", PREFIX_SHAPES)
def test_prefix_vs_torch_sdpa(shape):
    assert prefix_vs_torch(oprefix.ref64, shape)


def test_prefix_nan_inf_vs_torch():
    assert prefix_vs_torch(oprefix.ref64, dict(N=4, P=30, S=6), dist="nan_inf")


def test_prefix_identities():
    assert cascade_identity(oprefix.ref64, dict(N=3, P=64, S=17))
    assert prefix_as_spec(oprefix.ref64, ospec.ref64, dict(N=3, P=50, S=7))
    assert key_permutation(oprefix.ref64, dict(N=2, P=40, S=5))


@pytest.mark.parametrize("kind", ["no_scale", "gqa_transposed", "prefix_only", "ragged_ignored", "no_max"])
def test_prefix_checks_catch_planted_mistakes(kind):
    bad = prefix_mutant(kind)
    caught = not all([prefix_vs_torch(bad, s) for s in PREFIX_SHAPES]) or not cascade_identity(bad, dict(N=3, P=64, S=17))
    if kind == "no_max":  # only overflow shows it: large scores
        inp = prefix.make_inputs(dict(N=2, P=300, S=20), seed=1, dist="large")
        inp["q"] = inp["q"] * 40
        caught = not np.isfinite(bad(**inp)).all() and np.isfinite(oprefix.ref64(**inp)).all()
    assert caught


SPEC_SHAPES = [(dict(B=2, L=37, k=5), "randn"), (dict(B=1, L=8, k=8), "randn"), (dict(B=2, L=90, k=40), "randn"),
               (dict(B=1, L=200, k=64), "tree_bd"), (dict(B=2, L=60, k=6), "needle_masked"),
               (dict(B=1, L=70, k=33), "chain")]


@pytest.mark.parametrize("shape,dist", SPEC_SHAPES)
def test_spec_vs_torch_sdpa(shape, dist):
    assert spec_vs_torch(ospec.ref64, shape, dist=dist)


def test_spec_identities():
    assert spec_closed_forms(ospec.ref64)
    assert chain_is_causal(ospec.ref64)
    assert no_overflow_large(ospec.ref64)


@pytest.mark.parametrize("kind", ["bits_reversed", "mask_shifted", "no_max"])
def test_spec_checks_catch_planted_mistakes(kind):
    bad = spec_mutant(kind)
    caught = (not all(spec_vs_torch(bad, s, dist=d) for s, d in SPEC_SHAPES[:2] + SPEC_SHAPES[4:5])
              or not chain_is_causal(bad) or not no_overflow_large(bad))
    assert caught


def test_allowed_matches_reference_int32_layout():
    """Reference layout (B, kd) int32 with bit 31 set (kd = 32) and the word layout give the same mask."""
    w = spec.chain_bits(32)[None]                                    # (1, 32, 1) uint32
    a1 = ospec.allowed(torch.from_numpy(w.view(np.int32)[..., 0].copy()), 40, 32)
    a2 = ospec.allowed(torch.from_numpy(w.view(np.int32)), 40, 32)
    assert np.array_equal(a1, a2)
    assert np.array_equal(a1[0, :, 8:], np.tril(np.ones((32, 32), dtype=bool)))


DSA_SHAPES = [(dict(B=2, L=2100), "randn"), (dict(B=1, L=300), "randn"), (dict(B=3, L=2600), "ragged"),
              (dict(B=1, L=2049), "needle")]


@pytest.mark.parametrize("shape,dist", DSA_SHAPES)
def test_dsa_select_vs_sort(shape, dist):
    assert select_vs_sort(odsa.ref_select64, shape, dist=dist)


def test_dsa_scores_brute_force():
    assert scores_brute(odsa.ref_select64, dict(B=2, L=37))


@pytest.mark.parametrize("shape,dist", DSA_SHAPES[:3])
def test_dsa_attention_vs_torch_sdpa(shape, dist):
    assert dsa_vs_torch(odsa.ref64, shape, dist=dist)


@pytest.mark.parametrize("kind", ["no_relu", "unweighted", "lens_ignored", "off_by_one", "smallest"])
def test_dsa_select_checks_catch_planted_mistakes(kind):
    bad = select_mutant(kind)
    assert not (all(select_vs_sort(bad, s, dist=d) for s, d in DSA_SHAPES) and scores_brute(bad, dict(B=2, L=37)))


@pytest.mark.parametrize("kind", ["nope_only", "scale_128", "value_rope_side"])
def test_dsa_attention_checks_catch_planted_mistakes(kind):
    assert not all(dsa_vs_torch(dsa_mutant(kind), s, dist=d) for s, d in DSA_SHAPES[:3])


def test_topk_set_check_accepts_boundary_swaps_only():
    rng = np.random.default_rng(0)
    s = rng.standard_normal(5000)
    s[100] = s[200] = np.sort(s)[-2048]                  # an exact tie at the threshold
    top = np.argsort(-s, kind="stable")[:2048]
    bound = 1e-12
    ok, det = odsa.topk_set_check(top, 2048, s, 5000, bound)
    assert ok and det["boundary"] == 3                   # the value's own position and its two copies
    alt = top.copy()
    tied = [i for i in (100, 200) if i in set(top)]
    other = 300 - tied[0] if len(tied) == 1 else None
    if other is not None:                                # swapping the tied pair keeps the set valid
        alt[list(top).index(tied[0])] = other
        assert odsa.topk_set_check(alt, 2048, s, 5000, bound)[0]
    bad = top.copy()
    bad[0] = np.argsort(s)[0]                            # the smallest score is never in the top set
    assert not odsa.topk_set_check(bad, 2048, s, 5000, bound)[0]
    assert not odsa.topk_set_check(top[:2047], 2047, s, 5000, bound)[0]
    assert odsa.topk_set_check(np.arange(1500)[::-1], 1500, s, 1500, bound)[0]
    s2 = rng.standard_normal(5000)                       # no ties: the 2049th position for the 2048th passes
    order = np.argsort(-s2)                              # only if the band covers their gap
    near = order[:2048].copy()
    near[2047] = order[2048]
    gap = s2[order[2047]] - s2[order[2048]]
    assert odsa.topk_set_check(near, 2048, s2, 5000, gap)[0]
    assert not odsa.topk_set_check(near, 2048, s2, 5000, gap / 4)[0]


def _scores32(iq, ik, w, sequential):
    """An fp32 evaluation of the indexer scores from the same 16-bit values: products exact in fp32, the 128-term
    dot products by float32 BLAS (sequential=False) or summed strictly left to right (sequential=True), then the
    ReLU, the weight and a float32 sum over the heads."""
    q = iq.float().numpy().astype(np.float32)
    k = ik.float().numpy().astype(np.float32)
    w = w.numpy().astype(np.float32)
    if sequential:
        prod = q[:, :, None, :] * k[:, None, :, :]                 # (B, HI, L, DI), exact
        dots = np.add.accumulate(prod, axis=3, dtype=np.float32)[..., -1]
    else:
        dots = np.matmul(q, k.transpose(0, 2, 1))
    terms = (np.maximum(dots, np.float32(0)) * w[:, :, None]).astype(np.float32)
    return np.add.accumulate(terms, axis=1, dtype=np.float32)[:, -1].astype(np.float64)


@pytest.mark.parametrize("dist,L,seq", [("randn", 3000, False), ("randn", 300, True), ("needle", 300, True)])
def test_score_error_bound_covers_fp32_evaluations(dist, L, seq):
    inp = dsa.make_inputs(dict(B=2, L=L), seed=3, dist=dist)
    s64 = odsa.scores64(inp["iq"], inp["ik"], inp["w"])
    bound = odsa.score_error_bound(inp["iq"], inp["ik"], inp["w"])
    err = np.abs(_scores32(inp["iq"], inp["ik"], inp["w"], seq) - s64).max(1)
    assert np.all(err <= bound), (err, bound)
    assert np.all(bound < 2e-3 * s64.std(1)), (bound, s64.std(1))   # far below the scores' spread


def test_score_error_bound_keeps_the_c5_check_tight():
    """At C5's inputs the band (2 x bound, about 1.4e-3) holds 15-35 of each request's positions around the
    2048th score, and a selection from scores with one head dropped fails the check."""
    inp = dsa.make_inputs(dict(B=4, L=65536), seed=0, dist="randn")
    s64, sel = odsa.ref_select64(inp["iq"], inp["ik"], inp["w"])
    bound = odsa.score_error_bound(inp["iq"], inp["ik"], inp["w"])
    w_bad = inp["w"].clone()
    w_bad[:, 0] = 0
    s_bad, sel_bad = odsa.ref_select64(inp["iq"], inp["ik"], w_bad)
    for b in range(4):
        ok, det = odsa.topk_set_check(sel[b], 2048, s64[b], 65536, bound[b])
        assert ok and det["boundary"] <= 64 and det["swapped"] == 0, det
        assert not odsa.topk_set_check(sel_bad[b], 2048, s64[b], 65536, bound[b])[0]


DECODE_SHAPES = [(dict(B=2, L=37), "randn"), (dict(B=1, L=1), "randn"), (dict(B=4, L=90, L_min=1), "randn"),
                 (dict(B=2, L=300, Hq=8, Hkv=2), "needle"), (dict(B=3, L=64, L_min=30), "nan_inf")]


def decode_vs_torch(ref, shape, seed=0, dist="randn"):
    inp = decode.make_inputs(shape, seed=seed, dist=dist)
    m = decode.valid_mask(inp["k"].shape[2], inp["lens"], "cpu")
    o = F.scaled_dot_product_attention(t64(inp["q"])[:, :, None], t64(inp["k"]), t64(inp["v"]), attn_mask=m,
                                       enable_gqa=True)[:, :, 0]
    return np.allclose(ref(**inp), o.numpy(), rtol=1e-9, atol=1e-9, equal_nan=True)


def decode_as_spec(ref, shape, seed=0):
    """Decode of request b equals spec with one draft (bit 0: the draft sees itself) over the first lens[b] cache
    positions."""
    inp = decode.make_inputs(shape, seed=seed)
    r = ref(**inp)
    for b in range(inp["q"].shape[0]):
        n = inp["k"].shape[2] if inp["lens"] is None else int(inp["lens"][b])
        r2 = ospec.ref64(inp["q"][b:b + 1, None], inp["k"][b:b + 1, :, :n], inp["v"][b:b + 1, :, :n],
                         torch.ones(1, 1, dtype=torch.int32))[0, 0]
        if not np.allclose(r[b], r2, rtol=1e-12, atol=1e-12):
            return False
    return True


def decode_closed_forms(ref, seed=0):
    """q = 0 gives the mean of V over the positions in use; lens = 1 returns V row 0."""
    inp = decode.make_inputs(dict(B=3, L=50, L_min=1), seed=seed)
    inp["q"] = torch.zeros_like(inp["q"])
    v, G = to64(inp["v"]), decode.HQ // decode.HKV
    r = ref(**inp)
    for b in range(3):
        n = int(inp["lens"][b])
        if not np.allclose(r[b], np.repeat(v[b, :, :n].mean(1), G, 0), rtol=1e-12, atol=1e-12):
            return False
    inp = decode.make_inputs(dict(B=2, L=20), seed=seed + 1)
    inp["lens"] = torch.ones(2, dtype=torch.int32)
    return np.allclose(ref(**inp), np.repeat(to64(inp["v"])[:, :, 0], G, 1), rtol=1e-12, atol=1e-12)


def decode_mutant(kind):
    def out(q, k, v, lens=None):
        if kind == "lens_ignored":
            return odecode.ref64(q, k, v, None)
        if kind == "lens_off_by_one":
            return odecode.ref64(q, k, v, None if lens is None else lens - 1)
        if kind == "gqa_transposed":                    # head h reads KV head h % Hkv instead of h // G
            Hkv = k.shape[1]
            idx = torch.arange(q.shape[1]).reshape(Hkv, -1).t().reshape(-1)
            return odecode.ref64(q[:, idx], k, v, lens)[:, torch.argsort(idx)]
        if kind == "no_scale":
            return odecode.ref64(q * math.sqrt(q.shape[-1]), k, v, lens)
    return out


@pytest.mark.parametrize("shape,dist", DECODE_SHAPES)
def test_decode_vs_torch_sdpa(shape, dist):
    assert decode_vs_torch(odecode.ref64, shape, dist=dist)


def test_decode_identities():
    assert decode_as_spec(odecode.ref64, dict(B=3, L=70, L_min=1))
    assert decode_closed_forms(odecode.ref64)


@pytest.mark.parametrize("kind", ["lens_ignored", "lens_off_by_one", "gqa_transposed", "no_scale"])
def test_decode_checks_catch_planted_mistakes(kind):
    bad = decode_mutant(kind)
    assert not (all(decode_vs_torch(bad, s, dist=d) for s, d in DECODE_SHAPES) and decode_closed_forms(bad))


PAGED_SHAPES = [(dict(N=3, P=128, S=77, ps=32), "randn"), (dict(N=4, P=192, S=200, S_min=0, ps=64), "randn"),
                (dict(N=2, P=0, S=90, ps=32), "randn"), (dict(N=4, P=384, S=256, ps=96), "nan_inf"),
                (dict(N=3, P=256, S=130, S_min=1, ps=128), "needle_suffix")]


def paged_equals_contiguous(ref, shape, seed=0, dist="randn"):
    """With every page present the op is the contiguous op on the same draws (the generator scatters those draws):
    the paged oracle must give the contiguous oracle's float64 bits."""
    inp = prefix_paged.make_inputs(shape, seed=seed, dist=dist)
    c = prefix.make_inputs({k: v for k, v in shape.items() if k != "ps"}, seed=seed, dist=dist)
    if inp["slens"] is not None and c["slens"] is None:
        c["slens"] = inp["slens"]
    return np.array_equal(ref(**inp), oprefix.ref64(**c), equal_nan=True)


def paged_absent_vs_torch(ref, shape, seed=0):
    """Absent pages: torch float64 SDPA over a dense cache from which the absent pages' rows are deleted."""
    inp = prefix_paged.make_inputs(shape, seed=seed)
    kpool, vpool = t64(inp["k_pages"]), t64(inp["v_pages"])
    num_pages, Hkv, ps, d = kpool.shape
    pp, sp = inp["prefix_pages"].tolist(), inp["suffix_pages"].tolist()
    S = len(sp[0]) * ps
    outs = []
    for n in range(inp["q"].shape[0]):
        sn = S if inp["slens"] is None else min(max(int(inp["slens"][n]), 0), S)
        rows_k, rows_v = [], []
        for j, p in enumerate(pp):
            if 0 <= p < num_pages:
                rows_k.append(kpool[p]), rows_v.append(vpool[p])
        for j, p in enumerate(sp[n]):
            take = min(ps, sn - j * ps)
            if take > 0 and 0 <= p < num_pages:
                rows_k.append(kpool[p, :, :take]), rows_v.append(vpool[p, :, :take])
        k, v = torch.cat(rows_k, 1), torch.cat(rows_v, 1)
        outs.append(F.scaled_dot_product_attention(t64(inp["q"][n:n + 1])[:, :, None], k[None], v[None],
                                                   enable_gqa=True)[0, :, 0])
    return np.allclose(ref(**inp), torch.stack(outs).numpy(), rtol=1e-9, atol=1e-9, equal_nan=True)


def paged_mutant(kind):
    def out(q, k_pages, v_pages, prefix_pages, suffix_pages, slens=None):
        pp, sp = prefix_pages.clone(), suffix_pages.clone()
        if kind == "table_order_ignored":              # pages taken in pool order instead of table order
            pp = pp.sort().values
            sp = sp.sort(1).values
        elif kind == "absent_as_page0":                 # an absent page read as page 0
            pp, sp = pp.clamp(min=0), sp.clamp(min=0)
        elif kind == "slens_ignored":
            slens = None
        return opaged.ref64(q, k_pages, v_pages, pp, sp, slens)
    return out


@pytest.mark.parametrize("shape,dist", PAGED_SHAPES)
def test_paged_oracle_equals_contiguous(shape, dist):
    assert paged_equals_contiguous(opaged.ref64, shape, dist=dist)


def test_paged_oracle_absent_pages_vs_torch():
    assert paged_absent_vs_torch(opaged.ref64, dict(N=6, P=3072, S=500, S_min=0, ps=64, absent=3), seed=5)
    assert paged_absent_vs_torch(opaged.ref64, dict(N=5, P=640, S=40, ps=32, absent=2), seed=6)


def test_paged_standard_op_vs_oracle():
    inp = prefix_paged.make_inputs(dict(N=6, P=3072, S=500, S_min=0, ps=64, absent=3), seed=5)
    d = {k: (v.double() if v is not None and v.dtype == torch.float16 else v) for k, v in inp.items()}
    assert np.allclose(prefix_paged.torch_naive(**d).numpy(), opaged.ref64(**inp), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("kind", ["table_order_ignored", "absent_as_page0", "slens_ignored"])
def test_paged_checks_catch_planted_mistakes(kind):
    bad = paged_mutant(kind)
    ok = all(paged_equals_contiguous(bad, s, dist=d) for s, d in PAGED_SHAPES) and \
        paged_absent_vs_torch(bad, dict(N=6, P=3072, S=500, S_min=0, ps=64, absent=3), seed=5)
    assert not ok


def test_oracle_is_test_infrastructure():
    assert "TEST INFRASTRUCTURE ONLY" in oracle.__doc__
