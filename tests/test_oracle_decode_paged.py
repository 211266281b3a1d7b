"""Pins the float64 oracle of paged single-token decode (oracle/decode_paged.py).

Independent checks: with every page present the op is the contiguous decode op on the same draws, whose oracle is
pinned in tests/test_oracle.py (float64 PyTorch SDPA, closed forms), so the two oracles must agree bit for bit; with
absent pages, float64 PyTorch SDPA over a dense cache from which the absent pages' rows are deleted; an NHD pool
gives the HND pool's result; and a request whose pages are all absent is NaN.  Every check is also run against
planted mistakes that the set of checks must reject.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode as odecode, decode_paged as odp
from vmk.ops import decode, decode_paged

SHAPES = [(dict(B=3, L=300, ps=64), "randn"), (dict(B=2, L=77, ps=32), "randn"),
          (dict(B=4, L=500, L_min=1, ps=96), "randn"), (dict(B=2, L=400, ps=128), "nan_inf"),
          (dict(B=3, L=256, Hq=16, Hkv=2, ps=32), "needle")]


def t64(x):
    return x.double() if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x, np.float64))


def equals_contiguous(ref, shape, dist, seed=0):
    inp = decode_paged.make_inputs(shape, seed=seed, dist=dist)
    c = decode.make_inputs({k: v for k, v in shape.items() if k != "ps"}, seed=seed, dist=dist)
    if c["lens"] is None and inp["lens"] is not None:
        c["lens"] = inp["lens"]
    return np.array_equal(ref(**inp), odecode.ref64(**c), equal_nan=True)


def absent_vs_torch(ref, shape, seed=0):
    inp = decode_paged.make_inputs(shape, seed=seed)
    kpool, vpool = t64(inp["k_pages"]), t64(inp["v_pages"])
    num_pages, Hkv, ps, d = kpool.shape
    table = inp["page_table"].tolist()
    L = len(table[0]) * ps
    outs = []
    for b in range(inp["q"].shape[0]):
        n = L if inp["lens"] is None else min(max(int(inp["lens"][b]), 1), L)
        ks, vs = [], []
        for j, p in enumerate(table[b]):
            take = min(ps, n - j * ps)
            if take > 0 and 0 <= p < num_pages:
                ks.append(kpool[p, :, :take])
                vs.append(vpool[p, :, :take])
        k, v = torch.cat(ks, 1), torch.cat(vs, 1)
        outs.append(F.scaled_dot_product_attention(t64(inp["q"][b:b + 1])[:, :, None], k[None], v[None],
                                                   enable_gqa=True)[0, :, 0])
    return np.allclose(ref(**inp), torch.stack(outs).numpy(), rtol=1e-9, atol=1e-9)


def nhd_equals_hnd(ref, seed=0):
    shape = dict(B=3, L=500, L_min=1, ps=64, absent=1)
    a = decode_paged.make_inputs(shape, seed=seed)
    b = decode_paged.make_inputs(dict(shape, layout="NHD"), seed=seed)
    return np.array_equal(ref(**a), ref(**b), equal_nan=True)


def all_absent_is_nan(ref, seed=0):
    inp = decode_paged.make_inputs(dict(B=3, L=200, ps=64), seed=seed)
    inp["page_table"][1] = -1
    o = ref(**inp)
    return np.isnan(o[1]).all() and not np.isnan(o[[0, 2]]).any()


def passes(ref):
    return all(equals_contiguous(ref, s, d) for s, d in SHAPES) and \
        absent_vs_torch(ref, dict(B=5, L=3000, L_min=1, ps=64, absent=3), seed=4) and \
        absent_vs_torch(ref, dict(B=3, L=900, ps=96, absent=2), seed=5) and nhd_equals_hnd(ref) and \
        all_absent_is_nan(ref)


@pytest.mark.parametrize("shape,dist", SHAPES)
def test_oracle_equals_contiguous(shape, dist):
    assert equals_contiguous(odp.ref64, shape, dist)


def test_oracle_absent_pages_vs_torch():
    assert absent_vs_torch(odp.ref64, dict(B=5, L=3000, L_min=1, ps=64, absent=3), seed=4)
    assert absent_vs_torch(odp.ref64, dict(B=3, L=900, ps=96, absent=2), seed=5)


def test_oracle_nhd_and_empty_requests():
    assert nhd_equals_hnd(odp.ref64) and all_absent_is_nan(odp.ref64)


def test_standard_op_vs_oracle():
    for layout in ("HND", "NHD"):
        inp = decode_paged.make_inputs(dict(B=5, L=3000, L_min=1, ps=64, absent=3, layout=layout), seed=4)
        d = {k: (v.double() if isinstance(v, torch.Tensor) and v.dtype == torch.float16 else v)
             for k, v in inp.items()}
        assert np.allclose(decode_paged.torch_sdpa(**d).numpy(), odp.ref64(**inp), rtol=1e-9, atol=1e-9)


def mutant(kind):
    def out(q, k_pages, v_pages, page_table, lens=None, layout="HND"):
        pt = page_table.clone()
        if kind == "table_order_ignored":              # pages taken in pool order instead of table order
            pt = pt.sort(1).values
        elif kind == "absent_as_page0":                 # an absent page read as page 0
            pt = pt.clamp(min=0)
        elif kind == "lens_ignored":
            lens = None
        elif kind == "layout_ignored" and layout == "NHD":   # an NHD pool's memory read in the HND order
            layout = "HND"
            k_pages = k_pages.reshape(k_pages.shape[0], k_pages.shape[2], k_pages.shape[1], -1)
            v_pages = v_pages.reshape(v_pages.shape[0], v_pages.shape[2], v_pages.shape[1], -1)
        return odp.ref64(q, k_pages, v_pages, pt, lens, layout)
    return out


def test_oracle_passes_every_check():
    assert passes(odp.ref64)


@pytest.mark.parametrize("kind", ["table_order_ignored", "absent_as_page0", "lens_ignored", "layout_ignored"])
def test_checks_catch_planted_mistakes(kind):
    assert not passes(mutant(kind)), kind
