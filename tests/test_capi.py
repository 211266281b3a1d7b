"""The C-ABI library: builds, loads without a GPU, and exports exactly the entry points include/vmk.h declares.
Argument checks that reject before any launch are exercised here too (they never touch the GPU)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vmk.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(vmk_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from vmk import lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libvmk.so not built")
    return L.load()


def test_header_declares_the_binding_table():
    from vmk import lib as L
    assert declared() == sorted(L.exported_symbols())


def prototypes():
    """name -> (return type, [parameter types]) of every function include/vmk.h declares."""
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(vmk_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        params = [a.strip() for a in args.split(",")]
        params = [] if params == ["void"] else [re.sub(r"\s*\b\w+$", "", a) if not a.endswith("*") else a
                                                 for a in params]
        out[name] = (" ".join(ret.split()), params)
    return out


def test_binding_table_matches_the_header_prototypes():
    """Every ctypes signature in vmk/lib.py has the header's parameter count and types, and its return type, so a
    change on one side of the ABI cannot go unnoticed."""
    import ctypes as C
    from vmk import lib as L
    ctype = {"int64_t": C.c_int64, "size_t": C.c_size_t, "int": C.c_int, "float": C.c_float, "uint32_t": C.c_uint32}
    protos = prototypes()
    assert sorted(protos) == sorted(L.exported_symbols())
    for name, (ret, params) in protos.items():
        want = [C.c_void_p if "*" in t else ctype[t.replace("const ", "").strip()] for t in params]
        assert L._SIGS[name] == want, (name, params)
        want_ret = {"int": C.c_int, "size_t": C.c_size_t, "const char*": C.c_char_p}[ret]
        assert L._RET.get(name, C.c_int) == want_ret, (name, ret)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (vmk_[a-z0-9_]+)\b", out))
    missing = [s for s in declared() if s not in exported]
    assert not missing, missing


def test_version_and_error_string(lib):
    assert lib.vmk_version() == 1
    assert isinstance(lib.vmk_last_error(), bytes)


def test_workspace_queries_reject_bad_shapes(lib):
    assert lib.vmk_spec_workspace_size(1, 8, 32, 8, 64, 100) == 0        # D != 128
    assert lib.vmk_spec_workspace_size(1, 8, 30, 8, 128, 100) == 0       # Hq not a multiple of Hkv
    assert lib.vmk_spec_workspace_size(1, 8, 32, 8, 128, 4) == 0         # L < kd
    assert lib.vmk_spec_workspace_size(4, 8, 32, 8, 128, 32768) > 0
    assert lib.vmk_prefix_workspace_size(8, 32, 8, 128, 0, 0, 0) == 0     # no keys at all
    assert lib.vmk_prefix_workspace_size(8, 32, 8, 128, 2048, 256, 0) > 0
    assert lib.vmk_decode_workspace_size(2, 32, 8, 64, 100) == 0          # D != 128
    assert lib.vmk_decode_workspace_size(2, 32, 8, 128, 0) == 0           # no cache positions
    assert lib.vmk_decode_workspace_size(2, 32, 8, 128, 65536) > 0
    assert lib.vmk_prefix_paged_workspace_size(8, 32, 8, 128, 2048, 48, 4) == 0     # page size not a multiple of 32
    assert lib.vmk_prefix_paged_workspace_size(8, 32, 8, 128, 2000, 64, 4) == 0     # P not a whole number of pages
    assert lib.vmk_prefix_paged_workspace_size(8, 32, 8, 128, 2048, 64, 4) > 0
    assert lib.vmk_dsa_workspace_size(0, 100) == 0
    assert lib.vmk_dsa_workspace_size(4, 65536) > 4 * 65536 * 4


def test_entry_points_reject_before_launch(lib):
    """Host-side checks return 1 with a message and launch nothing (null pointers, bad sizes, small workspace)."""
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails its checks first
    rc = lib.vmk_spec_verify(None, fake, fake, fake, fake, 1, 8, 32, 8, 128, 100, 1, fake, 1 << 30, None)
    assert rc == 1 and b"null pointer" in lib.vmk_last_error()
    rc = lib.vmk_spec_verify(fake, fake, fake, fake, fake, 1, 40, 32, 8, 128, 100, 1, fake, 1 << 30, None)
    assert rc == 1 and b"words" in lib.vmk_last_error()
    rc = lib.vmk_spec_verify(fake, fake, fake, fake, fake, 1, 8, 32, 8, 128, 100, 1, fake, 16, None)
    assert rc == 1 and b"workspace too small" in lib.vmk_last_error()
    rc = lib.vmk_prefix_decode(fake, fake, fake, fake, fake, None, fake, 4, 32, 8, 128, 100, 10, 1, fake, 1 << 30,
                               None)
    assert rc == 1 and b"slens" in lib.vmk_last_error()
    rc = lib.vmk_decode(fake, fake, None, None, fake, 2, 32, 8, 128, 100, fake, 1 << 30, None)
    assert rc == 1 and b"null pointer" in lib.vmk_last_error()
    rc = lib.vmk_decode(fake, fake, fake, None, fake, 2, 32, 8, 128, 100, fake, 64, None)
    assert rc == 1 and b"workspace too small" in lib.vmk_last_error()
    rc = lib.vmk_prefix_decode_paged(fake, fake, fake, None, fake, None, fake, 4, 32, 8, 128, 100, 64, 128, 2, fake,
                                     1 << 30, None)
    assert rc == 1 and b"null pointer" in lib.vmk_last_error()
    rc = lib.vmk_prefix_decode_paged(fake, fake, fake, fake, fake, None, fake, 4, 32, 8, 128, 100, 48, 96, 2, fake,
                                     1 << 30, None)
    assert rc == 1 and b"page_size" in lib.vmk_last_error()
    rc = lib.vmk_prefix_decode_paged_nhd(fake, fake, fake, fake, fake, None, fake, 4, 32, 8, 128, 100, 48, 96, 2,
                                         fake, 1 << 30, None)
    assert rc == 1 and b"page_size" in lib.vmk_last_error()
    rc = lib.vmk_prefix_decode_paged_nhd(fake, fake, fake, fake, fake, None, fake, 4, 8192, 8192, 128, 100, 64, 128,
                                         2, fake, 1 << 30, None)
    assert rc == 1 and b"at most 4096 KV heads" in lib.vmk_last_error()
    # Paged decode: page size, heads per KV head and the workspace are checked before any launch.
    assert lib.vmk_decode_paged_workspace_size(4, 32, 8, 128, 48, 10) == 0
    assert lib.vmk_decode_paged_workspace_size(4, 32, 8, 128, 64, 10) > 0
    rc = lib.vmk_decode_paged(fake, fake, fake, fake, None, fake, 4, 32, 8, 128, 100, 48, 10, fake, 1 << 30, None)
    assert rc == 1 and b"page_size" in lib.vmk_last_error()
    rc = lib.vmk_decode_paged_nhd(fake, fake, fake, fake, None, fake, 4, 64, 2, 128, 100, 64, 10, fake, 1 << 30, None)
    assert rc == 1 and b"at most 16 query heads" in lib.vmk_last_error()
    rc = lib.vmk_decode_paged_bf16(fake, fake, fake, None, None, fake, 4, 32, 8, 128, 100, 64, 10, fake, 1 << 30,
                                   None)
    assert rc == 1 and b"null pointer" in lib.vmk_last_error()
    rc = lib.vmk_decode_paged(fake, fake, fake, fake, None, fake, 4, 32, 8, 128, 100, 64, 10, fake, 64, None)
    assert rc == 1 and b"workspace too small" in lib.vmk_last_error()
    rc = lib.vmk_dsa_decode(fake, fake, fake, fake, fake, None, fake, fake, fake, 2, 5000, fake, 1024, None)
    assert rc == 1 and b"workspace too small" in lib.vmk_last_error()
    rc = lib.vmk_dsa_decode(fake, fake, fake, fake, None, None, fake, fake, fake, 2, 5000, fake, 1 << 30, None)
    assert rc == 1 and b"null pointer" in lib.vmk_last_error()
    # The sparse attention addresses a request's latent rows by 32-bit offsets: L * 1152 bytes must stay < 2 GiB.
    big = 1864135
    ws = lib.vmk_dsa_workspace_size(1, big)
    assert ws > 0
    rc = lib.vmk_dsa_sparse_mla(fake, fake, fake, fake, fake, 1, big, fake, ws, None)
    assert rc == 1 and b"L <= 1864134" in lib.vmk_last_error()
    rc = lib.vmk_dsa_decode(fake, fake, fake, fake, fake, None, fake, fake, fake, 1, big, fake, ws, None)
    assert rc == 1 and b"L <= 1864134" in lib.vmk_last_error()


def test_python_wrappers_validate_shapes_without_gpu():
    import torch
    import vmk
    q = torch.zeros(2, 8, 32, 128, dtype=torch.float16)
    with pytest.raises(ValueError):   # CPU tensors are rejected before any device work
        vmk.spec_verify(q, torch.zeros(2, 8, 100, 128, dtype=torch.float16),
                        torch.zeros(2, 8, 100, 128, dtype=torch.float16), torch.zeros(2, 8, 1, dtype=torch.int32))
    with pytest.raises(TypeError):
        vmk.spec_verify(q.float(), q, q, q)
    # Paged prefix: the layout names the pool's shape, checked before the device.
    qp = torch.zeros(2, 32, 128, dtype=torch.float16)
    pool = torch.zeros(10, 8, 64, 128, dtype=torch.float16)                    # HND (num_pages, Hkv, ps, D)
    pp, sp = torch.zeros(2, dtype=torch.int32), torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="layout"):
        vmk.prefix_decode_paged(qp, pool, pool, pp, sp, layout="HDN")
    with pytest.raises(ValueError, match="expected"):
        vmk.prefix_decode_paged(qp, pool, pool[:, :4].contiguous(), pp, sp)
    nhd = pool.transpose(1, 2).contiguous()                                     # (num_pages, ps, Hkv, D)
    with pytest.raises(ValueError, match="ROCm device"):
        vmk.prefix_decode_paged(qp, nhd, nhd, pp, sp, layout="NHD")
    with pytest.raises(ValueError, match="expected"):
        vmk.prefix_decode_paged(qp, nhd, nhd[:, :32].contiguous(), pp, sp, layout="NHD")
    # Paged decode: the same layout rules.
    qd, table = torch.zeros(2, 32, 128, dtype=torch.float16), torch.zeros(2, 3, dtype=torch.int32)
    with pytest.raises(ValueError, match="layout"):
        vmk.decode_paged(qd, pool, pool, table, layout="nhd")
    with pytest.raises(ValueError, match="B rows"):
        vmk.decode_paged(qd, pool, pool, table[:1].contiguous())
    with pytest.raises(ValueError, match="ROCm device"):
        vmk.decode_paged(qd, nhd, nhd, table, layout="NHD")
    # A caller's out must have q's shape and dtype: the kernels write exactly that many rows.
    short, wrong = torch.zeros(1, 32, 128, dtype=torch.float16), torch.zeros(2, 32, 128, dtype=torch.bfloat16)
    kv = torch.zeros(2, 8, 100, 128, dtype=torch.float16)
    for bad, err in ((short, ValueError), (wrong, TypeError)):
        with pytest.raises(err, match="out"):
            vmk.decode(qd, kv, kv, out=bad)
        with pytest.raises(err, match="out"):
            vmk.decode_paged(qd, pool, pool, table, out=bad)
        with pytest.raises(err, match="out"):
            vmk.prefix_decode_paged(qp, pool, pool, pp, sp, out=bad)
        with pytest.raises(err, match="out"):
            vmk.prefix_decode(qp, kv[0], kv[0], kv, kv, out=bad)
    with pytest.raises(ValueError, match="out"):
        vmk.spec_verify(q, kv, kv, torch.zeros(2, 8, 1, dtype=torch.int32), out=q[:1].contiguous())


def test_bf16_reaches_the_bf16_entry_points():
    """bf16 inputs pass through the kernel modules to the _bf16 entry points (here: rejected as CPU tensors, after the
    dtype dispatch, DSA included); float32 q is rejected."""
    import torch
    import vmk
    import dsa_mi355x
    import spec_mi355x
    x = torch.zeros(1, 1, 32, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        spec_mi355x.kernel(x, x, x, torch.ones(1, 1, dtype=torch.int32))
    with pytest.raises(TypeError):
        vmk.decode(x[:, 0].float(), x, x)
    y = torch.zeros(1, 2100, 576, dtype=torch.bfloat16)
    iq, ik = torch.zeros(1, 64, 128, dtype=torch.bfloat16), torch.zeros(1, 2100, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        dsa_mi355x.kernel(y[:, :128], y, iq, ik, torch.zeros(1, 64), None)


def test_dsa_wrappers_check_every_shape_before_the_device():
    """Wrongly shaped DSA arguments are refused on the host (here CPU tensors, so nothing reaches a GPU): the
    attention's q/kv/idx/cnt and the indexer's lens length."""
    import torch
    import vmk
    B, L = 2, 3000
    f16 = dict(dtype=torch.float16)
    q, kv = torch.zeros(B, 128, 576, **f16), torch.zeros(B, L, 576, **f16)
    iq, ik, w = torch.zeros(B, 64, 128, **f16), torch.zeros(B, L, 128, **f16), torch.zeros(B, 64)
    idx, cnt = torch.zeros(B, 2048, dtype=torch.int32), torch.zeros(B, dtype=torch.int32)
    bad = [
        (vmk.dsa_sparse_mla, (torch.zeros(B, 128, 512, **f16), kv, idx, cnt), "q"),
        (vmk.dsa_sparse_mla, (q, torch.zeros(B, L, 512, **f16), idx, cnt), "kv"),
        (vmk.dsa_sparse_mla, (q, torch.zeros(B + 1, L, 576, **f16), idx, cnt), "kv"),
        (vmk.dsa_sparse_mla, (q, kv, torch.zeros(B, 1024, dtype=torch.int32), cnt), "idx"),
        (vmk.dsa_sparse_mla, (q, kv, idx, torch.zeros(B + 1, dtype=torch.int32)), "cnt"),
        (vmk.dsa_indexer_select, (iq, ik, w, torch.ones(B + 1, dtype=torch.int32)), "lens"),
        (vmk.dsa_indexer_select, (iq, torch.zeros(B, L, 64, **f16), w), "ik"),
        (vmk.dsa_decode, (q, torch.zeros(B, L + 1, 576, **f16), iq, ik, w), "positions"),
        (vmk.dsa_decode, (q, kv, iq, ik, w, torch.ones(1, dtype=torch.int32)), "lens"),
        (vmk.dsa_indexer, (iq, ik, w, None, torch.zeros(B, L + 1)), "scores"),
        (vmk.dsa_indexer, (iq, ik, torch.zeros(B, 63)), "w"),
        (vmk.dsa_topk, (torch.zeros(B, L), torch.ones(B + 1, dtype=torch.int32)), "lens"),
        (vmk.dsa_topk, (torch.zeros(B, L), None, torch.zeros(B, 2047, dtype=torch.int32), cnt), "idx"),
    ]
    for fn, args, needle in bad:
        with pytest.raises(ValueError, match=needle):
            fn(*args)
    with pytest.raises(ValueError, match="ROCm device"):        # well-formed: only the device check is left
        vmk.dsa_sparse_mla(q, kv, idx, cnt)
    with pytest.raises(TypeError, match="share one dtype"):
        vmk.dsa_decode(q, kv, iq.bfloat16(), ik.bfloat16(), w)
    with pytest.raises(TypeError, match="scores"):
        vmk.dsa_topk(torch.zeros(B, L, **f16))


def test_failed_call_sets_the_workspace_aside(monkeypatch):
    """A call that fails leaves the cached workspace out of use (the next call gets a fresh, zeroed one), and kept
    alive when the device then reports an error too.  Forced on the CPU by failing stand-ins for the library call and
    for the device drain, so the test means the same with or without a GPU."""
    import torch
    from vmk import api, lib
    buf = torch.zeros(16, dtype=torch.uint8)
    monkeypatch.setitem(api._ws, buf.device.index, buf)
    monkeypatch.setattr(api, "_retired", [])

    def fail(*a):
        raise lib.VmkError("launch failed")

    def drain_fails(key):
        raise RuntimeError("device error")
    monkeypatch.setattr(lib, "call", fail)
    monkeypatch.setattr(api, "_drain", drain_fails)
    with pytest.raises(lib.VmkError):
        api._launch("vmk_spec_verify", buf)
    assert buf.device.index not in api._ws and api._retired == [buf]


def _select_threshold(coarse, fine, need=2048):
    import ctypes
    from vmk import lib
    c = np.ascontiguousarray(coarse, dtype=np.uint32)
    f = np.ascontiguousarray(fine, dtype=np.uint32)
    out = np.zeros(3, dtype=np.uint32)
    lib.call("vmk_debug_select_threshold", c.ctypes.data_as(ctypes.c_void_p), f.ctypes.data_as(ctypes.c_void_p),
             need, out.ctypes.data_as(ctypes.c_void_p))
    return [int(x) for x in out]


def test_select_threshold_arithmetic_on_consistent_histograms():
    """The select kernels' bin arithmetic, replayed on the host: for histograms of real score keys the fine bucket
    holds the 2048th largest key, and the coarse result agrees with it."""
    rng = np.random.default_rng(3)
    for trial in range(40):
        n = int(rng.integers(2049, 200000))
        keys = rng.integers(0, 1 << 32, n, dtype=np.uint64) if trial % 2 else \
            (0x80000000 + rng.normal(0, 2 ** 24 * (1 + trial), n).astype(np.int64)).astype(np.uint64) % (1 << 32)
        fine = np.bincount((keys >> 19).astype(np.int64), minlength=8192).astype(np.uint32)
        coarse = fine.reshape(256, 32).sum(1).astype(np.uint32)
        c, rest, b1 = _select_threshold(coarse, fine)
        kth = np.sort(keys)[::-1][2047]
        assert b1 == int(kth >> 19) and c == b1 >> 5
        assert rest == 2048 - int(coarse[c + 1:].sum())


def test_select_threshold_stays_in_range_on_inconsistent_histograms():
    """An empty histogram, fewer than 2048 counts, coarse counts with no fine counts under them, and random garbage
    (sums that wrap): every bin returned lies inside the histograms, so the kernels never address outside them."""
    rng = np.random.default_rng(4)
    cases = [(np.zeros(256), np.zeros(8192)),
             (np.full(256, 7), np.zeros(8192)),
             (np.eye(1, 256, 200).ravel() * 5000, np.zeros(8192)),
             (np.zeros(256), np.full(8192, 9))]
    cases += [(rng.integers(0, 1 << 32, 256, dtype=np.uint64), rng.integers(0, 1 << 32, 8192, dtype=np.uint64))
              for _ in range(200)]
    cases += [(rng.integers(0, 40, 256), rng.integers(0, 3, 8192)) for _ in range(200)]
    for coarse, fine in cases:
        for need in (1, 2048, 0xFFFFFFFF):
            c, rest, b1 = _select_threshold(coarse, fine, need)
            assert 0 <= c < 256 and 0 <= b1 < 8192
    assert _select_threshold(np.zeros(256), np.zeros(8192)) == [0, 0, 0]


def test_noalloc_entry_point_refuses_oversized_shapes_without_a_gpu():
    """vmk_spec_verify_noalloc checks its arguments and its scratch limit before any HIP call, so a shape whose
    partials exceed the static scratch is refused here, on a machine without a GPU (dummy aligned pointers)."""
    from vmk import lib
    L = lib.load()
    assert L.vmk_spec_noalloc_max_bytes() == 32 << 20
    p = 1 << 20                                        # never dereferenced: the call is refused first
    rc = L.vmk_spec_verify_noalloc(p, p, p, p, p, 8, 64, 32, 8, 128, 64 << 20, 2, None)
    assert rc == 1 and b"static scratch" in L.vmk_last_error()
    rc = L.vmk_spec_verify_noalloc(p, p, p, p, p, 2, 64, 32, 8, 128, 65536, 1, None)   # wrong word count
    assert rc == 1 and b"ceil(kd/32)" in L.vmk_last_error()


def test_dsa_project_rejects_before_launch(lib):
    """The projections' host checks (weights struct, sizes, workspace) return 1 before anything is launched."""
    from vmk import lib as L
    assert lib.vmk_dsa_project_workspace_size(0) == 0
    assert lib.vmk_dsa_project_workspace_size(4) > (4 << 20)
    fake = ctypes.c_void_p(1 << 20)
    wts = L.DsaProjectWeights(*([1 << 20] * len(L.PROJECT_WEIGHT_FIELDS)))
    ws = lib.vmk_dsa_project_workspace_size(4)
    args = lambda wp, B, nbytes: (fake, fake, fake, fake, 64, wp, fake, fake, fake, fake, fake, B, 100, fake, nbytes,
                                  None)
    rc = lib.vmk_dsa_project(*args(None, 4, ws))
    assert rc == 1 and b"null weights" in lib.vmk_last_error()
    rc = lib.vmk_dsa_project(*args(ctypes.addressof(wts), 0, ws))
    assert rc == 1 and b"out of range" in lib.vmk_last_error()
    rc = lib.vmk_dsa_project(*args(ctypes.addressof(wts), 4, 1024))
    assert rc == 1 and b"workspace too small" in lib.vmk_last_error()
    wts.iw = None
    rc = lib.vmk_dsa_project_bf16(*args(ctypes.addressof(wts), 4, ws))
    assert rc == 1 and b"null weight pointer" in lib.vmk_last_error()


def test_dsa_project_wrapper_checks_shapes_without_gpu():
    import torch
    import vmk
    from vmk.ops import dsa_project as op
    pos = torch.zeros(2, dtype=torch.int32)
    cs = torch.zeros(16, 32)
    kv, ik = torch.zeros(2, 16, 576, dtype=torch.float16), torch.zeros(2, 16, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="7168"):
        vmk.dsa_project(torch.zeros(2, 100, dtype=torch.float16), pos, cs, cs, {}, kv, ik)
    x = torch.zeros(2, op.DIM, dtype=torch.float16)
    with pytest.raises(ValueError, match="weights must be a dict"):
        vmk.dsa_project(x, pos, cs, cs, {}, kv, ik)
    with pytest.raises(ValueError, match="rope tables"):
        vmk.dsa_project(x, pos, cs, torch.zeros(16, 31), {}, kv, ik)
