"""The workspace cache of vmk.api on the CPU: allocation, capture state and the device drain are stubbed, so the
rules themselves are checked without a GPU: geometric growth, outgrown buffers freed unless a graph was captured
over them, growth refused during capture, and a failed call setting its buffer aside only after a launch error."""
import pytest
import torch

from vmk import api, lib


@pytest.fixture
def cache(monkeypatch):
    state = dict(capturing=False, drains=0)
    monkeypatch.setattr(api, "_ws", {})
    monkeypatch.setattr(api, "_captured", set())
    monkeypatch.setattr(api, "_retired", [])
    monkeypatch.setattr(api, "_alloc", lambda n, key: torch.zeros(n, dtype=torch.uint8))
    monkeypatch.setattr(api, "_capturing", lambda: state["capturing"])

    def drain(key):
        state["drains"] += 1
    monkeypatch.setattr(api, "_drain", drain)
    monkeypatch.setattr(api, "_dev_index", lambda device: 0)
    return state


def test_growth_is_geometric_and_outgrown_buffers_are_freed(cache):
    a = api.workspace(100, "cuda:0")
    assert a.numel() == api.MIN_WORKSPACE
    assert api.workspace(api.MIN_WORKSPACE, "cuda:0") is a              # fits: same buffer
    sizes = []
    need = api.MIN_WORKSPACE
    for _ in range(40):                                                   # a cache that grows a little per call
        need += api.MIN_WORKSPACE // 4
        sizes.append(api.workspace(need, "cuda:0").numel())
    grown = sorted(set(sizes))
    assert all(b >= 2 * a for a, b in zip(grown, grown[1:]))              # each growth at least doubles
    assert len(grown) <= 4
    assert api._retired == []                                             # nothing captured: nothing retained
    assert cache["drains"] == len(grown)                                  # each outgrown buffer after a drain


def test_buffer_of_a_captured_graph_is_kept(cache):
    a = api.workspace(1 << 20, "cuda:0")
    cache["capturing"] = True
    assert api.workspace(1 << 19, "cuda:0") is a                          # a capture uses the current buffer
    with pytest.raises(lib.VmkError, match="during HIP graph capture"):
        api.workspace(4 << 20, "cuda:0")                                  # growth refused while capturing
    cache["capturing"] = False
    b = api.workspace(4 << 20, "cuda:0")
    assert b is not a and api._retired == [a]                             # the graph's buffer stays alive
    c = api.workspace(16 << 20, "cuda:0")
    assert c is not b and api._retired == [a]                             # b was never captured: freed


def test_failed_call_sets_aside_only_after_a_launch_error(cache, monkeypatch):
    class Dev:
        index = 0

    class Buf:
        device = Dev()
    buf = Buf()
    api._ws[0] = buf

    def fail(code):
        def call(name, *args):
            raise lib.VmkError("boom", code=code)
        return call
    monkeypatch.setattr(lib, "call", fail(lib.REJECTED))
    with pytest.raises(lib.VmkError):
        api._launch("vmk_x", buf)
    assert api._ws[0] is buf                                              # refused on the host: kept in use
    monkeypatch.setattr(lib, "call", fail(lib.LAUNCH_ERROR))
    with pytest.raises(lib.VmkError):
        api._launch("vmk_x", buf)
    assert 0 not in api._ws and api._retired == []                        # set aside and released after a drain
    assert cache["drains"] == 1
    assert api.workspace(1 << 20, "cuda:0") is not buf                    # the next call starts from a fresh one


def test_error_codes_are_kept():
    e = lib.VmkError("x", code=2)
    assert e.code == lib.LAUNCH_ERROR and isinstance(e, RuntimeError)
    assert lib.VmkError("y").code is None
