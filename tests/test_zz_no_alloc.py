"""The allocation-free spec entry point (vmk_spec_verify_noalloc, C-ABI through ctypes) against vmk_spec_verify on
the same inputs: the same kernels and plan, so the outputs must be bit-equal.  Two calls in a row, the second on a
smaller shape (the static scratch keeps the first call's partials), and then a third at the C4 size."""
import pytest
import torch

from vmk import lib
from vmk.ops import spec

pytestmark = pytest.mark.gpu


def call_noalloc(inp, out):
    q, k, v = inp["q"], inp["k"], inp["v"]
    words = spec.mask_words(inp["bits"], q.shape[1]).contiguous()
    B, kd, Hq, D = q.shape
    lib.call("vmk_spec_verify_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), words.data_ptr(), out.data_ptr(),
             B, kd, Hq, k.shape[1], D, k.shape[2], words.shape[2], torch.cuda.current_stream().cuda_stream)


def call_workspace(inp):
    import vmk
    q = inp["q"]
    return vmk.spec_verify(q, inp["k"], inp["v"], spec.mask_words(inp["bits"], q.shape[1]).contiguous())


@pytest.mark.parametrize("shapes", [[(dict(B=4, L=32768, k=8), "chain", 1), (dict(B=2, L=3000, k=5), "randn", 2),
                                     (dict(B=2, L=65536, k=64), "tree_bd", 3)]])
def test_noalloc_equals_workspace_entry_point(shapes):
    for shape, dist, seed in shapes:
        print(f"noalloc spec {shape} {dist} seed={seed}", flush=True)
        inp = spec.make_inputs(shape, seed=seed, dist=dist, device="cuda")
        out = torch.full_like(inp["q"], float("nan"))
        call_noalloc(inp, out)
        want = call_workspace(inp)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), shape


def test_noalloc_refuses_shapes_beyond_its_scratch():
    """A shape whose partials exceed the scratch is refused before anything is launched (the tensors are tiny: the
    call must not read them)."""
    x = torch.zeros(16, dtype=torch.float16, device="cuda")
    words = torch.zeros(16, dtype=torch.int32, device="cuda")
    L = 64 * 2 ** 20                                   # 16 splits x 256 items x 128 KiB of partials per 4096 keys
    with pytest.raises(lib.VmkError, match="static scratch"):
        lib.call("vmk_spec_verify_noalloc", x.data_ptr(), x.data_ptr(), x.data_ptr(), words.data_ptr(), x.data_ptr(),
                 8, 64, 32, 8, 128, L, 2, torch.cuda.current_stream().cuda_stream)


def test_noalloc_on_a_side_stream():
    """The scratch is looked up for the device of the stream the call is launched on (here a non-default stream
    of the current GPU), through the Python wrapper, and gives the same bits as the workspace entry point."""
    import vmk
    inp = spec.make_inputs(dict(B=2, L=5000, k=8), seed=4, dist="chain", device="cuda")
    words = spec.mask_words(inp["bits"], 8).contiguous()
    want = call_workspace(inp)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = torch.full_like(inp["q"], float("nan"))
        vmk.spec_verify_noalloc(inp["q"], inp["k"], inp["v"], words, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
