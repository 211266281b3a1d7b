"""libvmk calls under HIP graph capture: every op's launches (no allocation and no memset inside them once the
workspace is cached) are captured with torch.cuda.graph and replayed several times, with eager work and
synchronisation between the replays; every replay must reproduce the eager output bit for bit."""
import pytest
import torch

from vmk.ops import KEYS, decode, decode_paged, dsa, prefix, prefix_paged, spec

pytestmark = pytest.mark.gpu

CASES = [("spec", spec, dict(B=3, L=5000, k=8), "chain"), ("spec", spec, dict(B=2, L=8192, k=64), "tree_bd"),
         ("decode", decode, dict(B=4, L=9000, L_min=1), "randn"),
         ("decode_paged", decode_paged, dict(B=4, L=9000, L_min=1, ps=64, absent=1, layout="NHD"), "randn"),
         ("prefix", prefix, dict(N=8, P=2048, S=256, S_min=1), "randn"),               # mixed launch + merge
         ("prefix", prefix, dict(N=64, P=4096, S=1024, S_min=128), "outlier"),        # prefix launch, fused suffix
         ("prefix", prefix, dict(N=20, P=3000, S=2500, S_min=1), "randn"),            # combine launch
         ("prefix_paged", prefix_paged, dict(N=40, P=2048, S=300, S_min=1, ps=64, absent=2), "randn"),
         ("prefix_paged", prefix_paged, dict(N=12, P=1024, S=700, S_min=1, ps=128, absent=1, layout="NHD"),
          "randn"),
         ("dsa", dsa, dict(B=3, L=9000), "randn"), ("dsa", dsa, dict(B=2, L=1500), "randn")]


def kernel_of(opname):
    mod = __import__(f"{opname}_mi355x")
    return mod.kernel


@pytest.mark.parametrize("opname,op,shape,dist", CASES)
def test_graph_replays_equal_eager(opname, op, shape, dist):
    print(f"graph {opname} {shape} {dist}", flush=True)
    kern = kernel_of(opname)
    inps = [{k: v for k, v in op.make_inputs(shape, seed=s, dist=dist, device="cuda").items() if k in KEYS[opname]}
            for s in (60, 61)]
    eager = [kern(**i).clone() for i in inps]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in inps:
            kern(**i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [kern(**i) for i in inps]
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), rep
        kern(**inps[rep % 2])                           # eager work between replays
        torch.cuda.synchronize()


def test_graph_replays_equal_eager_dsa_project():
    """The DSA projections (two launches) under capture: q, iq, w and the cache rows they write, every replay."""
    import vmk
    from vmk.ops import dsa_project as op
    print("graph dsa_project B=5 and B=40", flush=True)
    inps = [op.make_inputs(dict(B=B, L=300), seed=s, device="cuda") for B, s in ((5, 60), (40, 61))]

    def run(i):
        return vmk.dsa_project(i["x"], i["pos"], i["rope_cos"], i["rope_sin"], i["weights"], i["kv"], i["ik"])

    def rows(i):
        b, p = torch.arange(i["x"].shape[0], device="cuda"), i["pos"].long()
        return i["kv"][b, p].clone(), i["ik"][b, p].clone()

    eager = [tuple(t.clone() for t in run(i)) + rows(i) for i in inps]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in inps:
            run(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [run(i) for i in inps]
    for rep in range(4):
        for i in inps:                                  # the rows are rewritten by every replay
            i["kv"].zero_()
            i["ik"].zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, i, e in zip(outs, inps, eager):
            for got, want in zip(tuple(o) + rows(i), e):
                assert torch.equal(got, want), rep
        run(inps[rep % 2])                              # eager work between replays
        torch.cuda.synchronize()
