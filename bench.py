"""Benchmark of the attention ops on one MI355X, in the driver's contract.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs C1,C2,...] [--no-cpu] [--ab-rounds R]
                    [--results DIR]

Prints human-readable progress on stderr and ONE short JSON line (a few KB) on stdout.  A "step" is one call of the
op on one batch of the headline configuration, C4 (tree verification, B=2, k=64, L=65536): BASELINE.json's metric
names no configuration, so the headline is the largest configuration that fits one GPU (C4, 539 MB and 137 GFLOP
per call).  `value` is its achieved HBM throughput (algorithmic bytes / time per call, inputs resident in HBM);
`roofline` is the dominant kernel's HBM fraction, with its MFMA fraction beside it since C4 sits near the ridge;
`ops` maps every configuration to [us/call, GB/s, % of 8 TB/s] (C1..C5, and this build's D1-D3 decode, P2/P2n
paged prefix in HND/NHD pages, D1p/D2n paged decode in HND/NHD pages, C2b bf16, DP the DSA input projections);
`ab` holds the per-op geomean speedups over the torch standard ops.  The full per-configuration rows and every A/B
sample go to DIR/bench_full.json and DIR/bench_<op>.json (DIR defaults to ./results), as the reference keeps its
per-shape detail in results/bench_<op>.json.
Method:
  * the kernel's output on the timed inputs is checked against the PyTorch standard op first
    (allclose atol=rtol=1e-2, bench.py:180-192 of the reference), and the inputs are checked for modification;
  * every call reads a different input set, rotating over enough distinct sets (>= 1 GiB in total) that the
    256 MB Infinity Cache cannot serve a repeat;
  * W untimed warm-up calls, then the per-call time: the K calls captured once in a HIP graph, replayed 15 times,
    each replay between two HIP events (synchronised before and after); the median is `us_per_call`, with p10/p90.
    Before timing, 3 replays are checked bit for bit against an eager call.  Then `eager` gives the same K calls
    launched one by one from Python, which adds the host's per-call overhead;
  * the dominant kernel of each op is bracketed by its own pair of HIP events on its launch stream inside that eager
    loop (libvmk's vmk_profile_next hook), which gives the roofline figure; the loop runs after the graph replays, in
    the steady state (a power-bound op's first calls after a short warm-up vary by +-25 %);
  * A/B against the torch standard ops (the reference's headline form, bench.py:99-126, 157-236): each kernel
    module is screened by the verifier's static gate before it is imported (reference bench.py:159-161); on the
    reference's BENCH_SHAPES and on this build's configurations, the output is checked against the standard op
    and the inputs for modification (reference bench.py:180-192), then the kernel module and every TORCH_REFS op
    each time a 16-call chain (each call's query is the previous call's output; DSA: [output | rope part of q])
    after a 1 GiB cache flush, in R shuffled rounds; reported: medians with p10/p90, and the median over rounds
    of t(strongest op) / t(kernel), with its p10/p90, and the geomean over BENCH_SHAPES.
The CPU baseline is the float64 NumPy oracle (oracle/) on the host, on a bounded sample of the same workload, the
median of 3 runs.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "verified-metal-kernels_amd")
for _p in (ROOT, PKG, os.path.join(PKG, "kernels")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_FP16_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
METRIC = "µs/call per op + achieved HBM GB/s (% of MI355X peak) at bench shapes"
HEADLINE = "C4"
DOMINANT = {"prefix": "prefix_partial", "spec": "spec_partial", "dsa": "dsa_indexer", "decode": "spec_partial",
            "prefix_paged": "prefix_partial", "dsa_project": "dsa_project_q", "decode_paged": "spec_partial"}
# Configurations whose dominant bracket is another kernel: C5s runs the DSA decode as one launch (the whole op).
DOMINANT_CFG = {"C5s": "dsa_single"}
# Inputs the ops write by contract (the projections append the new token's cache rows), left out of the
# input-mutation check.
WRITES = {"dsa_project": ("kv", "ik")}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def op_module(opname):
    from vmk.ops import OPS, dsa_project
    return dsa_project if opname == "dsa_project" else OPS[opname]


def config_table():
    from vmk.ops import decode, decode_paged, dsa, dsa_project, prefix, prefix_paged, spec
    return [("C1", "prefix", *prefix.CONFIGS["C1"]), ("C2", "prefix", *prefix.CONFIGS["C2"]),
            ("C3", "spec", *spec.CONFIGS["C3"]), ("C4", "spec", *spec.CONFIGS["C4"]),
            ("C5", "dsa", *dsa.CONFIGS["C5"]), ("C5s", "dsa", dict(dsa.CONFIGS["C5"][0], single=1), "randn"),
            ("D1", "decode", *decode.CONFIGS["D1"]), ("D2", "decode", *decode.CONFIGS["D2"]),
            ("D3", "decode", *decode.CONFIGS["D3"]), ("P2", "prefix_paged", *prefix_paged.CONFIGS["P2"]),
            ("P2n", "prefix_paged", *prefix_paged.CONFIGS["P2n"]),
            ("D1p", "decode_paged", *decode_paged.CONFIGS["D1p"]), ("D2n", "decode_paged", *decode_paged.CONFIGS["D2n"]),
            ("C2b", "prefix", *prefix.CONFIGS["C2b"]), ("DP", "dsa_project", *dsa_project.CONFIGS["DP"])]


class HipEvents:
    """Raw HIP events (libamdhip64 through ctypes) for the per-kernel brackets recorded inside libvmk.  They are
    created with hipEventDisableSystemFence: a timing-only event then skips the system-scope cache writeback and
    invalidation on recording, which would otherwise land inside the bracket (the elapsed times are read only after
    a device synchronisation)."""
    DISABLE_SYSTEM_FENCE = 0x20000000           # hipEventDisableSystemFence of hip_runtime_api.h

    def __init__(self, n):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.ev = []
        for _ in range(2 * n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreateWithFlags(ctypes.byref(e), ctypes.c_uint(self.DISABLE_SYSTEM_FENCE)) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.ev.append(e)

    def pair(self, i):
        return self.ev[2 * i], self.ev[2 * i + 1]

    def elapsed_ms(self, i):
        import ctypes
        ms = ctypes.c_float()
        a, b = self.pair(i)
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed: an event of the pair was not recorded")
        return ms.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def call_op(opname, inp):
    import vmk
    if opname == "prefix":
        return vmk.prefix_decode(inp["q"], inp["kp"], inp["vp"], inp["ks"], inp["vs"], inp.get("slens"))
    if opname == "spec":
        return vmk.spec_verify(inp["q"], inp["k"], inp["v"], inp["words"])
    if opname == "decode":
        return vmk.decode(inp["q"], inp["k"], inp["v"], inp.get("lens"))
    if opname == "decode_paged":
        return vmk.decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["page_table"], inp.get("lens"),
                                layout=inp.get("layout", "HND"))
    if opname == "prefix_paged":
        return vmk.prefix_decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["prefix_pages"],
                                       inp["suffix_pages"], inp.get("slens"), layout=inp.get("layout", "HND"))
    if opname == "dsa_project":                           # q stands for the three outputs in the checks
        return vmk.dsa_project(inp["x"], inp["pos"], inp["rope_cos"], inp["rope_sin"], inp["weights"], inp["kv"],
                               inp["ik"])[0]
    return vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp.get("lens"),
                          single=bool(inp.get("single")))


def std_op(opname, inp):
    """The PyTorch standard op used by the reference's output check (L1_REF of each op)."""
    from vmk.ops import decode, dsa, prefix, prefix_paged, spec
    if opname == "prefix":
        return prefix.torch_naive(**{k: inp[k] for k in ("q", "kp", "vp", "ks", "vs", "slens")})
    if opname == "prefix_paged":
        return prefix_paged.torch_naive(**inp)
    if opname == "spec":
        return spec.torch_sdpa(inp["q"], inp["k"], inp["v"], inp["bits"])
    if opname == "decode":
        return decode.torch_sdpa(inp["q"], inp["k"], inp["v"], inp.get("lens"))
    if opname == "decode_paged":
        from vmk.ops import decode_paged
        return decode_paged.torch_sdpa(**inp)
    if opname == "dsa_project":
        from vmk.ops import dsa_project
        return dsa_project.torch_ref(inp["x"], inp["pos"], inp["rope_cos"], inp["rope_sin"], inp["weights"])[0]
    return dsa.torch_fp32_ref(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp.get("lens"))


def op_bytes_flops(opname, shape, inp_host):
    from vmk.ops import decode, decode_paged, dsa, dsa_project, prefix, prefix_paged, spec
    if opname == "dsa_project":   # dominant: the heads launch (Wq_b, Wiq_b, W_uk against cq; q and iq out)
        m = dsa_project
        total = m.algorithmic_bytes(shape)
        B = shape["B"]
        q_rows = m.H * (m.DN + m.DR) + m.HI * m.DI
        dom = (q_rows * m.QL + m.H * m.DC * m.DN) * 2 + B * m.QL * 2 + B * (m.H * (m.DC + m.DR) + m.HI * m.DI) * 2
        return total, dom, m.flops(shape)
    if opname == "prefix_paged":
        sl = None if inp_host.get("slens") is None else inp_host["slens"].numpy()
        total = prefix_paged.algorithmic_bytes(shape, sl)
        out = shape["N"] * prefix.HQ * prefix.D * 2
        return total, total - out, prefix_paged.flops(shape, sl)
    if opname == "prefix":
        sl = None if inp_host.get("slens") is None else inp_host["slens"].numpy()
        total = prefix.algorithmic_bytes(shape, sl)
        out = shape["N"] * prefix.HQ * prefix.D * 2
        return total, total - out, prefix.flops(shape, sl)
    if opname == "spec":
        total = spec.algorithmic_bytes(shape)
        out = shape["B"] * shape["k"] * spec.HQ * spec.D * 2
        return total, total - out, spec.flops(shape)
    if opname in ("decode", "decode_paged"):
        m = decode if opname == "decode" else decode_paged
        ln = None if inp_host.get("lens") is None else inp_host["lens"].numpy()
        total = m.algorithmic_bytes(shape, ln)
        out = shape["B"] * decode.HQ * decode.D * 2
        return total, total - out, m.flops(shape, ln)
    total = dsa.algorithmic_bytes(shape)
    B, L = shape["B"], shape["L"]
    indexer = B * L * dsa.DI * 2 + B * dsa.HI * dsa.DI * 2 + B * dsa.HI * 4    # ik + iq + w
    return total, indexer, dsa.flops(shape)


def distinct_sets(opname, inp0, total_bytes, count=None):
    """Extra input sets with the same shapes and dtypes (synthetic N(0,1) data made on the GPU), so that the calls
    of the timed loop rotate over >= 1 GiB of inputs (or `count` sets in all); masks/lengths are shared."""
    import torch
    n = count or max(2, int(math.ceil((1 << 30) / max(total_bytes, 1))))
    sets = [inp0]
    big = {"prefix": ("q", "kp", "vp", "ks", "vs"), "spec": ("q", "k", "v"), "dsa": ("q", "kv", "iq", "ik"),
           "decode": ("q", "k", "v"), "prefix_paged": ("q", "k_pages", "v_pages"), "dsa_project": (),
           "decode_paged": ("q", "k_pages", "v_pages")}[opname]
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    if opname == "dsa_project":                            # fresh weights (N(0, 1/fan_in)) and hidden states
        from vmk.ops import dsa_project
        for _ in range(n - 1):
            s = dict(inp0, weights=dict(inp0["weights"]))
            s["x"] = torch.randn(inp0["x"].shape, device="cuda", generator=g).to(inp0["x"].dtype)
            for k, w in inp0["weights"].items():
                if k not in dsa_project.NORMS:
                    s["weights"][k] = (torch.randn(w.shape, device="cuda", generator=g) * w.shape[-1] ** -0.5).to(w.dtype)
            sets.append(s)
        return sets
    for _ in range(n - 1):
        s = dict(inp0)
        for k in big:
            s[k] = torch.randn(inp0[k].shape, device="cuda", generator=g, dtype=torch.float32).to(inp0[k].dtype)
        sets.append(s)
    return sets


def cpu_baseline(opname, shape, dist, inp_host, total_bytes, runs=3):
    """Times the float64 oracle on a bounded sample of the workload on the host cores: the median of `runs` runs
    (one when a run exceeds 60 s), scaled from the sample to a whole call; returns a dict."""
    import oracle
    host_cpus = os.cpu_count() or 1
    try:
        from threadpoolctl import threadpool_limits, threadpool_info
        cores = min(16, host_cpus)          # the GPU box's CPU share for one GPU
        ctx = threadpool_limits(limits=cores)
        blas = [d.get("num_threads") for d in threadpool_info() if d.get("user_api") == "blas"]
    except Exception:  # pragma: no cover - threadpoolctl missing
        import contextlib
        ctx, cores, blas = contextlib.nullcontext(), host_cpus, []
    sl = lambda x, n: None if x is None else x[:n]
    if opname == "dsa_project":
        work = lambda: oracle.dsa_project.ref64(inp_host["x"], inp_host["pos"], inp_host["rope_cos"],
                                                inp_host["rope_sin"], **inp_host["weights"])
        scale, sample = 1, f"the whole call ({shape['B']} tokens)"
    elif opname == "prefix":
        N = shape["N"]
        ns = min(N, 8)
        sub = {k: inp_host[k][:ns] for k in ("q", "ks", "vs")}
        sub.update(kp=inp_host["kp"], vp=inp_host["vp"], slens=sl(inp_host.get("slens"), ns))
        work, scale = (lambda: oracle.prefix.ref64(**sub)), N / ns
        sample = f"requests 0-{ns - 1} of {N}, time scaled x{N / ns:g}"
    elif opname == "spec":
        B = shape["B"]
        work = lambda: oracle.spec.ref64(inp_host["q"][:1], inp_host["k"][:1], inp_host["v"][:1], inp_host["bits"][:1])
        scale, sample = B, f"batch 0 of {B}, time scaled x{B}"
    elif opname == "prefix_paged":
        N = shape["N"]
        ns = min(N, 8)
        sub = dict(inp_host, q=inp_host["q"][:ns], suffix_pages=inp_host["suffix_pages"][:ns],
                   slens=sl(inp_host.get("slens"), ns))
        work, scale = (lambda: oracle.prefix_paged.ref64(**sub)), N / ns
        sample = f"requests 0-{ns - 1} of {N}, time scaled x{N / ns:g}"
    elif opname == "decode":
        B = shape["B"]
        work = lambda: oracle.decode.ref64(inp_host["q"][:1], inp_host["k"][:1], inp_host["v"][:1],
                                           sl(inp_host.get("lens"), 1))
        scale, sample = B, f"request 0 of {B}, time scaled x{B}"
    elif opname == "decode_paged":
        B = shape["B"]
        sub = dict(inp_host, q=inp_host["q"][:1], page_table=inp_host["page_table"][:1],
                   lens=sl(inp_host.get("lens"), 1))
        work, scale = (lambda: oracle.decode_paged.ref64(**sub)), B
        sample = f"request 0 of {B}, time scaled x{B}"
    else:
        B = shape["B"]
        work = lambda: oracle.dsa.ref64(inp_host["q"][:1], inp_host["kv"][:1], inp_host["iq"][:1],
                                        inp_host["ik"][:1], inp_host["w"][:1], None)
        scale, sample = B, f"request 0 of {B} (scores, top-2048, attention), time scaled x{B}"
    times = []
    with ctx:
        for _ in range(runs):
            t0 = time.perf_counter()
            work()
            times.append(time.perf_counter() - t0)
            if times[-1] > 60:
                break
    dt = float(np.median(times)) * scale
    return dict(value=round(total_bytes / dt / 1e9, 3), unit="GB/s", us_per_call=round(dt * 1e6, 1), cores=cores,
                host_cpu_count=host_cpus, blas_threads=blas, runs=len(times), kind="port",
                sample=f"{sample}; median of {len(times)} runs")


def bench_config(name, opname, shape, dist, steps, warmup, do_cpu):
    import torch
    import vmk
    from vmk import lib
    op = op_module(opname)
    log(f"[{name}] {opname} {shape} {dist}: generating inputs")
    host = op.make_inputs(shape, seed=0, dist=dist)
    to_gpu = lambda v: v.cuda() if isinstance(v, torch.Tensor) else ({k: to_gpu(x) for k, x in v.items()}
                                                                     if isinstance(v, dict) else v)
    inp0 = {k: to_gpu(v) for k, v in host.items()}
    if opname == "spec":
        inp0["words"] = op.mask_words(inp0["bits"], shape["k"]).contiguous()
    if shape.get("single"):
        inp0["single"] = True
    dom_kernel = DOMINANT_CFG.get(name, DOMINANT[opname])
    total_bytes, dom_bytes, flops = op_bytes_flops(opname, shape, host)
    # FLOPs inside the dominant bracket: all of them for the attention ops, the score GEMM for DSA's indexer.
    dom_flops = {"dsa": lambda: 2 * shape["B"] * shape["L"] * op.HI * op.DI, "dsa_project": lambda: None}.get(
        opname, lambda: flops)()
    if name in DOMINANT_CFG:                       # the bracket is the whole op
        dom_bytes, dom_flops = total_bytes, flops
    # Output check on the benchmark inputs and input-mutation check (reference bench.py:180-192).
    snap = {k: v.clone() for k, v in inp0.items() if isinstance(v, torch.Tensor) and k not in WRITES.get(opname, ())}
    out = call_op(opname, inp0)
    torch.cuda.synchronize()
    mutated = [k for k, v in snap.items() if not torch.equal(v.view(torch.uint8), inp0[k].view(torch.uint8))]  # bits
    ref = std_op(opname, inp0)
    torch.cuda.synchronize()
    ok = (not mutated) and out.shape == ref.shape and bool(
        torch.allclose(out.float(), ref.float(), atol=1e-2, rtol=1e-2, equal_nan=True))
    del snap, ref
    if not ok:
        raise SystemExit(f"{name}: kernel output differs from the standard op on the benchmark inputs"
                         + (f" (inputs modified: {mutated})" if mutated else ""))
    sets = distinct_sets(opname, inp0, total_bytes)
    for i in range(warmup):
        call_op(opname, sets[i % len(sets)])
    torch.cuda.synchronize()
    gt = graph_us_per_call(opname, sets, steps)
    # The eager loop with the dominant bracket runs after the graph replays: right after a short warm-up, a
    # power-bound op's first eager calls still vary by +-25 % (C4: 149-240 us against 163-172 once settled).
    kid = lib.KERNEL_IDS[dom_kernel]
    hev = HipEvents(steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    L = lib.load()
    torch.cuda.synchronize()
    e0.record()
    for i in range(steps):
        L.vmk_profile_next(*hev.pair(i), kid)
        call_op(opname, sets[i % len(sets)])
    e1.record()
    torch.cuda.synchronize()
    eager_us = e0.elapsed_time(e1) * 1e3 / steps
    dom_us = sum(hev.elapsed_ms(i) for i in range(steps)) * 1e3 / steps
    hev.close()
    us = gt["median"]
    gbs = total_bytes / us / 1e3
    dom_gbs = dom_bytes / dom_us / 1e3
    row = dict(op=opname, shape=shape, dist=dist, us_per_call=round(us, 2),
               us_spread=dict(p10=round(gt["p10"], 2), p90=round(gt["p90"], 2), replays=gt["n"]), gbs=round(gbs, 1),
               pct_peak=round(100 * gbs / PEAK_HBM_GBS, 2), algorithmic_bytes=int(total_bytes),
               tflops=round(flops / us / 1e6, 2), mfma_pct=round(100 * flops / us / 1e6 / PEAK_FP16_TFLOPS, 2),
               eager=dict(us_per_call=round(eager_us, 2), gbs=round(total_bytes / eager_us / 1e3, 1)),
               dominant=dict(kernel=dom_kernel, us=round(dom_us, 2), bytes=int(dom_bytes),
                             gbs=round(dom_gbs, 1), frac=round(dom_gbs / PEAK_HBM_GBS, 4),
                             tflops=round(dom_flops / dom_us / 1e6, 2) if dom_flops else None,
                             sq=measured_mfma(name, dom_kernel)),
               output_check="ok", distinct_input_sets=len(sets))
    if opname not in AB_OPS:                               # no reference A/B for this op: its torch form, graph-timed
        ts = graph_us_per_call(opname, sets, steps, fn=lambda s: std_op(opname, s), check=False)
        row["vs_torch"] = dict(torch_us_per_call=round(ts["median"], 2), speedup=round(ts["median"] / us, 2))
    row["dominant"]["traffic"] = measured_traffic(name, row["dominant"])
    log(f"[{name}] {us:9.2f} us/call (p10 {gt['p10']:.2f}, p90 {gt['p90']:.2f})  {gbs:7.1f} GB/s "
        f"({row['pct_peak']:.1f}% of 8 TB/s)  [median of {gt['n']} replays of a HIP graph of {steps} calls; "
        f"eager loop {eager_us:.2f} us/call]   dominant {dom_kernel} {dom_us:.2f} us = {dom_gbs:.0f} GB/s")
    if do_cpu and name not in DOMINANT_CFG:        # C5s is C5's workload: its CPU baseline is C5's
        row["cpu_baseline"] = cpu_baseline(opname, shape, dist, host, total_bytes)
        log(f"[{name}] CPU float64 oracle: {row['cpu_baseline']['us_per_call']:.0f} us/call "
            f"({row['cpu_baseline']['sample']}, {row['cpu_baseline']['cores']} cores)")
    del sets, inp0, host
    torch.cuda.empty_cache()
    return row


def graph_us_per_call(opname, sets, steps, replays=15, fn=None, check=True):
    """µs per call of the K calls captured once in a HIP graph (torch.cuda.CUDAGraph over the calls' launches on the
    capture stream, rotating over the same input sets), each replay timed between two events and synchronised:
    the GPU time of K steps without the Python and launch overhead of an eager loop, which dominates ops of a few
    µs.  Returns the median, p10 and p90 over `replays` replays.  Before timing, the output of the last captured call
    after each of 3 replays (with eager work and synchronisation in between) must equal an eager call on the same
    inputs bit for bit.  `fn(set)` replaces the op's call (then `check` may turn the bit comparison off)."""
    import torch
    call = fn or (lambda s: call_op(opname, s))
    n = steps
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            call(sets[i % len(sets)])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [call(sets[i % len(sets)]) for i in range(n)]
    last = outs[-1]
    ref = call(sets[(n - 1) % len(sets)]).clone()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        if check and not torch.equal(last.view(torch.int16), ref.view(torch.int16)):
            raise SystemExit(f"{opname}: a graph replay differs from the eager call")
        call(sets[0])                                     # eager work between replays
        torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / n)
    del g, outs
    return spread(times)


def spread(xs):
    """median, p10 and p90 of a list of timings (nearest-rank percentiles), and how many there are."""
    t = sorted(xs)
    rank = lambda p: t[min(len(t) - 1, max(0, int(math.ceil(p * len(t))) - 1))]
    return dict(median=float(np.median(t)), p10=rank(0.1), p90=rank(0.9), n=len(t))


# ------------------------------------------------------------------------------------------------ A/B vs torch
# The reference's benchmark scores a kernel by its speedup over the strongest standard op, interleaved in shuffled
# rounds (reference bench.py:99-126, 157-236).  Here the standard ops are the op contracts' PyTorch-ROCm
# compositions (TORCH_REFS), on the reference's BENCH_SHAPES and on this build's configurations.
AB_OPS = ("prefix", "spec", "dsa")


class CacheFlush:
    """Writes 1 GiB before each timed chain, which evicts the 256 MB Infinity Cache and every L2."""

    def __init__(self):
        import torch
        self.buf = torch.empty(1 << 28, dtype=torch.float32, device="cuda")

    def __call__(self):
        self.buf.fill_(1.0)


def ab_chain(opname):
    """How a chain layer's output becomes the next layer's query: the output itself (prefix, spec: same shape as
    q), or [output | the layer's rope part of q] for DSA (ops/dsa.py:145-147, chain_torch)."""
    from vmk.ops import dsa
    return dsa.chain_torch if opname == "dsa" else (lambda out, kw: out)


def ab_inputs(op, shape, dist, keys):
    """Input sets on the GPU for one shape: set 0 from the op's seeded generator, the others N(0,1) of the same
    shapes made on the GPU (masks and lengths shared), as many as make about 1.5 GiB of distinct kernel inputs
    (1 to 8, as the reference's bench.py:171-175); prefix sets also carry the standard ops' cache layouts (kf/vf,
    ku/vu), built outside the timed region as the reference's generator builds them."""
    import torch
    host = op.make_inputs(shape, seed=0, dist=dist)
    if op.NAME == "dsa":
        host["lens"] = None                           # the reference benchmarks full caches (bench.py:177-178)
    s0 = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in host.items()}
    per_set = sum(v.numel() * v.element_size() for k, v in s0.items() if isinstance(v, torch.Tensor) and k in keys)
    n = int(max(1, min(8, (3 << 29) // max(per_set, 1))))
    sets = distinct_sets(op.NAME, s0, 0, count=n)
    if op.NAME == "prefix":
        for st in sets:
            st.update(op.build_layouts(st["kp"], st["vp"], st["ks"], st["vs"]))
    return sets


def ab_runner(fn, layers, chain, flush):
    """A timed chain: flush, then every layer's call with q taken from the previous layer's output, between two
    events; returns µs per call."""
    import torch

    def run():
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        q = layers[0]["q"]
        e0.record()
        for kw in layers:
            kw = dict(kw, q=q)
            q = chain(fn(**kw), kw)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / len(layers)
    return run


def screened_module(opname):
    """The op's kernel module, imported only after its source passes the verifier's static gate (the reference
    screens a module before importing it, bench.py:159-161); a refused module ends the benchmark."""
    import importlib
    tests = os.path.join(ROOT, "tests")
    if tests not in sys.path:
        sys.path.insert(0, tests)
    from verify import screen
    path = os.path.join(PKG, "kernels", f"{opname}_mi355x.py")
    with open(path) as f:
        problems = screen(f.read())
    if problems:
        raise SystemExit(f"A/B {opname}: {path} fails the static gate: " + "; ".join(problems))
    return importlib.import_module(f"{opname}_mi355x")


def ab_shape(op, shape, dist, rounds, flush, seed):
    """One shape: output and input-mutation check, then `rounds` shuffled rounds of the kernel module and every
    standard op."""
    import random
    import torch
    from vmk.ops import KEYS
    mod = screened_module(op.NAME)
    keys = KEYS[op.NAME]
    kernel = lambda **kw: mod.kernel(**{k: kw.get(k) for k in keys})
    sets = ab_inputs(op, shape, dist, keys)
    n = len(sets)
    layers = [sets[i % n] for i in range(max(16, n))]
    std = getattr(op, op.L1_REF)
    snap = {k: v.clone() for k, v in sets[0].items() if k in keys and isinstance(v, torch.Tensor)}
    out = kernel(**sets[0])
    torch.cuda.synchronize()
    mutated = [k for k, v in snap.items() if not torch.equal(v.view(torch.uint8), sets[0][k].view(torch.uint8))]
    del snap
    if mutated:
        raise SystemExit(f"A/B {op.NAME} {shape}: the kernel modified its inputs {mutated}")
    ref = std(**sets[0])
    torch.cuda.synchronize()
    if not torch.allclose(out.float(), ref.float(), atol=1e-2, rtol=1e-2, equal_nan=True):
        raise SystemExit(f"A/B {op.NAME} {shape}: the kernel differs from {op.L1_REF} on the benchmark inputs")
    del out, ref
    chain = ab_chain(op.NAME)
    runners = {"kernel": ab_runner(kernel, layers, chain, flush)}
    runners.update({name: ab_runner(f, layers, chain, flush) for name, f in op.TORCH_REFS.items()})
    for r in runners.values():                        # warm-up: compile paths, allocator, clocks
        r()
    rng = random.Random(seed)
    times = {name: [] for name in runners}
    for _ in range(rounds):
        order = list(runners)
        rng.shuffle(order)
        for name in order:
            times[name].append(runners[name]())
    refs = [k for k in runners if k != "kernel"]
    med = {k: spread(v) for k, v in times.items()}
    strongest = min(refs, key=lambda k: med[k]["median"])
    ratios = {k: spread([b / a for a, b in zip(times["kernel"], times[k])]) for k in refs}
    del sets, layers, runners
    torch.cuda.empty_cache()
    return dict(shape=shape, dist=dist, distinct_sets=n, chain=max(16, n), input_check="unmodified",
                median_us={k: round(v["median"], 2) for k, v in med.items()},
                p10_us={k: round(v["p10"], 2) for k, v in med.items()},
                p90_us={k: round(v["p90"], 2) for k, v in med.items()},
                strongest_ref=strongest, speedup_vs_strongest_ref=round(ratios[strongest]["median"], 3),
                speedup_p10=round(ratios[strongest]["p10"], 3), speedup_p90=round(ratios[strongest]["p90"], 3),
                speedup_vs_each_ref={k: round(v["median"], 3) for k, v in ratios.items()},
                samples_us={k: [round(t, 3) for t in v] for k, v in times.items()})


def ab_bench(rounds, configs):
    """The A/B table: per op, every BENCH_SHAPE (geomean of the speedups, as the reference publishes) and every
    configuration of this build that belongs to the op."""
    from vmk.ops import OPS
    flush = CacheFlush()
    res = {}
    for opname in AB_OPS:
        op = OPS[opname]
        shapes = [(None, s, "randn") for s in op.BENCH_SHAPES]
        shapes += [(c, s, d) for c, (s, d) in op.CONFIGS.items() if c in configs and "dtype" not in s]
        rows = []
        for i, (cname, shape, dist) in enumerate(shapes):
            log(f"[A/B] {opname} {cname or 'bench shape'} {shape} {dist}")
            r = ab_shape(op, shape, dist, rounds, flush, seed=i)
            r["config"] = cname
            log(f"[A/B]   kernel {r['median_us']['kernel']:.1f} us, {r['strongest_ref']} "
                f"{r['median_us'][r['strongest_ref']]:.1f} us: {r['speedup_vs_strongest_ref']:.2f}x "
                f"(p10 {r['speedup_p10']:.2f}, p90 {r['speedup_p90']:.2f})")
            rows.append(r)
        sp = [r["speedup_vs_strongest_ref"] for r in rows if r["config"] is None]
        res[opname] = dict(rounds=rounds, shapes=rows,
                           geomean_bench_shapes=round(float(np.exp(np.mean(np.log(sp)))), 3),
                           min_bench_shapes=min(sp), max_bench_shapes=max(sp))
    del flush
    return res


def measured_traffic(name, dom):
    """HBM bytes per call of the dominant kernel from the committed PMC summary of this configuration
    (profiles/<config>_traffic.json, FETCH_SIZE + WRITE_SIZE scaled by a copy-kernel calibration), else None."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    if t.get("kernel") != dom["kernel"]:
        return None
    return int(t["read_bytes"] + t["write_bytes"])


def measured_mfma(name, kernel):
    """The dominant kernel's MFMA-busy share from the committed SQ counter summary of this configuration
    (profiles/<config>_mfma.json: SQ_VALU_MFMA_BUSY_CYCLES over the kernel's active cycles), else None."""
    path = os.path.join(ROOT, "profiles", f"{name}_mfma.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    if t.get("kernel") != kernel:
        return None
    return {k: t[k] for k in ("mfma_busy", "coexec", "valu_per_mfma") if k in t}


def write_results(outdir, rows, ab, device):
    """Every configuration's full row and every A/B sample, to outdir/bench_full.json and one
    outdir/bench_<op>.json per A/B op (reference bench.py:276-284 keeps its per-shape samples the same way);
    returns the path of the full file, or None when outdir is empty."""
    if not outdir:
        return None
    os.makedirs(outdir, exist_ok=True)
    full = os.path.join(outdir, "bench_full.json")
    with open(full, "w") as f:
        json.dump(dict(device=device, ops=rows, ab_vs_torch=ab), f, indent=1)
    for opname, r in (ab or {}).items():
        with open(os.path.join(outdir, f"bench_{opname}.json"), "w") as f:
            json.dump(dict(device=device, op=opname, **r), f, indent=1)
    return full


def summary_line(rows, ab, steps, warmup, results=None):
    """The one stdout line: the headline configuration's figures, its roofline and CPU baseline, and a compact
    map of every configuration to [us/call, GB/s, % of peak HBM]; a few KB whatever the number of rows."""
    head_name = HEADLINE if HEADLINE in rows else next(iter(rows))
    head = rows[head_name]
    dom = head["dominant"]
    cpu = head.get("cpu_baseline") or {}
    roof = dict(bound="hbm", achieved=dom["gbs"], peak=PEAK_HBM_GBS, unit="GB/s", frac=dom["frac"],
                traffic=dom.get("traffic"), kernel=dom["kernel"], kernel_us=dom["us"],
                algorithmic_bytes=dom["bytes"])
    if dom.get("tflops") is not None:
        roof["mfma"] = dict(achieved=dom["tflops"], peak=PEAK_FP16_TFLOPS, unit="TFLOP/s",
                            frac=round(dom["tflops"] / PEAK_FP16_TFLOPS, 4), sq=dom.get("sq"))
    return dict(
        metric=METRIC, value=head["gbs"], unit="GB/s", n_gpus=1, steps=steps, warmup=warmup,
        ms_per_step=round(head["us_per_call"] / 1e3, 5), higher_is_better=True, scaling="weak", vs_baseline=None,
        dtype="fp16 (fp32 accumulate)", data="synthetic (seeded N(0,1) inputs of the BASELINE configuration)",
        config=dict(workload=f"{head_name}: {head['op']} " + ", ".join(f"{k}={v}" for k, v in head["shape"].items())
                    + f", dist={head['dist']}",
                    us_per_call=head["us_per_call"], pct_peak=head["pct_peak"], tflops=head.get("tflops"),
                    timing=f"median of {head['us_spread']['replays']} replays of a HIP graph of {steps} calls "
                           f"(p10 {head['us_spread']['p10']}, p90 {head['us_spread']['p90']}); eager loop "
                           f"{head['eager']['us_per_call']} us/call"),
        roofline=roof,
        cpu_baseline=None if not cpu else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample",
                                                               "us_per_call") if k in cpu},
        ops={name: [r["us_per_call"], r["gbs"], r["pct_peak"]] for name, r in rows.items()},
        ops_fields=["us_per_call", "GB/s", "pct_of_8TB/s"],
        ab=None if ab is None else {op: dict(geomean=r["geomean_bench_shapes"], min=r["min_bench_shapes"],
                                             max=r["max_bench_shapes"], rounds=r["rounds"]) for op, r in ab.items()},
        results=None if results is None else os.path.relpath(results, ROOT))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="C1,C2,C3,C4,C5,C5s,D1,D2,D3,P2,P2n,D1p,D2n,C2b,DP")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle timings")
    ap.add_argument("--ab-rounds", type=int, default=10,
                    help="shuffled rounds of the A/B comparison with the torch standard ops (0: skip it)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="first run a plain streaming kernel that reads BYTES and writes BYTES (torch.bitwise_not "
                         "on int32), the calibration of the PMC traffic counters")
    ap.add_argument("--results", default=os.path.join(ROOT, "results"), metavar="DIR",
                    help="where the full rows and A/B samples are written ('' to skip)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one MI355X: the three ops run on a single GPU and this build has no multi-GPU path "
            "(how the ops would shard over several GPUs is a design only).  Run with --gpus 1.")
        sys.exit(2)
    import torch
    import vmk
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    vmk.device_ok("cuda:0")
    if a.calibrate_copy:
        x = torch.ones(a.calibrate_copy // 4, dtype=torch.int32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(2):
            torch.bitwise_not(x, out=y)
        torch.cuda.synchronize()
        del x, y
        log(f"calibration kernel over {a.calibrate_copy} bytes done")
    want = [c for c in a.configs.split(",") if c]
    rows = {}
    for name, opname, shape, dist in config_table():
        if name in want:
            rows[name] = bench_config(name, opname, shape, dist, a.steps, a.warmup,
                                      do_cpu=not a.no_cpu)
    ab = ab_bench(a.ab_rounds, want) if a.ab_rounds > 0 else None
    results = write_results(a.results, rows, ab, device=torch.cuda.get_device_name(0))
    log(f"full rows and A/B samples: {results}")
    line = summary_line(rows, ab, a.steps, a.warmup, results)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
