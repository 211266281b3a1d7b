"""Benchmark of the attention ops on one MI355X, in the driver's contract.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs C1,C2,...] [--no-cpu]

Prints human-readable progress on stderr and ONE JSON line on stdout.  A "step" is one call of the op on one batch
of the headline configuration (BASELINE configs[1] = C2, shared-prefix decode at scale); `value` is its achieved
HBM throughput (algorithmic bytes / time per call, inputs resident in HBM), `ops` holds the same figures for every
configuration (C1..C5, and this build's D1-D3 decode, P2 paged prefix, C2b bf16).  Method (a counterpart of the
reference's bench.py:44-140 timing):
  * the kernel's output on the timed inputs is checked against the PyTorch standard op first
    (allclose atol=rtol=1e-2, bench.py:180-192 of the reference), and the inputs are checked for modification;
  * every call reads a different input set, rotating over enough distinct sets (>= 1 GiB in total) that the
    256 MB Infinity Cache cannot serve a repeat;
  * W untimed warm-up calls, then the per-call time: the K calls captured once in a HIP graph and replayed between
    two HIP events (synchronised before and after), after 3 replays checked bit for bit against an eager call;
    `eager` gives the same K calls launched one by one from Python, which adds the host's per-call overhead;
  * the dominant kernel of each op is bracketed by its own pair of HIP events on its launch stream inside the eager
    loop (libvmk's vmk_profile_next hook), which gives the roofline figure.
The CPU baseline is the float64 NumPy oracle (oracle/) on the host, on a bounded sample of the same workload.
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
HEADLINE = "C2"
DOMINANT = {"prefix": "prefix_partial", "spec": "spec_partial", "dsa": "dsa_indexer", "decode": "spec_partial",
            "prefix_paged": "prefix_partial"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def config_table():
    from vmk.ops import decode, dsa, prefix, prefix_paged, spec
    return [("C1", "prefix", *prefix.CONFIGS["C1"]), ("C2", "prefix", *prefix.CONFIGS["C2"]),
            ("C3", "spec", *spec.CONFIGS["C3"]), ("C4", "spec", *spec.CONFIGS["C4"]),
            ("C5", "dsa", *dsa.CONFIGS["C5"]),
            ("D1", "decode", *decode.CONFIGS["D1"]), ("D2", "decode", *decode.CONFIGS["D2"]),
            ("D3", "decode", *decode.CONFIGS["D3"]), ("P2", "prefix_paged", *prefix_paged.CONFIGS["P2"]),
            ("C2b", "prefix", *prefix.CONFIGS["C2b"])]


class HipEvents:
    """Raw HIP events (libamdhip64 through ctypes) for the per-kernel brackets recorded inside libvmk."""

    def __init__(self, n):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.ev = []
        for _ in range(2 * n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
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
    if opname == "prefix_paged":
        return vmk.prefix_decode_paged(inp["q"], inp["k_pages"], inp["v_pages"], inp["prefix_pages"],
                                       inp["suffix_pages"], inp.get("slens"))
    return vmk.dsa_decode(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp.get("lens"))


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
    return dsa.torch_fp32_ref(inp["q"], inp["kv"], inp["iq"], inp["ik"], inp["w"], inp.get("lens"))


def op_bytes_flops(opname, shape, inp_host):
    from vmk.ops import decode, dsa, prefix, prefix_paged, spec
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
    if opname == "decode":
        ln = None if inp_host.get("lens") is None else inp_host["lens"].numpy()
        total = decode.algorithmic_bytes(shape, ln)
        out = shape["B"] * decode.HQ * decode.D * 2
        return total, total - out, decode.flops(shape, ln)
    total = dsa.algorithmic_bytes(shape)
    B, L = shape["B"], shape["L"]
    indexer = B * L * dsa.DI * 2 + B * dsa.HI * dsa.DI * 2 + B * dsa.HI * 4    # ik + iq + w
    return total, indexer, dsa.flops(shape)


def distinct_sets(opname, inp0, total_bytes):
    """Extra input sets with the same shapes and dtypes (synthetic N(0,1) data made on the GPU), so that the calls
    of the timed loop rotate over >= 1 GiB of inputs; masks/lengths are shared."""
    import torch
    n = max(2, int(math.ceil((1 << 30) / max(total_bytes, 1))))
    sets = [inp0]
    big = {"prefix": ("q", "kp", "vp", "ks", "vs"), "spec": ("q", "k", "v"), "dsa": ("q", "kv", "iq", "ik"),
           "decode": ("q", "k", "v"), "prefix_paged": ("q", "k_pages", "v_pages")}[opname]
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    for _ in range(n - 1):
        s = dict(inp0)
        for k in big:
            s[k] = torch.randn(inp0[k].shape, device="cuda", generator=g, dtype=torch.float32).to(inp0[k].dtype)
        sets.append(s)
    return sets


def cpu_baseline(opname, shape, dist, inp_host, total_bytes):
    """Times the float64 oracle on a bounded sample of the workload on the host cores; returns a dict."""
    import oracle
    try:
        from threadpoolctl import threadpool_limits, threadpool_info
        cores = min(16, os.cpu_count() or 1)
        ctx = threadpool_limits(limits=cores)
        blas = [d.get("num_threads") for d in threadpool_info() if d.get("user_api") == "blas"]
    except Exception:  # pragma: no cover - threadpoolctl missing
        import contextlib
        ctx, cores, blas = contextlib.nullcontext(), os.cpu_count() or 1, []
    with ctx:
        if opname == "prefix":
            N = shape["N"]
            ns = min(N, 8)
            sub = {k: inp_host[k][:ns] for k in ("q", "ks", "vs")}
            sub.update(kp=inp_host["kp"], vp=inp_host["vp"],
                       slens=None if inp_host.get("slens") is None else inp_host["slens"][:ns])
            t0 = time.perf_counter()
            oracle.prefix.ref64(**sub)
            dt = (time.perf_counter() - t0) * N / ns
            sample = f"requests 0-{ns - 1} of {N}, time scaled x{N / ns:g}"
        elif opname == "spec":
            B = shape["B"]
            t0 = time.perf_counter()
            oracle.spec.ref64(inp_host["q"][:1], inp_host["k"][:1], inp_host["v"][:1], inp_host["bits"][:1])
            dt = (time.perf_counter() - t0) * B
            sample = f"batch 0 of {B}, time scaled x{B}"
        elif opname == "prefix_paged":
            N = shape["N"]
            ns = min(N, 8)
            sub = dict(inp_host, q=inp_host["q"][:ns], suffix_pages=inp_host["suffix_pages"][:ns],
                       slens=None if inp_host.get("slens") is None else inp_host["slens"][:ns])
            t0 = time.perf_counter()
            oracle.prefix_paged.ref64(**sub)
            dt = (time.perf_counter() - t0) * N / ns
            sample = f"requests 0-{ns - 1} of {N}, time scaled x{N / ns:g}"
        elif opname == "decode":
            B = shape["B"]
            t0 = time.perf_counter()
            oracle.decode.ref64(inp_host["q"][:1], inp_host["k"][:1], inp_host["v"][:1],
                                None if inp_host.get("lens") is None else inp_host["lens"][:1])
            dt = (time.perf_counter() - t0) * B
            sample = f"request 0 of {B}, time scaled x{B}"
        else:
            B = shape["B"]
            t0 = time.perf_counter()
            oracle.dsa.ref64(inp_host["q"][:1], inp_host["kv"][:1], inp_host["iq"][:1], inp_host["ik"][:1],
                             inp_host["w"][:1], None)
            dt = (time.perf_counter() - t0) * B
            sample = f"request 0 of {B} (scores, top-2048, attention), time scaled x{B}"
    return dict(value=round(total_bytes / dt / 1e9, 3), unit="GB/s", us_per_call=round(dt * 1e6, 1), cores=cores,
                blas_threads=blas, kind="port", sample=sample)


def bench_config(name, opname, shape, dist, steps, warmup, do_cpu):
    import torch
    import vmk
    from vmk import lib
    from vmk.ops import OPS
    op = OPS[opname]
    log(f"[{name}] {opname} {shape} {dist}: generating inputs")
    host = op.make_inputs(shape, seed=0, dist=dist)
    inp0 = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in host.items()}
    if opname == "spec":
        inp0["words"] = op.mask_words(inp0["bits"], shape["k"]).contiguous()
    total_bytes, dom_bytes, flops = op_bytes_flops(opname, shape, host)
    # Output check on the benchmark inputs and input-mutation check (reference bench.py:180-192).
    snap = {k: v.clone() for k, v in inp0.items() if isinstance(v, torch.Tensor)}
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
    kid = lib.KERNEL_IDS[DOMINANT[opname]]
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
    us = graph_us_per_call(opname, sets, steps)
    gbs = total_bytes / us / 1e3
    dom_gbs = dom_bytes / dom_us / 1e3
    row = dict(op=opname, shape=shape, dist=dist, us_per_call=round(us, 2), gbs=round(gbs, 1),
               pct_peak=round(100 * gbs / PEAK_HBM_GBS, 2), algorithmic_bytes=int(total_bytes),
               tflops=round(flops / us / 1e6, 2), mfma_pct=round(100 * flops / us / 1e6 / PEAK_FP16_TFLOPS, 2),
               eager=dict(us_per_call=round(eager_us, 2), gbs=round(total_bytes / eager_us / 1e3, 1)),
               dominant=dict(kernel=DOMINANT[opname], us=round(dom_us, 2), bytes=int(dom_bytes),
                             gbs=round(dom_gbs, 1), frac=round(dom_gbs / PEAK_HBM_GBS, 4)),
               output_check="ok", distinct_input_sets=len(sets))
    log(f"[{name}] {us:9.2f} us/call  {gbs:7.1f} GB/s ({row['pct_peak']:.1f}% of 8 TB/s)  [HIP graph of {steps} calls; "
        f"eager loop {eager_us:.2f} us/call]   dominant {DOMINANT[opname]} {dom_us:.2f} us = {dom_gbs:.0f} GB/s")
    if do_cpu:
        row["cpu_baseline"] = cpu_baseline(opname, shape, dist, host, total_bytes)
        log(f"[{name}] CPU float64 oracle: {row['cpu_baseline']['us_per_call']:.0f} us/call "
            f"({row['cpu_baseline']['sample']}, {row['cpu_baseline']['cores']} cores)")
    del sets, inp0, host
    torch.cuda.empty_cache()
    return row


def graph_us_per_call(opname, sets, steps):
    """µs per call of the K calls captured once in a HIP graph (torch.cuda.CUDAGraph over the calls' launches on the
    capture stream, rotating over the same input sets) and replayed once between two events, synchronised before and
    after: the GPU time of K steps without the Python and launch overhead of an eager loop, which dominates ops of a
    few µs.  Before timing, the output of the last captured call after each of 3 replays (with eager work and
    synchronisation in between) must equal an eager call on the same inputs bit for bit."""
    import torch
    n = steps
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            call_op(opname, sets[i % len(sets)])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [call_op(opname, sets[i % len(sets)]) for i in range(n)]
    last = outs[-1]
    ref = call_op(opname, sets[(n - 1) % len(sets)]).clone()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(last.view(torch.int16), ref.view(torch.int16)):
            raise SystemExit(f"{opname}: a graph replay differs from the eager call")
        call_op(opname, sets[0])                          # eager work between replays
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g, outs
    return e0.elapsed_time(e1) * 1e3 / n


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


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="C1,C2,C3,C4,C5,D1,D2,D3,P2,C2b")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle timings")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="first run a plain streaming kernel that reads BYTES and writes BYTES (torch.bitwise_not "
                         "on int32), the calibration of the PMC traffic counters")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one MI355X: the three ops run on a single GPU and this build has no multi-GPU path "
            "(the sharding design is in DESIGN.md).  Run with --gpus 1.")
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
    head = rows.get(HEADLINE) or next(iter(rows.values()))
    head_name = HEADLINE if HEADLINE in rows else next(iter(rows))
    dom = head["dominant"]
    line = dict(
        metric=METRIC, value=head["gbs"], unit="GB/s", n_gpus=1, steps=a.steps, warmup=a.warmup,
        ms_per_step=round(head["us_per_call"] / 1e3, 5), higher_is_better=True, scaling="weak", vs_baseline=None,
        dtype="fp16 (fp32 accumulate)", data="synthetic (seeded N(0,1) inputs of the BASELINE configuration)",
        config=dict(workload=f"{head_name}: {head['op']} {head['shape']} dist={head['dist']}",
                    us_per_call=head["us_per_call"], pct_peak=head["pct_peak"],
                    timing=f"{a.steps} calls replayed from one HIP graph; eager loop {head['eager']['us_per_call']} "
                           f"us/call"),
        roofline=dict(bound="hbm", achieved=dom["gbs"], peak=PEAK_HBM_GBS, unit="GB/s", frac=dom["frac"],
                      kernel=dom["kernel"], kernel_us=dom["us"], traffic=measured_traffic(head_name, dom)),
        cpu_baseline={k: v for k, v in head.get("cpu_baseline", {}).items()} or None,
        ops=rows,
        device=torch.cuda.get_device_name(0),
    )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
