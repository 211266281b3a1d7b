"""Builds libvmk.so (all HIP sources under csrc/) for gfx950 with hipcc, in-tree next to this file."""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "csrc")
INCLUDE = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include")   # the C ABI header (vmk.h)
LIB = os.path.join(HERE, "libvmk.so")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         # packed fp32 VALU forms are disabled: ordinary float code must not turn into them.
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose=False, extra=()):
    """Compiles every source to an object in parallel (each carries its own gfx950 code object), then links them
    into libvmk.so; the library is replaced only when the whole build succeeds."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    compile_flags = [f for f in FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="vmk_build_") as odir:
        jobs = []
        for src in sources():
            obj = os.path.join(odir, os.path.basename(src) + ".o")
            jobs.append(([hipcc, *compile_flags, *extra, "-I", CSRC, "-I", INCLUDE, "-c", src, "-o", obj], obj))
        link = [hipcc, *FLAGS, *extra, *[o for _, o in jobs], "-o", tmp]
        workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with ThreadPoolExecutor(workers) as pool:
            results = list(pool.map(lambda j: _run(j[0], verbose), jobs))
        msgs = [m for m in results if m]
        msgs.append(_run(link, verbose))
    msg = "\n".join(m for m in msgs if m)
    if verbose and msg.strip():
        print(msg)
    os.replace(tmp, LIB)
    return LIB


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed ({p.returncode}): {' '.join(cmd)}\n{msg}")
    return msg


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
    print("built", LIB)
