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
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    cmd = [hipcc, *FLAGS, *extra, "-I", CSRC, "-I", INCLUDE, *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed ({p.returncode}):\n{msg}")
    if verbose and msg.strip():
        print(msg)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
    print("built", LIB)
