"""Compile libmoeprefetch.so for gfx950 (hipcc) and the CPU oracle (gcc).

Run from anywhere:  python moe-prefetch_amd/build.py
The library lands next to the Python package (moe_prefetch/libmoeprefetch.so)
so the in-tree package loads it; nothing is installed anywhere.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "moe_prefetch", "libmoeprefetch.so")
SOURCES = ["mp_kernels.hip", "mp_batched.hip", "mp_runtime.cpp", "mp_cpu.cpp", "mp_predictor.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # explicit fmaf only: the router's bit-exact order depends on it
    "-ffp-contract=off",
    # no packed fp32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument",
]


def build(verbose=False):
    cmd = [HIPCC] + FLAGS + [os.path.join(CSRC, s) for s in SOURCES] + ["-o", OUT + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
