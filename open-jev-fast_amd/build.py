"""Builds libojx.so (the HIP kernels + C-ABI of the projection path) in-tree for gfx950 with hipcc.

Run as `python open-jev-fast_amd/build.py` or through `__graft_entry__.build()`. The library lands next to this file
so that it travels with the source tree; nothing is installed.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libojx.so")
SOURCES = ["gemm.hip", "epilogue.hip", "api.hip"]
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: hipcc would otherwise fuse float pairs into v_pk_{add,mul,fma}_f32, which this fleet
# must not run. The host pass warns that it does not know the feature; that warning is expected.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # the fragment epilogues must unroll completely, or the accumulator array is left in scratch memory
         "-mllvm", "-pragma-unroll-threshold=1000000",
         f"-I{INCLUDE}", f"-I{CSRC}"]


def build(verbose: bool = False) -> str:
    """Compiles every source into libojx.so (always rebuilds). Returns the library path."""
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
