"""Build recipe for the HIP library `libmce.so` (gfx950 only).

Run `python -m memarch_amd.build` (or `__graft_entry__.build()`). The library is written in-tree next to this file
so that it travels with the source tree; it is a plain C-ABI shared object loaded through ctypes.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", f) for f in ("mce.hip", "induct.hip", "swiglu.hip")]
LIB = os.path.join(HERE, "libmce.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: hipcc may otherwise emit packed fp32 VALU ops on its own.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def build(verbose=False):
    """Compile libmce.so from source every time it is called; raises CalledProcessError on failure. Returns its
    path."""
    _compile(SRCS, LIB, verbose)
    return LIB


def _compile(srcs, lib, verbose):
    tmp = lib + ".tmp"
    cmd = [HIPCC, *FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        sys.stderr.write("\n".join(msgs) + "\n")
        raise subprocess.CalledProcessError(res.returncode, cmd)
    if verbose and msgs:
        print("\n".join(msgs))
    os.replace(tmp, lib)


if __name__ == "__main__":
    print(build(verbose=True))
