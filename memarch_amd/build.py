"""Build recipe for the HIP library `libmce.so` (gfx950 only), and for `libmce_probe.so`, the MFMA-rate probe that
bench.py --calibrate-mfma runs (a measurement aid, not part of the operator's C ABI).

Run `python -m memarch_amd.build` (or `__graft_entry__.build()`). The libraries are written in-tree next to this
file so that they travel with the source tree; they are plain C-ABI shared objects loaded through ctypes.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", f) for f in ("mce.hip", "induct.hip", "swiglu.hip")]
LIB = os.path.join(HERE, "libmce.so")
PROBE_SRCS = [os.path.join(HERE, "csrc", "probe.hip")]
PROBE_LIB = os.path.join(HERE, "libmce_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: hipcc may otherwise emit packed fp32 VALU ops on its own.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def build(verbose=False):
    """Compile libmce.so and libmce_probe.so from source every time it is called; raises CalledProcessError on
    failure. Returns the path of libmce.so."""
    _compile(SRCS, LIB, verbose)
    _compile(PROBE_SRCS, PROBE_LIB, verbose)
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
