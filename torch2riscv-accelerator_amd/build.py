"""Builds libt2r.so (the C-ABI of include/t2r.h) for gfx950 with hipcc, in-tree.

    python -m t2r_amd.build            (or __graft_entry__.build())

Flags: -O3, -ffp-contract=off (no fused multiply-add: every fp32 step rounds once, as the
reference's vector engine), the default f32 denormal mode (IEEE, as NumPy float32), and packed
fp32 instructions switched off.
"""
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "t2r.hip")
LIB = os.path.join(HERE, "libt2r.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("T2R_ARCH", "gfx950")
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]


def build(verbose=False):
    t0 = time.time()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{' '.join(cmd)}\n{err}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f} s" + (f"\n{err}" if err.strip() else ""), flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
