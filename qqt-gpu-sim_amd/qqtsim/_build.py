"""Build libqqt_hip.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950.

    python -m qqtsim._build            # from qqt-gpu-sim_amd/

Flags: -ffp-contract=off keeps every float32 product and sum separately
rounded (bit-exact state needs the reference's operation order);
`-target-feature -packed-fp32-ops` keeps the compiler from emitting packed
fp32 arithmetic.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)                       # qqt-gpu-sim_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIBDIR = os.path.join(PKG, "_lib")
LIB = os.path.join(LIBDIR, "libqqt_hip.so")
SOURCES = ["tick.hip", "mlp.hip", "mlp_grad.hip", "ppo.hip", "cnn.hip", "bot.hip", "gae.hip", "timing.hip"]
ARCH = os.environ.get("QQT_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libqqt_hip.so)")


def flags() -> list[str]:
    return ["-O3", f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", INCLUDE, "-I", CSRC, "-Wno-unused-result"]


def build(verbose: bool = True) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *flags(), "-shared", "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
