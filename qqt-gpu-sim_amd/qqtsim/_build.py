"""Build libqqt_hip.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950.

    python -m qqtsim._build            # from qqt-gpu-sim_amd/

Flags: -ffp-contract=off keeps every float32 product and sum separately
rounded (bit-exact state needs the reference's operation order);
`-target-feature -packed-fp32-ops` keeps the compiler from emitting packed
fp32 arithmetic in the device code.  The clang driver cannot forward that
`-Xclang` pair to the device pass alone (`-Xarch_device` rejects options
that take an argument), so both passes get it and the host pass's
"not a recognized feature" notice is dropped from the build output.
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
SOURCES = ["tick.hip", "tick_group.hip", "mlp.hip", "mlp_sparse.hip", "mlp_grad.hip", "ppo.hip", "cnn.hip", "lstm.hip", "bot.hip", "gae.hip",
           "timing.hip"]
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


HOST_FEATURE_NOTICE = "'-packed-fp32-ops' is not a recognized feature for this target"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(ln for ln in res.stdout.splitlines() if HOST_FEATURE_NOTICE not in ln)
    if out.strip() and (verbose or res.returncode):
        print(out, flush=True)
    if res.returncode:
        raise subprocess.CalledProcessError(res.returncode, cmd)


def build(verbose: bool = True) -> str:
    """Compile every source to an object (in parallel), then link."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIBDIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    missing = [s for s in srcs if not os.path.exists(s)]
    if missing:
        raise FileNotFoundError(f"HIP sources missing: {missing}")
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        for f in [ex.submit(_run, [hipcc(), *flags(), "-c", "-o", o, s], verbose)
                  for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
