"""Builds the gfx950 HIP library libssm_mamba_hip.so in-tree with hipcc.

Each .hip translation unit is compiled separately (in parallel) and linked into
one shared object exporting the C ABI of include/ssm_mamba.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libssm_mamba_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
SOURCES = ["scan_fwd.hip", "scan_bwd.hip", "state_update.hip", "conv1d.hip", "decode.hip", "norm.hip", "capi.hip"]

ARCH = os.environ.get("SSM_MAMBA_ARCH", "gfx950")

# Packed fp32 VALU forms are disabled for all device code on this platform.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall",
                "-Wno-unused-command-line-argument"]


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return p


def _compile(src: str, obj: str) -> str:
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = True, jobs: int = 4) -> str:
    """Compile every .hip source for gfx950 and link the shared library.
    Always rebuilds.  Returns the library path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    objs = [os.path.join(LIB_DIR, s.replace(".hip", ".o")) for s in SOURCES]
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, SOURCES, objs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB_PATH)
    for o in objs:
        os.remove(o)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
