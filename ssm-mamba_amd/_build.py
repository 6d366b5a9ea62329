"""Builds, in-tree:

* the gfx950 HIP library ``_lib/libssm_mamba_hip.so`` with hipcc: each .hip
  translation unit compiled separately (in parallel) and linked into one
  shared object exporting the C ABI of include/ssm_mamba.h;
* the PyTorch-ROCm extension modules ``_ext/selective_scan`` and
  ``_ext/selective_update`` (host C++ over that C ABI, the counterparts of
  the reference's compiled modules), compiled with the host compiler against
  torch's headers and linked to the HIP library (rpath ``$ORIGIN/../_lib``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libssm_mamba_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
SOURCES = ["scan_fwd.hip", "scan_bwd.hip", "state_update.hip", "conv1d.hip", "decode.hip", "norm.hip", "capi.hip"]
EXT_DIR = os.path.join(PKG_DIR, "_ext")
EXT_MODULES = ["selective_scan", "selective_update"]
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def ext_path(name: str) -> str:
    return os.path.join(EXT_DIR, name + EXT_SUFFIX)


def _torch_flags():
    """Compile and link flags for a torch C++ extension on this ROCm build
    (what torch.utils.cpp_extension passes, without its hipify step)."""
    import torch
    from torch.utils import cpp_extension as ce
    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    cflags = ["-O2", "-std=c++17", "-fPIC", "-DTORCH_API_INCLUDE_EXTENSION_H",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    for inc in ce.include_paths():
        cflags += ["-isystem", inc]
    cflags += ["-isystem", sysconfig.get_paths()["include"], "-I/opt/rocm/include"]
    ldflags = ["-shared", f"-L{tlib}", "-lc10_hip", "-lc10", "-ltorch_cpu", "-ltorch",
               "-ltorch_python", f"-Wl,-rpath,{tlib}", f"-L{LIB_DIR}", "-lssm_mamba_hip",
               "-Wl,-rpath,$ORIGIN/../_lib"]
    return cflags, ldflags

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


def _compile_ext(name: str, cflags) -> str:
    obj = os.path.join(EXT_DIR, name + ".o")
    cmd = ["g++", *cflags, f"-DTORCH_EXTENSION_NAME={name}", "-c",
           os.path.join(CSRC, "ext", name + ".cpp"), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for extension {name}:\n{r.stderr[-6000:]}")
    return obj


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr[-6000:]}")


def build(verbose: bool = True, jobs: int = 4) -> str:
    """Compile every .hip source for gfx950 and link the shared library, then
    the two extension modules against it.  Always rebuilds.  Returns the
    library path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(EXT_DIR, exist_ok=True)
    objs = [os.path.join(LIB_DIR, s.replace(".hip", ".o")) for s in SOURCES]
    cflags, ldflags = _torch_flags()
    with ThreadPoolExecutor(max_workers=jobs + len(EXT_MODULES)) as ex:
        ext_jobs = [ex.submit(_compile_ext, n, cflags) for n in EXT_MODULES]
        list(ex.map(_compile, SOURCES, objs))
        ext_objs = [j.result() for j in ext_jobs]
    tmp = LIB_PATH + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB_NAME}",
          "-o", tmp, *objs], "link")
    os.replace(tmp, LIB_PATH)
    for o in objs:
        os.remove(o)
    for name, obj in zip(EXT_MODULES, ext_objs):
        out = ext_path(name)
        _run(["g++", obj, *ldflags, "-o", out + ".tmp"], f"link of extension {name}")
        os.replace(out + ".tmp", out)
        os.remove(obj)
    if verbose:
        print(f"built {LIB_PATH} and {', '.join(ext_path(n) for n in EXT_MODULES)}",
              file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
