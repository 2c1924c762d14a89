#!/usr/bin/env python3
"""Build the cmpext3 native code in-tree for gfx950 (MI355X).

Outputs (next to the Python package, so they travel with the tree):
  cmpext3/libcmpext3_attn.so          HIP kernels + the C ABI of include/cmpext3_attn.h
  cmpext3/_native<EXT_SUFFIX>         torch binding (ops.attention), links the above

Usage: python torch-cmp-patch_amd/build.py [-j N] [--verbose]
Every HIP file is compiled with packed-fp32 instructions disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "cmpext3")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(REPO, "include")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["attn_fwd_mfma16.hip", "attn_fwd_pipe16.hip", "attn_fwd_pipe16w.hip", "attn_fwd_pipe16wm.hip", "attn_fwd_short16.hip", "attn_fwd_mfma32.hip",
               "attn_fwd_decode16.hip", "attn_bwd16.hip", "attn_bwd32.hip", "attn_abi.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in arch VGPRs (no AGPR<->VGPR copies around the
    # softmax), and no sNaN quieting in front of every v_max: the kernels
    # never rely on signalling-NaN semantics.
    "-mllvm", "-amdgpu-mfma-vgpr-form", "-mno-amdgpu-ieee", "-fno-honor-nans",
    f"-I{INCLUDE}",
]

# The pipelined kernel keeps IEEE mode: with it off the compiler schedules the
# fp16 D <= 64 instantiations into spills at 3 waves per SIMD.  Its common
# path has no max operations, so the quieting instructions cost nothing there.
FILE_FLAGS_DROP = {"attn_fwd_pipe16.hip": {"-mno-amdgpu-ieee", "-fno-honor-nans"},
                   "attn_fwd_pipe16w.hip": {"-mno-amdgpu-ieee", "-fno-honor-nans"},
                   "attn_fwd_pipe16wm.hip": {"-mno-amdgpu-ieee", "-fno-honor-nans"}}

LIB_NAME = "libcmpext3_attn.so"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature: harmless, filtered
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "is not a recognized feature for this target" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def _compile_hip(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    drop = FILE_FLAGS_DROP.get(src, set())
    flags = [f for f in HIP_FLAGS if f not in drop]
    _run([HIPCC, *flags, *lang, "-c", os.path.join(CSRC, src), "-o", obj], verbose)
    return obj


def build_lib(jobs: int, verbose: bool) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile_hip(s, verbose), HIP_SOURCES))
    out = os.path.join(PKG, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname," + LIB_NAME], verbose)
    os.replace(tmp, out)
    return out


def build_native(verbose: bool) -> str:
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    py_inc = sysconfig.get_paths()["include"]
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_native" + suffix)
    tmp = out + ".tmp"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = os.environ.get("CXX", shutil.which("g++") or "g++")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", os.path.join(CSRC, "main.cpp"), "-o", tmp,
           *[f"-I{p}" for p in cpp_extension.include_paths()], f"-I{py_inc}", f"-I{ROCM}/include",
           f"-I{INCLUDE}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_native",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-Wno-deprecated-declarations",
           f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
           "-ltorch_hip", f"-L{PKG}", "-l:" + LIB_NAME,
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(jobs: int = 4, verbose: bool = False) -> list[str]:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f_lib = ex.submit(build_lib, jobs, verbose)
        lib = f_lib.result()
        native = build_native(verbose)
    return [lib, native]


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    for path in build(a.jobs, a.verbose):
        print("built", os.path.relpath(path, REPO))
    return 0


if __name__ == "__main__":
    sys.exit(main())
