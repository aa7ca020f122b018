"""Build the gfx950 GEMM library and its Python binding, in-tree.

Outputs (git-ignored, shipped to the GPU box with the tree):
  cmp_ext_amd/lib/libcmpext3_gemm.so   HIP kernels + C ABI (include/cmpext3_gemm.h)
  cmp_ext_amd/_cmpext3<EXT_SUFFIX>      pybind11 module `cmpext3` (links the above)

The kernels are compiled with hipcc for gfx950 only; the host-only sources
(selector, C ABI, bindings) with g++.  No hipify step is involved: the
sources are HIP-native.  Usage:  python -m cmp_ext_amd.build [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libcmpext3_gemm.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_SOURCES = [f"tile_{t}_{lay}_{k}.hip" for t in ("f16", "bf16") for lay in ("kn", "nk") for k in ("whole", "ragged")] + \
    ["skinny.hip", "tall.hip", "stream.hip", "stream_nk.hip", "f32.hip", "generic.hip", "pad.hip", "noalloc.hip", "sem.hip"]
HOST_SOURCES = ["selector.cpp", "api.cpp"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops (v_pk_*_f32) stay off on this platform
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + CSRC,
    "-I" + os.path.join(ROOT, "include"),
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-Wall",
    "-D__HIP_PLATFORM_AMD__=1",
    "-I" + CSRC,
    "-I" + os.path.join(ROOT, "include"),
    "-I" + os.path.join(ROCM, "include"),
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _obj(src: str) -> str:
    return os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")


def build_library(jobs: int) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    cmds = []
    for s in HIP_SOURCES:
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, s), "-o", _obj(s)])
    for s in HOST_SOURCES:
        cmds.append(["g++", *HOST_FLAGS, "-c", os.path.join(CSRC, s), "-o", _obj(s)])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    objs = [_obj(s) for s in HIP_SOURCES + HOST_SOURCES]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-soname,libcmpext3_gemm.so"])
    os.replace(tmp, LIB)
    return LIB


def build_binding() -> str:
    import torch
    from torch.utils import cpp_extension

    ext = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_cmpext3" + ext)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"],
                                            os.path.join(ROCM, "include")]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = "1" if torch.compiled_with_cxx11_abi() else "0"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-DTORCH_EXTENSION_NAME=_cmpext3", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *("-I" + i for i in incs),
           os.path.join(CSRC, "main.cpp"), "-o", out + ".tmp",
           "-L" + torch_lib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-L" + LIBDIR, "-lcmpext3_gemm", "-Wl,-rpath,$ORIGIN/lib"]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int | None = None) -> None:
    jobs = jobs or min(8, os.cpu_count() or 1)
    lib = build_library(jobs)
    mod = build_binding()
    print(f"built {os.path.relpath(lib, ROOT)} and {os.path.relpath(mod, ROOT)}")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    try:
        build(a.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
