"""Build recipe for the native parts (run by ``__graft_entry__.build()``).

* ``libwlq_hip.so``: the C ABI (include/wlq_abi.h) with the gfx950 kernels,
  compiled by hipcc; no torch dependency.
* ``vllm_wlq/_C.<abi>.so``: the PyTorch-ROCm extension, compiled by the host
  C++ compiler against torch's headers and linked to ``libwlq_hip.so``
  (rpath ``$ORIGIN/..``).

Everything is written in-tree so the built files travel with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

LIB_PATH = os.path.join(PKG, "libwlq_hip.so")
EXT_DIR = os.path.join(PKG, "vllm_wlq")

HIP_SOURCES = ["wlq_abi.hip", "wlq_skinny.hip", "wlq_stream.hip", "wlq_wide.hip", "wlq_prefill.hip", "wlq_gemm.hip",
               "wlq_dequant.hip",
               "wlq_epilogue.hip"]
HOST_SOURCES = ["wlq_host.cpp"]

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed FP32 ops are kept out of generated code (they have produced wrong
    # results on this hardware pool); hipcc's host pass warns about the flag.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if p.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + p.stdout)
    return p.stdout


def ext_filename() -> str:
    return "_C" + sysconfig.get_config_var("EXT_SUFFIX")


def build_lib(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cmds, objs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
        cmds.append(["g++", "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-I", INCLUDE,
                     "-I", os.path.join(ROCM, "include"), "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_ext() -> str:
    import torch.utils.cpp_extension as ce

    inc = []
    for p in ce.include_paths(device_type="cuda"):
        inc += ["-I", p]
    inc += ["-I", sysconfig.get_paths()["include"], "-I", INCLUDE, "-I", os.path.join(ROCM, "include")]
    libdirs = ce.library_paths(device_type="cuda")
    torch_lib = libdirs[0]
    out = os.path.join(EXT_DIR, ext_filename())
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-D_GLIBCXX_USE_CXX11_ABI=1", "-Wno-deprecated-declarations",
           *inc, os.path.join(CSRC, "binding.cpp"), "-o", tmp,
           "-L", PKG, "-lwlq_hip", "-Wl,-rpath,$ORIGIN/..",
           "-L", torch_lib, "-Wl,-rpath," + torch_lib,
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python"]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all(jobs: int = 8) -> None:
    build_lib(jobs)
    build_ext()


if __name__ == "__main__":
    build_all(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print("built", LIB_PATH, "and", os.path.join(EXT_DIR, ext_filename()))
