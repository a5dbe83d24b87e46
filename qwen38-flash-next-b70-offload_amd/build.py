"""Builds the HIP library and the torch op library in-tree:

  exl3xpu/libexl3moe.so   C-ABI (include/exl3moe.h): HIP kernels for gfx950 + entry points; links only the HIP runtime
  exl3xpu/_moe.so         torch.ops.exl3xpu_moe (reference op schemas) over the C-ABI

Usage: python build.py [--jobs N]   (also called by __graft_entry__.build())
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "exl3xpu")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_SOURCES = ["moe_decode.hip", "moe_cache.hip", "moe_prefill.hip", "linear.hip", "moe_capi.hip"]
HOST_SOURCES = ["tier_host.cpp"]          # host-only C++ (g++)
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")
    return r


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    srcs = [s for s in HIP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = [os.path.join(BUILD, s.replace(".hip", ".o")) for s in srcs]

    hsrcs = [s for s in HOST_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    hobjs = [os.path.join(BUILD, s.replace(".cpp", ".o")) for s in hsrcs]

    def comp(i):
        if i < len(srcs):
            _run([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, srcs[i]), "-o", objs[i]])
        else:
            j = i - len(srcs)
            _run(["g++", "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(CSRC, hsrcs[j]), "-o", hobjs[j]])
    with ThreadPoolExecutor(max(1, jobs)) as ex:
        list(ex.map(comp, range(len(srcs) + len(hsrcs))))
    objs = objs + hobjs
    lib = os.path.join(OUT, "libexl3moe.so")
    tmp = lib + ".tmp"
    _run([hipcc, "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, lib)
    return lib


def build_torch_ops() -> str:
    import torch
    from torch.utils import cpp_extension as ce
    inc = ce.include_paths() + [os.path.join(ROCM, "include")]
    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    so = os.path.join(OUT, "_moe.so")
    tmp = so + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_moe", "-Wno-deprecated-declarations",
           *[f"-I{p}" for p in inc], os.path.join(CSRC, "torch_ops.cpp"), "-o", tmp,
           f"-L{OUT}", "-lexl3moe", f"-L{tlib}", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip",
           f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"]
    _run(cmd)
    os.replace(tmp, so)
    return so


def build(jobs: int = 8) -> list:
    with ThreadPoolExecutor(2) as ex:
        f1 = ex.submit(build_hip, jobs)
        f1.result()
        f2 = ex.submit(build_torch_ops)
        return [f1.result(), f2.result()]


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    print("\n".join(build(ap.parse_args().jobs)))
