#!/usr/bin/env python3
"""Build libfa_hip.so (the C-ABI kernel library) and fused_attn/_C.so (the torch binding) in-tree.

  libfa_hip.so  hipcc --offload-arch=gfx950: csrc/dispatch.cpp + csrc/attn_{f16,bf16,f32}.hip +
                csrc/scratch.hip.
                Exports exactly the functions of include/fa/attention.h.
  _C.so         csrc/ext.cpp against PyTorch-ROCm, linked to libfa_hip.so (rpath $ORIGIN).
  bench/fa_bench  the torch-free benchmark binary (bench/fa_bench.hip), linked to libfa_hip.so.

Both land in fused-attention-cuda_amd/fused_attn/, next to the Python package that loads them.
Object files go to fused-attention-cuda_amd/_build/. Every call rebuilds everything (the build
check must exercise the compiler each time); translation units compile in parallel.

Usage: python fused-attention-cuda_amd/build.py [--jobs N]
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT = PKG_ROOT / "fused_attn"
BUILD = PKG_ROOT / "_build"
INCLUDE = REPO / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 VALU forms are switched off for all device code (the compiler would otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code).
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Keep MFMA accumulators in ordinary VGPRs: the O accumulator is rescaled by VALU every tile, and
# in AGPRs each rescale costs a v_accvgpr_read + v_accvgpr_write per element.
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
             "-Wall", "-Wno-unused-function",
             f"-I{INCLUDE}", f"-I{CSRC}", *NO_PACKED_FP32, *MFMA_VGPR]
HIP_SOURCES = ["attn_f16.hip", "attn_bf16.hip", "attn_f32.hip", "scratch.hip"]
HOST_SOURCES = ["dispatch.cpp"]


def run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(f"$ {' '.join(cmd)}\n{res.stdout}{res.stderr}")
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def compile_hip(src: str) -> Path:
    obj = BUILD / (src + ".o")
    run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def compile_host(src: str) -> Path:
    obj = BUILD / (src + ".o")
    run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", f"-I{INCLUDE}",
         f"-I{CSRC}", "-c",
         str(CSRC / src), "-o", str(obj)])
    return obj


def torch_flags() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths(device_type="cuda")
    libs = cpp_extension.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = [f"-I{p}" for p in inc] + [f"-I{sysconfig.get_paths()['include']}",
                                         "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1",
                                         "-DTORCH_API_INCLUDE_EXTENSION_H",
                                         "-DTORCH_EXTENSION_NAME=_C",
                                         f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    ldflags = [f"-L{p}" for p in libs] + [f"-Wl,-rpath,{torch_lib}", "-lc10", "-lc10_hip",
                                           "-ltorch", "-ltorch_cpu", "-ltorch_hip",
                                           "-ltorch_python"]
    return cflags, ldflags


def build(jobs: int = 8) -> None:
    BUILD.mkdir(parents=True, exist_ok=True)
    OUT.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        hip_objs = list(ex.map(compile_hip, HIP_SOURCES))
        host_objs = list(ex.map(compile_host, HOST_SOURCES))
    lib = OUT / "libfa_hip.so"
    tmp = lib.with_suffix(".so.tmp")
    run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
         *map(str, host_objs), *map(str, hip_objs), "-Wl,-soname,libfa_hip.so"])
    os.replace(tmp, lib)

    bench_src = PKG_ROOT / "bench" / "fa_bench.hip"
    bench_bin = PKG_ROOT / "bench" / "fa_bench"
    tmp = bench_bin.with_suffix(".tmp")
    run([HIPCC, *HIP_FLAGS, str(bench_src), "-o", str(tmp), f"-L{OUT}", "-lfa_hip",
         "-Wl,-rpath,$ORIGIN/../fused_attn"])
    os.replace(tmp, bench_bin)

    cflags, ldflags = torch_flags()
    ext_obj = BUILD / "ext.cpp.o"
    run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter",
         f"-I{INCLUDE}", "-I/opt/rocm/include", *cflags, "-c", str(CSRC / "ext.cpp"), "-o",
         str(ext_obj)])
    ext = OUT / "_C.so"
    tmp = ext.with_suffix(".so.tmp")
    run(["g++", "-shared", "-fPIC", "-o", str(tmp), str(ext_obj), f"-L{OUT}", "-lfa_hip",
         "-Wl,-rpath,$ORIGIN", *ldflags])
    os.replace(tmp, ext)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    a = ap.parse_args()
    build(a.jobs)
    print(f"built {OUT / 'libfa_hip.so'}, {OUT / '_C.so'} and {PKG_ROOT / 'bench' / 'fa_bench'}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
