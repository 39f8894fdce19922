"""Build the gfx950 HIP library ``libpulsarlm_amd.so`` in-tree with hipcc, and the
C++ host layer ``_host.so`` (pulsarlm-core's operator signatures over the C ABI,
bound for Python) with g++ against PyTorch-ROCm.

Usage: ``python -m pulsarlm_amd.build [-DNAME=VALUE ...]`` (or ``__graft_entry__.build()``);
extra ``-D`` definitions go to every hipcc compile (measurement builds such as
``-DPLM_MEASURE_SKIP_REDUCTION=1``, whose results are invalid by design).
Every call recompiles; objects go to ``pulsarlm_amd/_build/`` and are linked
in parallel-compiled order into ``pulsarlm_amd/libpulsarlm_amd.so``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libpulsarlm_amd.so"

SOURCES = ["repack.hip", "gemm_decode.hip", "gemm_mfma.hip", "quant.hip", "moe.hip", "routing.hip", "gemm_plain.hip", "capi.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops (v_pk_*_f32) are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


# Per-source flags. The MFMA kernel keeps its accumulators in VGPRs (the VGPR form of
# v_mfma): with the default AGPR form the register allocator splits the accumulator set
# between the two files and copies it back and forth every K step.
SOURCE_FLAGS = {"gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


EXTRA_DEFINES: list[str] = []


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    # The compiler's per-kernel resource report (registers, LDS, scratch) is kept next to
    # the object: tests/test_build.py checks that no kernel spills to scratch.
    cmd = [HIPCC, *FLAGS, *EXTRA_DEFINES, *SOURCE_FLAGS.get(src, []), "-Rpass-analysis=kernel-resource-usage", "-c",
           str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    (BUILD / (Path(src).stem + ".resources.txt")).write_text(res.stderr)
    return obj


HOST_SOURCES = ["host/pulsarlm_ops.cpp", "host/linear.cpp", "host/module.cpp"]
HOST_LIB = PKG / "_host.so"


def _host_flags():
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ext

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in ext.include_paths()] + [f"-I{sysconfig.get_paths()['include']}",
                                                     "-I/opt/rocm/include", f"-I{PKG.parent / 'include'}"]
    return ["-std=c++17", "-O2", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
            "-Wno-unused-parameter", *inc]


def _compile_host(src: str) -> Path:
    obj = BUILD / (Path(src).stem + "_host.o")
    cmd = [os.environ.get("CXX", "g++"), *_host_flags(), "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {src}:\n{res.stderr[-4000:]}")
    return obj


def build_host(objs) -> Path:
    """Link the C++ host layer (pybind module) against libpulsarlm_amd.so and torch."""
    import torch.utils.cpp_extension as ext

    libdirs = ext.library_paths()
    tmp = HOST_LIB.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
           *[f"-L{d}" for d in libdirs], f"-L{PKG}", "-lpulsarlm_amd", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-Wl,-rpath,$ORIGIN",
           *[f"-Wl,-rpath,{d}" for d in libdirs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES) + len(HOST_SOURCES), os.cpu_count() or 4)) as ex:
        dev = [ex.submit(_compile, s) for s in SOURCES]
        host = [ex.submit(_compile_host, s) for s in HOST_SOURCES]
        objs = [f.result() for f in dev]
        host_objs = [f.result() for f in host]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_host(host_objs)
    if verbose:
        print(f"built {LIB} and {HOST_LIB}")
    return LIB


if __name__ == "__main__":
    EXTRA_DEFINES.extend(a for a in sys.argv[1:] if a.startswith("-D"))
    build(verbose=True)
    sys.exit(0)
