"""Builds the gfx950 shared library and the ``seera_cuda`` Python module in-tree.

  libseera_hip.so        HIP kernels + the C ABI of include/seera_hip.h
                         (hipcc --offload-arch=gfx950)
  seera_cuda*.so         pybind11 module with the reference's function names
                         (g++, host only, linked against libseera_hip.so)

Run ``python -m ml_framework_amd.build`` (or ``__graft_entry__.build()``).
Cross-compiles without a GPU.
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
OBJ = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

LIB_NAME = "libseera_hip.so"
HIP_SOURCES = ["gemm.hip", "conv.hip", "conv_band.hip", "conv_stream.hip", "conv_split.hip", "conv_phase2.hip", "conv_stride2.hip", "conv_wgrad.hip", "conv_wgrad_s2.hip", "conv_bwd_fused.hip", "memory.hip", "pool.hip", "tensor_ops.hip", "noalloc.hip", "runtime.cpp", "capi.cpp",
               "capi_tensor_ops.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n{' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _obj(src: str) -> str:
    return os.path.join(OBJ, os.path.splitext(src)[0] + ".o")


def _compile_hip(src: str) -> str:
    out = _obj(src)
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", out])
    return out


def module_filename() -> str:
    return "seera_cuda" + sysconfig.get_config_var("EXT_SUFFIX")


def build(jobs: int | None = None) -> None:
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile_hip, HIP_SOURCES))
    lib = os.path.join(PKG, LIB_NAME)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", lib + ".tmp"])
    os.replace(lib + ".tmp", lib)

    import pybind11

    mod = os.path.join(PKG, module_filename())
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
        f"-I{os.path.join(ROOT, 'include')}",
        os.path.join(CSRC, "seera_cuda_module.cpp"),
        f"-L{PKG}", "-lseera_hip", "-Wl,-rpath,$ORIGIN",
        "-o", mod + ".tmp",
    ])
    os.replace(mod + ".tmp", mod)


if __name__ == "__main__":
    build()
    print("built", os.path.join(PKG, LIB_NAME), "and", module_filename())
