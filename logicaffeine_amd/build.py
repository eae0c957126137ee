"""Build recipe of liblgx (no cmake, no JIT cache: everything lands in-tree).

    lgx_kernels.hsaco  hipcc --genco --offload-arch=gfx950 (device code only)
    liblgx.so          g++ host launcher over the HIP module API

Run as ``python -m logicaffeine_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`.  Both artefacts sit next to this file, which is where
``lgx_ctx_create(dev, NULL, ...)`` looks for the code object.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HSACO = os.path.join(HERE, "lgx_kernels.hsaco")
LIB = os.path.join(HERE, "liblgx.so")

# -ffp-contract=off: no implicit fusion, the float schedule is what the source
# says.  Correctly rounded binary32 division and square root.  Packed-FP32
# instructions disabled (v_pk_*_f32 are never generated).  MFMA destinations
# in VGPRs.
HIP_FLAGS = [
    "--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs (gfx950 allows it): the epilogues read
    # them directly instead of copying each value out of an AGPR first
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd):
    print("[lgx build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_kernels() -> str:
    src = os.path.join(CSRC, "lgx_kernels.hip")
    tmp = HSACO + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, "-I", CSRC, "-o", tmp, src])
    os.replace(tmp, HSACO)
    return HSACO


HOST_SOURCES = ["lgx_host.cpp", "lgx_glue.cpp", "lgx_model.cpp", "lgx_gen.cpp", "lgx_gguf.cpp",
                "lgx_f16gemm.cpp"]
BUILD_DIR = os.path.join(HERE, "_build")


def build_scratch() -> str:
    """lgx_scratch.hip: host code plus a gfx950 code object holding only the
    no-alloc entry point's device scratch array, registered with the HIP
    runtime when liblgx.so loads."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    obj = os.path.join(BUILD_DIR, "lgx_scratch.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", "-O2", "-std=c++17", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", CSRC, "-o", obj, os.path.join(CSRC, "lgx_scratch.hip")])
    return obj


def build_host() -> str:
    srcs = [os.path.join(CSRC, s) for s in HOST_SOURCES]
    scratch_obj = build_scratch()
    tmp = LIB + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off", "-Wall", "-Wextra", "-pthread",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", "-I", CSRC,
          "-o", tmp, *srcs, scratch_obj, f"-L{ROCM}/lib", "-lamdhip64", "-lhipblaslt", f"-Wl,-rpath,{ROCM}/lib", "-ldl"])
    os.replace(tmp, LIB)
    return LIB


def build() -> None:
    build_kernels()
    build_host()


if __name__ == "__main__":
    build()
    sys.exit(0)
