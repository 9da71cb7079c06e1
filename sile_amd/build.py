"""Builds libsile_hip.so in-tree.

1. Each kernels/<name>.hip is compiled for gfx950 into a raw ELF code object
   sile_amd/_build/<name>.hsaco (hipcc --genco --no-gpu-bundle-output).
2. The host runtime (runtime.cpp, ops.cpp, llir.cpp, tile_ir.cpp) is
   compiled with g++ against the HIP runtime headers; runtime.cpp assembles
   the code objects into the library image with .incbin.  launch_noalloc.hip
   (host code plus the device array its entry point uses) is compiled by
   hipcc for the host and gfx950.
3. The objects are linked into sile_amd/libsile_hip.so against libamdhip64.

Run: python -m sile_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
KDIR = os.path.join(CSRC, "kernels")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libsile_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNELS = ["dsl", "softmax", "gemm", "attention", "flash_attn"]
HOST_SOURCES = ["runtime.cpp", "ops.cpp", "llir.cpp", "tile_ir.cpp"]
HIP_HOST_SOURCES = ["launch_noalloc.hip"]

# Device code: gfx950 only; packed-fp32 instructions disabled (the compiler
# would otherwise form v_pk_{add,mul,fma}_f32 from scalar float code).
DEVICE_FLAGS = [
    "--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def build_kernel(name: str) -> str:
    src = os.path.join(KDIR, name + ".hip")
    out = os.path.join(BUILD, name + ".hsaco")
    _run([HIPCC, *DEVICE_FLAGS, "-o", out + ".tmp", src])
    os.replace(out + ".tmp", out)
    return out


def build_host(src_name: str) -> str:
    src = os.path.join(CSRC, src_name)
    obj = os.path.join(BUILD, src_name + ".o")
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
          f'-DSILE_CO_DIR="{BUILD}"', "-c", src, "-o", obj])
    return obj


def build_hip_host(src_name: str) -> str:
    """A host source with device data of its own: hipcc, host + gfx950."""
    src = os.path.join(CSRC, src_name)
    obj = os.path.join(BUILD, src_name + ".o")
    _run([HIPCC, "-c", "-fPIC", "-O2", "-std=c++17", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wall", "-Wno-unused-command-line-argument", src, "-o", obj])
    return obj


def build(verbose: bool = True) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(KERNELS))) as ex:
        for path in ex.map(build_kernel, KERNELS):
            if verbose:
                print("built", os.path.relpath(path, ROOT), flush=True)
    objs = [build_host(s) for s in HOST_SOURCES] + [build_hip_host(s) for s in HIP_HOST_SOURCES]
    # Export the C ABI (sile_hip_*) and nothing else.
    vscript = os.path.join(BUILD, "exports.map")
    with open(vscript, "w") as f:
        f.write("{\n  global: sile_hip_*;\n  local: *;\n};\n")
    tmp = LIB + ".tmp"
    _run(["g++", "-shared", "-o", tmp, *objs, f"-L{ROCM}/lib", "-lamdhip64", "-lhiprtc",
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,--no-undefined", f"-Wl,--version-script={vscript}"])
    os.replace(tmp, LIB)
    if verbose:
        print("built", os.path.relpath(LIB, ROOT), flush=True)
    return LIB


def clean():
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build()
