"""Build recipe for the native parts of brimkern_amd (no cmake / node-gyp needed).

1. ``csrc/kernels/brik_kernels.hip`` -> ``_build/brik_gfx950.hsaco``  (hipcc --genco, gfx950 only), then
   ``check_lds_reads.py`` on its disassembly (the GEMM's inline-asm LDS reads)
2. ``csrc/brik_scratch.hip`` -> ``_build/brik_scratch.o`` (hipcc -c: the no-allocation scratch array)
3. ``csrc/brik_runtime.cpp`` + ``csrc/brik_embed.S`` (embeds the code object) + that object ->
   ``libbrik.so`` (the C ABI declared in ``include/brik.h``)
4. ``csrc/brik_napi.cc`` -> ``js/brik.node`` (Node N-API addon over libbrik.so, rpath $ORIGIN/..)
5. ``tests/native/host_sanitize.cpp`` + the runtime sources, host code built with AddressSanitizer and
   UndefinedBehaviorSanitizer -> ``tests/native/host_sanitize`` (a test driver, not part of the library;
   skipped when g++ cannot link the sanitizer runtimes)

Run ``python -m brimkern_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
NODE_INC = "/usr/include/node"

HSACO = os.path.join(BUILD, "brik_gfx950.hsaco")
SCRATCH_OBJ = os.path.join(BUILD, "brik_scratch.o")
LIB = os.path.join(PKG, "libbrik.so")
ADDON = os.path.join(PKG, "js", "brik.node")
SANITIZE_SRC = os.path.join(ROOT, "tests", "native", "host_sanitize.cpp")
SANITIZE_BIN = os.path.join(ROOT, "tests", "native", "host_sanitize")

# Device flags. packed-fp32-ops is switched off: the compiler would otherwise fuse pairs of f32
# operations into v_pk_* forms.
HIP_DEVICE_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=fast",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    subprocess.check_call(cmd)


def build_hsaco(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    src = os.path.join(CSRC, "kernels", "brik_kernels.hip")
    tmp = HSACO + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "--genco", "--no-gpu-bundle-output", *HIP_DEVICE_FLAGS,
          "-o", tmp, src], verbose)
    os.replace(tmp, HSACO)
    return HSACO


def build_scratch(verbose=False):
    """``csrc/brik_scratch.hip`` (the fixed device scratch of the no-allocation entry point and its
    address lookup) as a HIP object, linked into libbrik.so."""
    os.makedirs(BUILD, exist_ok=True)
    tmp = SCRATCH_OBJ + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", *HIP_DEVICE_FLAGS, "-Wall",
          "-o", tmp, os.path.join(CSRC, "brik_scratch.hip")], verbose)
    os.replace(tmp, SCRATCH_OBJ)
    return SCRATCH_OBJ


def build_lib(verbose=False):
    tmp = LIB + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
          f'-DBRIK_HSACO_PATH="{HSACO}"',
          os.path.join(CSRC, "brik_runtime.cpp"), os.path.join(CSRC, "brik_embed.S"), SCRATCH_OBJ,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
          "-Wl,--no-undefined", "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_addon(verbose=False):
    src = os.path.join(CSRC, "brik_napi.cc")
    if not os.path.exists(src) or not os.path.exists(os.path.join(NODE_INC, "node_api.h")):
        return None
    tmp = ADDON + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-Wextra", "-DNODE_GYP_MODULE_NAME=brik",
          "-I", NODE_INC, "-I", os.path.join(ROOT, "include"), src,
          "-L", PKG, "-lbrik", "-Wl,-rpath,$ORIGIN/..", "-o", tmp], verbose)
    os.replace(tmp, ADDON)
    return ADDON


def build_host_sanitize(verbose=False):
    """The runtime's host code with ASan + UBSan (g++, host only; the kernels stay the ordinary code
    object), linked with the driver that exercises every entry point (tests/test_host_sanitize.py)."""
    if not os.path.exists(SANITIZE_SRC):
        return None
    tmp = SANITIZE_BIN + ".tmp"
    try:
        _run(["g++", "-O1", "-g", "-std=c++17", "-Wall", "-Wextra", "-fno-omit-frame-pointer",
              "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-static-libasan",
              "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
              f'-DBRIK_HSACO_PATH="{HSACO}"', SANITIZE_SRC,
              os.path.join(CSRC, "brik_runtime.cpp"), os.path.join(CSRC, "brik_embed.S"), SCRATCH_OBJ,
              "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
              "-o", tmp], verbose)
    except (subprocess.CalledProcessError, OSError):
        if verbose:
            print("+ host sanitizer driver skipped: g++ could not build it", flush=True)
        return None
    os.replace(tmp, SANITIZE_BIN)
    return SANITIZE_BIN


def check_hsaco(verbose=False):
    """The GEMM kernels' inline-asm LDS reads must be waited for before their registers are touched
    (check_lds_reads.py); a violation fails the build."""
    from brimkern_amd.check_lds_reads import check_file
    bad = check_file(HSACO)
    if bad:
        raise RuntimeError("LDS-read register check failed:\n" + "\n".join(bad[:10]))
    if verbose:
        print("+ LDS-read register check: ok", flush=True)


def build(verbose=False):
    build_hsaco(verbose)
    check_hsaco(verbose)
    build_scratch(verbose)
    build_lib(verbose)
    build_addon(verbose)
    build_host_sanitize(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
