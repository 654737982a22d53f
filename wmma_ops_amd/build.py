"""Build the gfx950 C-ABI library and the PyTorch extension in-tree.

    python -m wmma_ops_amd.build            # or wmma_ops_amd.build.build()

Outputs (inside the package directory, next to this file):
    libwmma_ops_amd.so                      HIP kernels + C-ABI (include/wmma_ops_amd.h)
    _C.cpython-*.so                         pybind/torch layer, links the library above
    libwmma_calib.so                        calibration kernels (include/wmma_calib.h)

Only hipcc (for *.hip, --offload-arch=gfx950) and the host C++ compiler are used; no
JIT cache, so the built files travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

LIB_NAME = "libwmma_ops_amd.so"
EXT_NAME = "_C" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")

HIP_SOURCES = ["capi.hip", "gemm.hip", "w4a16.hip", "flash_fwd.hip", "flash_bwd.hip"]
HOST_SOURCES = ["plan.cpp"]

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # No packed-FP32 VALU instructions anywhere in this library's device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        l for l in res.stdout.splitlines()
        if "packed-fp32-ops" not in l and "unknown target feature" not in l.lower()
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_library(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        jobs.append(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-c",
                     os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(len(jobs), 8)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    lib = os.path.join(PKG, LIB_NAME)
    tmp = lib + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, lib)
    return lib


CALIB_NAME = "libwmma_calib.so"


def build_calib(verbose: bool = False) -> str:
    """The calibration kernels (include/wmma_calib.h), a library of their own."""
    os.makedirs(BUILD, exist_ok=True)
    obj = os.path.join(BUILD, "calib.hip.o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "calib.hip"), "-o", obj], verbose)
    lib = os.path.join(PKG, CALIB_NAME)
    tmp = lib + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj], verbose)
    os.replace(tmp, lib)
    return lib


def build_extension(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension as ce

    try:
        incs = ce.include_paths(device_type="cuda")
        libdirs = ce.library_paths(device_type="cuda")
    except TypeError:  # older signature
        incs = ce.include_paths(True)
        libdirs = ce.library_paths(True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    py_inc = sysconfig.get_paths()["include"]
    out = os.path.join(PKG, EXT_NAME)
    tmp = out + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        # HIP runtime headers used by torch's HIP stream API target the AMD platform.
        "-D__HIP_PLATFORM_AMD__=1",
        "-Wno-deprecated-declarations",
        *[f"-I{p}" for p in incs], f"-I{py_inc}",
        os.path.join(CSRC, "torch_ext.cpp"),
        *[f"-L{p}" for p in libdirs], f"-L{PKG}",
        "-lwmma_ops_amd", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-ltorch_python", f"-L{ROCM}/lib", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        "-o", tmp,
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)
    build_calib(verbose)


# ------------------------------------------------------------- host sanitizer build --
# AddressSanitizer + UndefinedBehaviorSanitizer on the CPU side only: the C-ABI's argument
# validation and host code (capi.hip and the host halves of the kernel files), the planner
# (plan.cpp) and the plain-C oracle.  Device code is built exactly as in the product
# (every -fsanitize= applies to the host pass only).  Outputs go to _build/sanitize/; the
# product library is untouched.
SAN_DIR = os.path.join(BUILD, "sanitize")
LLVM_BIN = os.path.join(ROCM, "lib", "llvm", "bin")
SAN_HOST = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
            "-fno-omit-frame-pointer"]


def _asan_runtime() -> str:
    out = subprocess.run([os.path.join(LLVM_BIN, "clang"), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         stdout=subprocess.PIPE, text=True, check=True).stdout.strip()
    if not os.path.isfile(out):  # older layouts keep it under lib/linux
        import glob
        hits = glob.glob(os.path.join(ROCM, "lib", "llvm", "lib", "clang", "*", "lib", "linux",
                                      "libclang_rt.asan-x86_64.so"))
        out = hits[0] if hits else out
    return out


def build_sanitized(verbose: bool = False) -> dict:
    """Host-sanitized copies of the C-ABI library and the C oracle (clang for every host
    pass, so one ASan runtime serves both)."""
    os.makedirs(SAN_DIR, exist_ok=True)
    host_flags = [x for f in SAN_HOST for x in ("-Xarch_host", f)]
    objs, jobs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(SAN_DIR, src + ".o")
        objs.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, *host_flags, "-g", "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(SAN_DIR, src + ".o")
        objs.append(obj)
        jobs.append([os.path.join(LLVM_BIN, "clang++"), "-O1", "-g", "-std=c++17", "-fPIC", "-Wall",
                     *SAN_HOST, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(len(jobs), 8)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    lib = os.path.join(SAN_DIR, LIB_NAME)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", *host_flags,
          "-o", lib, *objs], verbose)
    odir = os.path.join(ROOT, "oracle")
    olib = os.path.join(SAN_DIR, "liboracle.so")
    _run([os.path.join(LLVM_BIN, "clang"), "-O1", "-g", "-fPIC", "-std=c11", "-Wall",
          "-ffp-contract=off", *SAN_HOST, "-shared-libsan", "-shared", "-o", olib,
          os.path.join(odir, "gemm_ref.c"), os.path.join(odir, "int4_ref.c"), "-lm"], verbose)
    return {"library": lib, "oracle": olib, "runtime": _asan_runtime()}


def run_sanitized_tests(verbose: bool = False) -> int:
    """The CPU suites that drive the sanitized code -- tests/test_capi.py (every C-ABI
    validation path, the planner) and tests/test_oracle.py (the C oracle) -- with the
    sanitized libraries in place of the product ones and the ASan runtime preloaded.  Any
    ASan or UBSan report aborts the process (halt_on_error), so a clean exit means none."""
    paths = build_sanitized(verbose)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": paths["runtime"],
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "WMMA_OPS_AMD_LIBRARY": paths["library"],
        "WMMA_ORACLE_LIBRARY": paths["oracle"],
    })
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           os.path.join(ROOT, "tests", "test_capi.py"), os.path.join(ROOT, "tests", "test_oracle.py")]
    return subprocess.run(cmd, cwd=ROOT, env=env).returncode


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        sys.exit(run_sanitized_tests(verbose="-v" in sys.argv))
    build(verbose="-v" in sys.argv)
    print("built", os.path.join(PKG, LIB_NAME), os.path.join(PKG, EXT_NAME))
