#!/usr/bin/env python3
"""Builds flash-train for MI355X in-tree with hipcc (gfx950).

Outputs (all git-ignored, all shipped to the GPU box with the tree):
  flash_train/libflash_train.so           the C-ABI library (exports the ftrain* API only)
  flash_train/libflash_train_testing.so   same objects plus host-only test hooks
  flash_train/torch/_flash_train_torch*.so the flash_train.torch.gemm binding
  bench/plan_overhead                     C++ host-overhead probe used by bench.py

Usage: python build.py [--jobs N] [--no-torch] [--incremental]
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "_build")
PKG = os.path.join(HERE, "flash_train")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-fvisibility-inlines-hidden",
    "-Wall",
    "-Wno-unused-function",
    f"-I{os.path.join(HERE, 'csrc', 'include')}",
    f"-I{os.path.join(REPO, 'include')}",
]
# Device code: gfx950 only, and no packed-FP32 instructions.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

LIB_SOURCES = [
    "csrc/runtime/error.cpp",
    "csrc/runtime/values.cpp",
    "csrc/runtime/pattern.cpp",
    "csrc/runtime/cache.cpp",
    "csrc/runtime/plan.cpp",
    "csrc/runtime/handle.cpp",
    "csrc/runtime/trace.cpp",
    "csrc/gemm/catalog.cpp",
    "csrc/gemm/problem.cpp",
    "csrc/gemm/finder.cpp",
    "csrc/gemm/primitives.cpp",
    "csrc/gemm/grouped.cpp",
    "csrc/gemm/kernels.hip",
    "csrc/gemm/kernels_layout_tn.hip",
    "csrc/gemm/kernels_layout_nt.hip",
    "csrc/gemm/kernels_layout_tt.hip",
    "csrc/gemm/kernels_m16_nn.hip",
    "csrc/gemm/kernels_m16_tn.hip",
    "csrc/gemm/kernels_m16_nt.hip",
    "csrc/gemm/kernels_m16_tt.hip",
    "csrc/gemm/kernels_half_bf16_nn.hip",
    "csrc/gemm/kernels_half_bf16_tn.hip",
    "csrc/gemm/kernels_half_bf16_nt.hip",
    "csrc/gemm/kernels_half_bf16_tt.hip",
    "csrc/gemm/kernels_half_fp16_nn.hip",
    "csrc/gemm/kernels_half_fp16_tn.hip",
    "csrc/gemm/kernels_half_fp16_nt.hip",
    "csrc/gemm/kernels_half_fp16_tt.hip",
    "csrc/gemm/kernels_dma32.hip",
    "csrc/gemm/kernels_dma32_tb.hip",
    "csrc/gemm/kernels_dma32_ta.hip",
    "csrc/gemm/kernels_half_dma_bf16.hip",
    "csrc/gemm/kernels_half_dma_fp16.hip",
    "csrc/gemm/kernels_gemv_half.hip",
    "csrc/gemm/kernels_deepk.hip",
    "csrc/api/c_api.cpp",
    "csrc/api/scratch.hip",
]
TESTING_SOURCES = ["csrc/api/testing_api.cpp"]


def run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout)
        raise SystemExit(f"build step failed: {cmd[-1]}")


# Host-code sanitizer for a checking build (None for the product build); device code is unchanged.
SANITIZER = None


def out_dir() -> str:
    return os.path.join(BUILD, SANITIZER) if SANITIZER else BUILD


def sanitizer_flags() -> list[str]:
    flags = [f"-fsanitize={SANITIZER}", "-fno-omit-frame-pointer", "-g"]
    if SANITIZER == "undefined":
        flags.append("-fno-sanitize-recover=undefined")
    return flags


def obj_path(src: str) -> str:
    return os.path.join(out_dir(), src.replace("/", "_") + ".o")


def up_to_date(out: str) -> bool:
    """True when `out` and its dependency file exist and no listed dependency is newer."""
    dep = out + ".d"
    if not (os.path.exists(out) and os.path.exists(dep)):
        return False
    with open(dep) as f:
        text = f.read().replace("\\\n", " ")
    deps = text.split(":", 1)[1].split() if ":" in text else []
    t = os.path.getmtime(out)
    return all(os.path.exists(x) and os.path.getmtime(x) <= t for x in deps)


INCREMENTAL = False


def compile_one(src: str) -> str:
    out = obj_path(src)
    if INCREMENTAL and up_to_date(out):
        return out
    cmd = [HIPCC, *COMMON, "-MD", "-MF", out + ".d"]
    if src.endswith(".hip"):
        cmd += ["-x", "hip", *DEVICE]
        if SANITIZER:
            cmd += [x for f in sanitizer_flags() for x in ("-Xarch_host", f)]
    elif SANITIZER:
        cmd += ["-O1", *sanitizer_flags()]
    cmd += ["-c", os.path.join(HERE, src), "-o", out]
    run(cmd)
    return out


def link_shared(objs: list[str], out: str, soname: str) -> None:
    # Export the ftrain* C entry points only; library-internal and C++
    # standard-library template symbols stay local.
    script = os.path.join(BUILD, "exports.map")
    with open(script, "w") as f:
        f.write("{ global: ftrain*; local: *; };\n")
    san = [f"-fsanitize={SANITIZER}", "-shared-libsan"] if SANITIZER else []
    run([HIPCC, f"-Wl,--version-script={script}", "-shared", "-fPIC", f"--offload-arch={ARCH}", *san, *objs, "-o", out,
         f"-Wl,-soname,{soname}", f"-L{ROCM}/lib", "-lroctx64", f"-Wl,-rpath,{ROCM}/lib",
         *([] if SANITIZER else ["-Wl,--no-undefined"])])


def torch_flags() -> tuple[list[str], list[str]]:
    import torch.utils.cpp_extension as ce  # imported lazily: only the binding needs torch

    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    libdirs = ce.library_paths()
    abi = "1" if __import__("torch")._C._GLIBCXX_USE_CXX11_ABI else "0"
    cflags = inc + ["-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                    "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_flash_train_torch",
                    "-Wno-unused-result", "-Wno-deprecated-declarations"]
    ldflags = [f"-L{d}" for d in libdirs] + [f"-Wl,-rpath,{d}" for d in libdirs] + [
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python"]
    return cflags, ldflags


def build_torch_binding() -> None:
    cflags, ldflags = torch_flags()
    src = os.path.join(PKG, "torch", "csrc", "flash_train_torch.cpp")
    obj = os.path.join(BUILD, "flash_train_torch.o")
    run([HIPCC, *COMMON, *cflags, "-c", src, "-o", obj])
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "torch", "_flash_train_torch" + suffix)
    run([HIPCC, "-shared", "-fPIC", obj, "-o", out, f"-L{PKG}", "-lflash_train", "-Wl,-rpath,$ORIGIN/..",
         *ldflags, f"-L{ROCM}/lib"])


def build_plan_overhead() -> None:
    os.makedirs(os.path.join(HERE, "bench"), exist_ok=True)
    src = os.path.join(HERE, "bench", "plan_overhead.hip")
    out = os.path.join(HERE, "bench", "plan_overhead")
    run([HIPCC, "-O2", "-std=c++17", *DEVICE, f"-I{os.path.join(REPO, 'include')}", src, "-o", out, f"-L{PKG}",
         "-lflash_train", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{ROCM}/lib"])


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--no-torch", action="store_true")
    ap.add_argument("--incremental", action="store_true",
                    help="skip sources whose object is newer than every file it includes")
    ap.add_argument("--host-sanitizer", choices=("address", "undefined"),
                    help="a checking build: both libraries with their host code under this sanitizer (device "
                         "code unchanged), into _build/<sanitizer>/, for the CPU suite: FTRAIN_LIBRARY_DIR="
                         "flash-train_amd/_build/<sanitizer> LD_PRELOAD=<clang's asan or ubsan_standalone runtime> "
                         "python -m pytest tests -m 'not gpu'")
    args = ap.parse_args(argv)
    global INCREMENTAL, SANITIZER
    INCREMENTAL = args.incremental
    SANITIZER = args.host_sanitizer
    os.makedirs(out_dir(), exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(args.jobs) as pool:
        lib_objs = list(pool.map(compile_one, LIB_SOURCES))
        test_objs = list(pool.map(compile_one, TESTING_SOURCES))
    lib_dir = out_dir() if SANITIZER else PKG
    link_shared(lib_objs, os.path.join(lib_dir, "libflash_train.so"), "libflash_train.so")
    link_shared(lib_objs + test_objs, os.path.join(lib_dir, "libflash_train_testing.so"), "libflash_train_testing.so")
    if SANITIZER:
        return
    build_plan_overhead()
    if not args.no_torch:
        build_torch_binding()


if __name__ == "__main__":
    main()
