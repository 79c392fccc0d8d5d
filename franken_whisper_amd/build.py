"""In-tree build of the native libraries.

  lib/libfwhip.so   HIP kernels + C ABI (include/fwhip.h), gfx950 only
  lib/libfwsynth.so seeded synthetic weights/audio (host C, OpenMP)

Compiles every time it is called (the driver's "does it build" check); hipcc
cross-compiles gfx950 code objects without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["fwhip.hip", "dec_kernels.hip", "load_kernels.hip", "encoder.hip", "enc_kernels.hip", "enc_gemm.hip", "dec_fast.hip", "dec_gemv16.hip", "enc_tome.hip", "mel.hip", "ggml.hip", "dec_window.hip", "transcribe.hip"]
# Packed-FP32 instructions are disabled for every HIP translation unit; exact
# reference epilogues need -ffp-contract=off (Rust never contracts a*b+c).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-Wno-unknown-warning-option", "-Wno-unused-value",
    "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_synth():
    os.makedirs(LIBDIR, exist_ok=True)
    out = os.path.join(LIBDIR, "libfwsynth.so")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-std=gnu11",
          os.path.join(CSRC, "synth.c"), "-o", out, "-lm"])
    return out


def build_hip(jobs: int | None = None):
    """Each translation unit compiles to its own object in parallel (objects
    under _build/, outside the package), then one link step."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(ROOT, "_build", "hip")
    os.makedirs(objdir, exist_ok=True)
    out = os.path.join(LIBDIR, "libfwhip.so")
    tmp = out + ".tmp"
    cflags = [f for f in HIP_FLAGS if f != "-shared"]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]

    def compile_one(i):
        _run([HIPCC] + cflags + ["-c", os.path.join(CSRC, HIP_SOURCES[i]), "-o", objs[i]])

    n = jobs or min(len(HIP_SOURCES), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=n) as ex:
        list(ex.map(compile_one, range(len(HIP_SOURCES))))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp])
    os.replace(tmp, out)
    return out


def build_hip_asan(jobs: int | None = None):
    """The same library with AddressSanitizer and UndefinedBehaviorSanitizer
    on its host code only (the ggml parser, argument checks, the drivers; the
    gfx950 code objects are built as usual), into _build/asan/libfwhip.so.
    The CPU tests run against it with FWHIP_LIB pointing there and clang's
    ASan runtime preloaded (see the DESIGN notes); it is never shipped."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(ROOT, "_build", "asan")
    os.makedirs(objdir, exist_ok=True)
    out = os.path.join(objdir, "libfwhip.so")
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]
    cflags = [f for f in HIP_FLAGS if f != "-shared"] + san
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]

    def compile_one(i):
        _run([HIPCC] + cflags + ["-c", os.path.join(CSRC, HIP_SOURCES[i]), "-o", objs[i]])

    n = jobs or min(len(HIP_SOURCES), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=n) as ex:
        list(ex.map(compile_one, range(len(HIP_SOURCES))))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + san + objs + ["-o", out])
    return out


def build_all():
    build_synth()
    build_hip()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for w in what:
        {"all": build_all, "synth": build_synth, "hip": build_hip, "asan": build_hip_asan}[w]()
