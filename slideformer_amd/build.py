"""Build recipe for the in-tree HIP library ``slideformer_amd/lib/libslideformer_amd.so``.

Usage: ``python -m slideformer_amd.build`` (also called by ``__graft_entry__.build()``);
it also writes the small-grid test build ``lib/libslideformer_amd_smallgrid.so``, the
stream-probe library ``lib/libslideformer_amd_probe.so`` (bench only) and the C test
driver ``tests/native/_build/device_from_c``.

The library is one HIP translation unit compiled for gfx950 only.  Flags:
  -ffp-contract=off       every FMA in the kernels is an explicit fmaf(), so the
                          op order matches the reference CPU Adam exactly;
  no fast-math flags      fp32 division and sqrt stay correctly rounded and
                          denormals are kept;
  -packed-fp32-ops off    no v_pk_{add,mul,fma}_f32 in the generated code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_NAME = "libslideformer_amd.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
SOURCES = [os.path.join(CSRC, "layer_adam.hip"), os.path.join(CSRC, "pipeline.hip"),
           os.path.join(CSRC, "disk_offload.hip")]
ARCH = "gfx950"

BASE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def build_library(out: str = LIB_PATH, defines: dict | None = None, verbose: bool = False,
                  sources: list | None = None) -> str:
    """Compile the library for gfx950 into ``out`` (atomically replaced)."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *BASE_FLAGS]
    for k, v in (defines or {}).items():
        cmd.append(f"-D{k}={v}")
    cmd += ["-I", os.path.join(REPO_DIR, "include"), "-o", tmp, *(sources or SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with code {res.returncode}")
    os.replace(tmp, out)
    return out


# A build with tiny grid caps, loaded only by the GPU tests: the update kernel's
# grid-stride loop (taken by the product build only above 2^34 elements per
# call), la_adam_update_multi's batch splits and the own grid-stride launch of
# a segment too large for one batch (above LA_MAX_GRID / 2 runs: 2^33 elements
# in the product build, 32 runs = 8192 elements here) and the grad norm's
# many-trip loop then run at test sizes.  Same sources, same flags; only these
# launch limits differ.
SMALL_GRID_LIB = os.path.join(LIB_DIR, "libslideformer_amd_smallgrid.so")
SMALL_GRID_DEFINES = {"LA_MAX_GRID": 64, "LA_NORM_MAX_GRID": 2}


# The update kernel's memory-ceiling probes (csrc/stream_probe.hip: its exact
# memory side with the arithmetic removed), loaded only by
# `bench.py --update-ceiling`; a library of their own, so that the product
# library holds no measurement-only kernels.
PROBE_LIB = os.path.join(LIB_DIR, "libslideformer_amd_probe.so")
PROBE_SOURCES = [os.path.join(CSRC, "stream_probe.hip")]


# A plain C program that runs the step on the GPU through the C-ABI alone
# (HIP runtime API for memory, no torch); run by the GPU tests.
C_DRIVER_SRC = os.path.join(REPO_DIR, "tests", "native", "device_from_c.c")
C_DRIVER = os.path.join(REPO_DIR, "tests", "native", "_build", "device_from_c")


def build_c_driver(verbose: bool = False) -> str:
    """Compile tests/native/device_from_c.c as C11 with gcc against the header and the library."""
    gcc = shutil.which("gcc")
    if gcc is None:
        raise RuntimeError("gcc not found")
    os.makedirs(os.path.dirname(C_DRIVER), exist_ok=True)
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    cmd = [gcc, "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(REPO_DIR, "include"), "-I", os.path.join(rocm, "include"), C_DRIVER_SRC,
           "-L", LIB_DIR, "-lslideformer_amd", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../../slideformer_amd/lib", f"-Wl,-rpath,{os.path.join(rocm, 'lib')}",
           "-o", C_DRIVER + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"gcc failed with code {res.returncode}")
    os.replace(C_DRIVER + ".tmp", C_DRIVER)
    return C_DRIVER


def build_all(verbose: bool = False) -> list:
    """The product library, the small-grid test build, the stream probes and the C test driver."""
    return [build_library(verbose=verbose),
            build_library(out=SMALL_GRID_LIB, defines=SMALL_GRID_DEFINES, verbose=verbose),
            build_library(out=PROBE_LIB, sources=PROBE_SOURCES, verbose=verbose),
            build_c_driver(verbose=verbose)]


if __name__ == "__main__":
    for path in build_all(verbose=True):
        print(path)
