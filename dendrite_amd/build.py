"""Builds libdendrite_hip.so in-tree with hipcc for gfx950, and beside it
libdendrite_testdata.so, the seeded input generators of the tests and
benchmarks (host code only, include/dendrite_testdata.h; not part of the
backend).

Usage: python -m dendrite_amd.build  (or dendrite_amd.build.build()).
Every call compiles from scratch; objects go to dendrite_amd/_build/.

python -m dendrite_amd.build --sanitize builds a second library,
dendrite_amd/_build_san/libdendrite_hip.so, whose host code (api, planner,
block model, synth) carries AddressSanitizer and UndefinedBehaviorSanitizer
(the kernels are built as usual).  Load it in place of the product library
with the sanitizer runtime preloaded; the command it prints runs the CPU test
suite that way.
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
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libdendrite_hip.so")
TESTDATA_LIB = os.path.join(PKG, "libdendrite_testdata.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{os.path.join(ROOT, 'include')}"]
# Packed FP32 VALU forms are kept out of the generated code.  The kernels do
# not rely on IEEE NaN semantics (inputs are finite; NaN inputs give NaN or
# unspecified outputs), so the IEEE mode bit is off: fmax then needs no
# operand canonicalisation.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-fno-honor-nans", "-mno-amdgpu-ieee"]
HOST = ["-D__HIP_PLATFORM_AMD__", f"-I{os.path.join(ROCM, 'include')}", "-x", "c++"]

# Host-only instrumentation: every -fsanitize= on a hipcc line sits behind
# -Xarch_host, so no device code is built with it.
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]
SAN_BUILD = os.path.join(PKG, "_build_san")
SAN_LIB = os.path.join(SAN_BUILD, "libdendrite_hip.so")

HIP_SOURCES = ["decode_kernels.hip", "write_kernels.hip"]
HOST_SOURCES = ["api.cpp", "planner.cpp", "block_model.cpp"]
TESTDATA_SOURCES = ["synth.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{msg}")


def build(verbose: bool = False, sanitize: bool = False) -> str:
    """Compile every source and link the shared library; returns its path.
    sanitize: the host-sanitized library under _build_san/ instead."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    bdir, lib = (SAN_BUILD, SAN_LIB) if sanitize else (BUILD, LIB)
    shutil.rmtree(bdir, ignore_errors=True)
    os.makedirs(bdir, exist_ok=True)
    host_flags = [*HOST, *SANITIZE] if sanitize else HOST
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(bdir, src + ".o")
        jobs.append(([HIPCC, *COMMON, *DEVICE, "-c", os.path.join(CSRC, src), "-o", obj], obj))
    for src in HOST_SOURCES:
        obj = os.path.join(bdir, src + ".o")
        jobs.append(([HIPCC, *COMMON, *host_flags, "-c", os.path.join(CSRC, src), "-o", obj], obj))
    td_objs = [os.path.join(bdir, src + ".o") for src in TESTDATA_SOURCES]
    td_jobs = [[HIPCC, *COMMON, *HOST, "-c", os.path.join(CSRC, src), "-o", obj]
               for src, obj in zip(TESTDATA_SOURCES, td_objs)] if not sanitize else []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs) + len(td_jobs))) as ex:
        for fut in [ex.submit(_run, cmd) for cmd in [c for c, _ in jobs] + td_jobs]:
            fut.result()
    if td_jobs:
        _run([HIPCC, "-shared", "-o", TESTDATA_LIB + ".tmp", *td_objs, "-lpthread"])
        os.replace(TESTDATA_LIB + ".tmp", TESTDATA_LIB)
    tmp = lib + ".tmp"
    link_san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-shared-libsan"] if sanitize else []
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", *link_san, "-o", tmp, *[o for _, o in jobs],
          "-lpthread"])
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


def sanitizer_runtime() -> str:
    """The clang AddressSanitizer runtime the sanitized library links."""
    proc = subprocess.run([os.path.join(ROCM, "llvm", "bin", "clang"), "-print-file-name=",
                           "--rtlib=compiler-rt"], capture_output=True, text=True)
    base = os.path.join(proc.stdout.strip(), "lib", "linux") if proc.returncode == 0 else ""
    path = os.path.join(base, "libclang_rt.asan-x86_64.so")
    if not os.path.exists(path):
        raise RuntimeError(f"AddressSanitizer runtime not found at {path!r}")
    return path


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        build(verbose=True, sanitize=True)
        print("run the CPU tests on it with:\n"
              f"  LD_PRELOAD={sanitizer_runtime()} DENDRITE_HIP_LIB={SAN_LIB} "
              "ASAN_OPTIONS=detect_leaks=0 python -m pytest tests -m 'not gpu' -q")
    else:
        build(verbose=True)
    sys.exit(0)
