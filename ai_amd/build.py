"""Builds the native libraries in-tree.

  ai_amd/_lib/libfa_rocm.so   HIP kernels + C ABI (include/fa_rocm.h), gfx950
  ai_amd/_lib/libfa_synth.so  seeded synthetic inputs (include/fa_synth.h), host only
  ai_amd/_lib/libfiber_host.so  C++ mirror of the reference's tensor/gemma API
                                (ai_amd/host/fiber.hpp) over libfa_rocm.so
  _build/cpp_tests/*          C++ tests of that mirror (tests/cpp), run by
                              tests/test_cpp_host.py on a GPU

Compiles every source on every call (the driver's "does it build" check).
Usage: python -m ai_amd.build [-v]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ai_amd")
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "_lib")
BUILD = os.path.join(ROOT, "_build")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for device code (they are generated
# from ordinary float code at -O3 otherwise).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]

ROCM_SOURCES = ["context.cpp", "matmul.cpp", "model.cpp", "plan.cpp", "gemm.hip", "rowops.hip", "attention.hip", "score.hip", "cluster.hip"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_rocm(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    objs = []
    jobs = []
    for src in ROCM_SOURCES:
        obj = os.path.join(BUILD, src.replace(".", "_") + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        jobs.append([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        for f in [ex.submit(_run, j, verbose) for j in jobs]:
            f.result()
    out = os.path.join(LIB, "libfa_rocm.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


def build_synth(verbose: bool = False) -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libfa_synth.so")
    tmp = out + ".tmp"
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O3", "-std=c++17", "-fPIC", "-fopenmp", "-shared", "-Wall", "-I", INCLUDE,
          os.path.join(CSRC, "synth.cpp"), "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


HOST = os.path.join(PKG, "host")
HOST_SOURCES = ["fiber.cpp", "json.cpp", "tokenizer.cpp", "safetensors.cpp", "cluster.cpp"]
CPP_TESTS = ["test_tensor", "test_gemma", "test_tokenizer", "test_cluster", "test_config"]
CPP_CPU_TESTS = ["test_tokenizer", "test_config", "test_plan"]  # need no GPU
CPP_PLAN_TEST = "test_plan"  # the encoder's host plan (csrc/plan.cpp) alone, no library
CPP_DRIVERS = ["st_dump", "embed_dir"]  # programs the Python tests drive
C_DRIVERS = ["exit_open"]  # C programs the Python tests drive
CPP_TEST_BIN = os.path.join(BUILD, "cpp_tests")


def build_host(verbose: bool = False) -> str:
    """libfiber_host.so (host C++ only; the device work is in libfa_rocm.so)."""
    cxx = shutil.which("g++") or "g++"
    out = os.path.join(LIB, "libfiber_host.so")
    tmp = out + ".tmp"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I", INCLUDE, "-I", HOST,
          *[os.path.join(HOST, f) for f in HOST_SOURCES], "-o", tmp, "-L", LIB, "-lfa_rocm",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, out)
    os.makedirs(CPP_TEST_BIN, exist_ok=True)
    tdir = os.path.join(ROOT, "tests", "cpp")
    # rpath relative to the binary, so the tree can be moved to another host
    rpath = "-Wl,-rpath,$ORIGIN/" + os.path.relpath(LIB, CPP_TEST_BIN)
    jobs = []
    for t in CPP_TESTS + CPP_DRIVERS:
        jobs.append([cxx, "-O2", "-std=c++17", "-Wall", "-I", INCLUDE, "-I", HOST, "-I", tdir,
                     os.path.join(tdir, t + ".cpp"), "-o", os.path.join(CPP_TEST_BIN, t),
                     "-L", LIB, "-lfiber_host", "-lfa_rocm", "-lfa_synth", rpath])
    jobs.append([cxx, "-O2", "-std=c++17", "-Wall", "-I", CSRC, "-I", tdir, os.path.join(tdir, CPP_PLAN_TEST + ".cpp"),
                 os.path.join(CSRC, "plan.cpp"), "-o", os.path.join(CPP_TEST_BIN, CPP_PLAN_TEST)])
    cc = shutil.which("gcc") or "gcc"
    for t in C_DRIVERS:  # plain C callers of the C ABI
        jobs.append([cc, "-O2", "-std=c99", "-Wall", "-I", INCLUDE, os.path.join(tdir, t + ".c"),
                     "-o", os.path.join(CPP_TEST_BIN, t), "-L", LIB, "-lfa_rocm", "-lfa_synth", rpath])
    with cf.ThreadPoolExecutor(len(jobs)) as ex:
        for f in [ex.submit(_run, j, verbose) for j in jobs]:
            f.result()
    return out


def build_oracle(verbose: bool = False) -> None:
    """The CPU oracle is test infrastructure; it is built beside the product."""
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "-j2"], verbose)


def build_all(verbose: bool = False) -> None:
    build_synth(verbose)
    build_rocm(verbose)
    build_host(verbose)
    build_oracle(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", os.listdir(LIB))
