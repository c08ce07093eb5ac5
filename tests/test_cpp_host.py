"""The C++ host mirror of the reference's tensor/gemma API (ai_amd/host).

The tests run the C++ test binaries built from tests/cpp (each restates
reference tests: tensor/rope_test.go, tensor/attention_test.go,
tensor/matmul_fused_test.go, internal/blas/gemm_test.go,
models/gemma/gemma_test.go on the GPU; tokenizer/synthetic_test.go and
tokenizer/tokenizer_test.go plus Hugging Face golden ids on the CPU), and
check that the mirror library and its tests were built and link against the
product library.
"""
import ctypes
import os
import subprocess

import pytest

from ai_amd import build as B

BINARIES = [os.path.join(B.CPP_TEST_BIN, t) for t in B.CPP_TESTS]


def _need(path):
    if not os.path.exists(path):
        pytest.fail(f"{path} is missing: run __graft_entry__.build() first")


def test_host_library_loads():
    lib = os.path.join(B.LIB, "libfiber_host.so")
    _need(lib)
    ctypes.CDLL(lib)  # resolves libfa_rocm.so through its rpath
    for b in BINARIES:
        _need(b)


def _run(name):
    binary = os.path.join(B.CPP_TEST_BIN, name)
    _need(binary)
    print(f"running {binary}", flush=True)
    r = subprocess.run([binary], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=110,
                       cwd=B.ROOT)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "--- FAIL" not in r.stdout


@pytest.mark.parametrize("name", B.CPP_CPU_TESTS)
def test_cpp_host_cpu(name):
    _run(name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", [t for t in B.CPP_TESTS if t not in B.CPP_CPU_TESTS])
def test_cpp_mirror(name):
    _run(name)
