"""A program that never closes its context and model exits cleanly.

Regression test: a script that left a context and an encoder model open
aborted at exit ("terminate called ... std::bad_variant_access") in the HIP
runtime's own teardown, which runs after Python's. The binding now closes
what is still open at interpreter exit, models before contexts. Runs the
program in a child process (one GPU process besides the test runner).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = """
import numpy as np
from ai_amd import _native as N, gemma as G, synth as S
ctx = N.Context(0)
model = G.Model(S.ModelShape(num_hidden_layers=2, vocab_size=4096), ctx)
model.load_synthetic()
ids = np.full((2, 40), 7, np.int32); ids[:, 0] = 2
emb = model.embed_ids(ids, np.array([40, 25], np.int32))
print("embedded", emb.shape, flush=True)
"""


def test_exit_with_handles_open():
    r = subprocess.run([sys.executable, "-c", PROGRAM], cwd=ROOT, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=100)
    print(r.stdout, flush=True)
    assert "embedded (2, 768)" in r.stdout
    assert "terminate called" not in r.stdout
    assert r.returncode == 0, r.returncode


def test_c_program_exits_with_model_and_context_open():
    """The library's own exit handler (registered at fa_create) closes the
    model and context a C caller left open, before the HIP runtime's teardown
    (tests/cpp/exit_open.c)."""
    from ai_amd import build as B
    binary = os.path.join(B.CPP_TEST_BIN, "exit_open")
    assert os.path.exists(binary), "run __graft_entry__.build() first"
    print(f"running {binary}", flush=True)
    r = subprocess.run([binary], cwd=ROOT, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=100)
    print(r.stdout, flush=True)
    assert "embedded 2 x 768" in r.stdout
    assert "terminate called" not in r.stdout
    assert r.returncode == 0, r.returncode
