"""CPU checks of the drop-in boundary: the C-ABI libraries load and export
every function their headers declare, the product never reaches the oracle,
and the host-side argument checks reject what the reference rejects (no
compute call is made: there is no GPU here)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from ai_amd import _native as N
from ai_amd import synth as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def test_rocm_library_exports_header():
    names = N.header_functions(N.HEADER)
    assert len(names) >= 25
    syms = exported(N.lib_path())
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    N.lib()  # loads and binds every signature


def test_synth_library_exports_header():
    names = N.header_functions(N.SYNTH_HEADER)
    syms = exported(os.path.join(N.LIB_DIR, "libfa_synth.so"))
    assert not [n for n in names if n not in syms]
    N.synth()


def test_product_never_reaches_the_oracle():
    syms = exported(N.lib_path())
    assert not [s for s in syms if s.startswith("orc_")]
    deps = subprocess.run(["ldd", N.lib_path()], capture_output=True, text=True).stdout
    assert "oracle" not in deps
    for dirpath, _, files in os.walk(os.path.join(ROOT, "ai_amd")):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle_lib" not in text and "fa_oracle" not in text, f


def test_version_and_null_context_errors():
    assert N.lib().fa_version().startswith(b"fa_rocm")
    rc = N.lib().fa_create(0, None)
    assert rc == N.FA_ERR_ARG
    assert b"NULL" in N.lib().fa_last_error(None)
    assert N.lib().fa_sync(None) == N.FA_ERR_ARG
    assert N.lib().fa_matmul_fused(None, 1, 1, 1, None, 1, None, 1, 0, 0, None, None, 1) == N.FA_ERR_ARG


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(N, "LIB_DIR", str(tmp_path))
    monkeypatch.setattr(N, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        N.lib()


# ---- synthetic inputs -------------------------------------------------------------

def test_synth_deterministic_and_thread_independent():
    a = S.normal_bf16(1, "w", 0.02, (3, 1 << 20))  # several generator chunks
    b = S.normal_bf16(1, "w", 0.02, (3, 1 << 20))
    assert np.array_equal(a, b)
    env = dict(os.environ, OMP_NUM_THREADS="1")
    code = ("import sys; sys.path.insert(0, %r); from ai_amd import synth as S; import numpy as np; "
            "a = S.normal_bf16(1, 'w', 0.02, (3, 1 << 20)); print(int(a.astype(np.int64).sum()))" % ROOT)
    one = subprocess.run(["python", "-c", code], env=env, capture_output=True, text=True, check=True).stdout
    assert int(one) == int(a.astype(np.int64).sum())
    assert not np.array_equal(a, S.normal_bf16(1, "v", 0.02, (3, 1 << 20)))


def test_synth_normal_statistics_and_bf16_rounding():
    f = S.normal_f32(9, "n", 0.02, (1 << 20,))
    assert abs(f.mean()) < 1e-4 and abs(f.std() - 0.02) < 1e-4
    b = S.normal_bf16(9, "n", 0.02, (1 << 20,))
    w = S.bf16_to_f32(b)
    # bf16 of the same stream, round-to-nearest-even
    assert np.array_equal(S.f32_to_bf16(f), b)
    assert np.all(np.abs(w - f) <= np.abs(f) * 2.0 ** -8)
    assert np.array_equal(w.view(np.uint32) & 0xFFFF, np.zeros_like(w, np.uint32))


def test_bf16_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, 1.0078125, -2.5, 3.4e38, np.inf], np.float32)
    got = S.f32_to_bf16(x)
    # 1.00390625 = 1 + 2^-8 is a tie -> even (1.0); 1.01171875 = 1 + 3*2^-8 tie -> 1.015625
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x7F80, 0x7F80], np.uint16)
    assert got.tolist() == want.tolist()


def test_batches_follow_the_configs():
    b1 = S.make_batch("C1")
    assert b1.ids.shape == (1, 128) and b1.ids[0, 0] == 2 and b1.ids[0, 1:].min() >= 3
    b2 = S.make_batch("C2")
    assert b2.ids.shape == (32, 256)
    assert b2.lengths.min() >= 64 and b2.lengths.max() <= 256
    for b in range(32):
        L = b2.lengths[b]
        assert b2.ids[b, 0] == 2 and np.all(b2.ids[b, 1:L] >= 3) and np.all(b2.ids[b, L:] == 0)
    b3 = S.make_batch("C3")
    assert b3.ids.shape == (64, 512) and np.all(b3.lengths == 512)
    b4 = S.make_batch("C4")
    assert b4.ids.shape == (8, 2048) and b4.lengths.min() >= 1024
    b5 = S.make_batch("C5", with_corpus=False)
    assert b5.ids.shape == (256, 128) and b5.lengths.min() >= 16 and b5.lengths.max() <= 128
    # Zipf(1.1): id 3 (rank 1) is the most frequent token
    ids = b2.ids[b2.ids >= 3]
    vals, counts = np.unique(ids, return_counts=True)
    assert vals[counts.argmax()] == 3
    assert np.array_equal(S.make_batch("C2").ids, b2.ids)


def test_zipf_law_shape():
    z = S.zipf_i32(3, "z", 1.1, 1000, 0, 200000)
    c = np.bincount(z, minlength=1001)[1:]
    p = np.arange(1, 1001, dtype=np.float64) ** -1.1
    p /= p.sum()
    assert abs(c[0] / 200000 - p[0]) < 0.01 and abs(c[9] / 200000 - p[9]) < 0.005


def test_unit_rows():
    u = S.unit_rows(5, "c", 100, 768)
    assert np.allclose(np.linalg.norm(u.astype(np.float64), axis=1), 1, atol=1e-6)


def test_weight_specs_complete():
    specs = S.weight_specs(S.ModelShape())
    names = [s[0] for s in specs]
    assert len(names) == len(set(names)) == 2 + 2 + 13 * 24
    assert sum(int(np.prod(s[1])) for s in specs) == 307_581_696


# ---- tensor.MatMul's views in the Python mirror (host logic only) -------------

def test_matmul_view_strides_and_broadcast():
    """The fa_matrix the mirror builds for numpy views: element strides of
    the matrix dimensions and broadcastStrides over the batch
    (tensor/shape.go:94-131); no device call."""
    from ai_amd import tensor as T
    a = np.zeros((3, 1, 4, 5), np.float32)
    b = np.zeros((2, 6, 5), np.float32).swapaxes(1, 2)  # [2, 5, 6], rows of stride 1
    batch = T._broadcast_shapes(a.shape[:-2], b.shape[:-2])
    assert batch == (3, 2)
    ma, mb = T._matrix(a, batch), T._matrix(b, batch)
    assert (ma.rs, ma.cs, list(ma.bstride[:2])) == (5, 1, [20, 0])  # a's size-1 dim broadcasts: stride 0
    assert (mb.rs, mb.cs, list(mb.bstride[:2])) == (1, 5, [0, 30])  # b has no first batch dim
    c = np.broadcast_to(np.zeros((1, 8), np.float32), (7, 8))
    mc = T._matrix(c, ())
    assert (mc.rs, mc.cs) == (0, 1)
    with pytest.raises(T.TensorError, match="not broadcastable"):
        T._broadcast_shapes((2, 3), (3, 3))
    # negative or odd byte strides are copied, float64 converted
    assert T._view(np.zeros((4, 4), np.float32)[::-1]).strides == (16, 4)
    assert T._view(np.zeros((4, 4))).dtype == np.float32


def test_matmul_strided_rejects_without_context():
    assert N.lib().fa_matmul_strided(None, 0, None, 1, 1, 1, None, None, None, None) == N.FA_ERR_ARG
    assert N.lib().fa_matmul_strided_dev(None, 0, None, 1, 1, 1, None, None, None, None) == N.FA_ERR_ARG
