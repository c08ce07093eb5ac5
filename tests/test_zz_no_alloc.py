"""fa_similarities_topk_dev_noalloc (fixed per-device scratch, no allocation)
against fa_similarities_topk_dev, through the C ABI: two calls in a row, the
second with fewer queries and docs, must give identical indices and values
(the same kernels on the same inputs), and both equal the exact dot products
rounded to float32 in (value desc, index asc) order; sizes beyond the fixed
scratch are refused."""
import ctypes as C

import numpy as np
import pytest

from ai_amd import _native as N

pytestmark = pytest.mark.gpu


def unit(a):
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float32)


def dev(ctx, a):
    p = C.c_void_p()
    N.check(ctx.h, N.lib().fa_device_alloc(ctx.h, max(a.nbytes, 4), C.byref(p)))
    N.check(ctx.h, N.lib().fa_memcpy_h2d(ctx.h, p, a.ctypes.data, a.nbytes))
    return p


def run(ctx, fn, dq, nq, dd, nd, d, k):
    L = N.lib()
    di, dv = C.c_void_p(), C.c_void_p()
    N.check(ctx.h, L.fa_device_alloc(ctx.h, nq * k * 4, C.byref(di)))
    N.check(ctx.h, L.fa_device_alloc(ctx.h, nq * k * 4, C.byref(dv)))
    N.check(ctx.h, fn(ctx.h, dq, nq, dd, nd, d, k, di, dv))
    ctx.sync()
    idx = np.empty((nq, k), np.int32)
    val = np.empty((nq, k), np.float32)
    N.check(ctx.h, L.fa_memcpy_d2h(ctx.h, idx.ctypes.data, di, idx.nbytes))
    N.check(ctx.h, L.fa_memcpy_d2h(ctx.h, val.ctypes.data, dv, val.nbytes))
    L.fa_device_free(ctx.h, di)
    L.fa_device_free(ctx.h, dv)
    return idx, val


@pytest.fixture(scope="module")
def nctx():
    c = N.Context(0)
    yield c
    c.close()


def test_noalloc_matches_dev_entry_point(nctx):
    L = N.lib()
    r = np.random.default_rng(77)
    q = unit(r.standard_normal((300, 768)))
    docs = unit(r.standard_normal((20000, 768)))
    docs[1000:1040] = docs[7]  # ties that take the exact fallback for the query below
    q[5] = docs[7]
    dq, dd = dev(nctx, q), dev(nctx, docs)
    for nq, nd, k in ((300, 20000, 16), (130, 5000, 10)):
        a_i, a_v = run(nctx, L.fa_similarities_topk_dev_noalloc, dq, nq, dd, nd, 768, k)
        b_i, b_v = run(nctx, L.fa_similarities_topk_dev, dq, nq, dd, nd, 768, k)
        assert np.array_equal(a_i, b_i), (nq, nd, k)
        assert np.array_equal(a_v, b_v), (nq, nd, k)
        # independently of the other entry point: every list is the float64
        # dot products rounded to float32 in (value desc, index asc) order;
        # only exchanges of (nearly) equal scores are allowed
        s64 = q[:nq].astype(np.float64) @ docs[:nd].astype(np.float64).T
        s32 = s64.astype(np.float32)
        for i in range(nq):
            want = np.lexsort((np.arange(nd), -s32[i]))[:k]
            if not np.array_equal(a_i[i], want):
                assert np.allclose(s64[i, a_i[i]], s64[i, want], rtol=0, atol=1e-12), (nq, i, a_i[i], want)
        np.testing.assert_allclose(a_v, np.take_along_axis(s32, a_i.astype(np.int64), axis=1), rtol=0, atol=1e-7)
        print(f"no-alloc == dev entry point == rounded exact order at nq={nq} nd={nd} k={k}", flush=True)
    assert a_i[5].tolist() == [7] + list(range(1000, 1009))
    L.fa_device_free(nctx.h, dq)
    L.fa_device_free(nctx.h, dd)


def test_noalloc_refuses_what_the_scratch_cannot_hold(nctx):
    L = N.lib()
    q = np.zeros((4, 4096), np.float32)
    dq = dev(nctx, q)
    out = C.c_void_p()
    N.check(nctx.h, L.fa_device_alloc(nctx.h, 4 * 4 * 17, C.byref(out)))
    assert L.fa_similarities_topk_dev_noalloc(nctx.h, dq, 4, dq, 4, 4096, 1, out, out) == N.FA_ERR_ARG
    assert b"2048" in L.fa_last_error(nctx.h)
    assert L.fa_similarities_topk_dev_noalloc(nctx.h, dq, 4, dq, 4, 64, 17, out, out) == N.FA_ERR_ARG
    assert L.fa_similarities_topk_dev_noalloc(nctx.h, dq, 4, dq, 4, 48, 1, out, out) == N.FA_ERR_ARG
    L.fa_device_free(nctx.h, dq)
    L.fa_device_free(nctx.h, out)


def test_noalloc_allocates_no_device_memory(nctx):
    """The point of the entry point: calls of several sizes (after one warm-up
    call that loads the kernels) leave the device's free memory unchanged."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L = N.lib()
    r = np.random.default_rng(78)
    q = unit(r.standard_normal((260, 512)))
    docs = unit(r.standard_normal((9000, 512)))
    dq, dd = dev(nctx, q), dev(nctx, docs)
    di, dv = C.c_void_p(), C.c_void_p()
    N.check(nctx.h, L.fa_device_alloc(nctx.h, 260 * 16 * 4, C.byref(di)))
    N.check(nctx.h, L.fa_device_alloc(nctx.h, 260 * 16 * 4, C.byref(dv)))
    N.check(nctx.h, L.fa_similarities_topk_dev_noalloc(nctx.h, dq, 260, dd, 9000, 512, 16, di, dv))
    nctx.sync()
    free0, free1, total = C.c_size_t(), C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free0), C.byref(total)) == 0
    for nq, nd, k in ((260, 9000, 16), (7, 300, 3), (129, 9000, 10), (1, 17, 1)):
        N.check(nctx.h, L.fa_similarities_topk_dev_noalloc(nctx.h, dq, nq, dd, nd, 512, k, di, dv))
    nctx.sync()
    assert hip.hipMemGetInfo(C.byref(free1), C.byref(total)) == 0
    print(f"free device memory before {free0.value} after {free1.value}", flush=True)
    assert free1.value == free0.value
    for p in (dq, dd, di, dv):
        L.fa_device_free(nctx.h, p)


def test_noalloc_array_belongs_to_one_context(nctx):
    """A second context on the same GPU is refused (FA_ERR_STATE) while the
    first owns the array, instead of racing on it; once the owner is
    destroyed the other context may claim it."""
    L = N.lib()
    r = np.random.default_rng(79)
    q = unit(r.standard_normal((8, 256)))
    other = N.Context(0)
    dq = dev(other, q)
    out = C.c_void_p()
    N.check(other.h, L.fa_device_alloc(other.h, 8 * 4 * 2, C.byref(out)))
    N.check(nctx.h, L.fa_similarities_topk_dev_noalloc(nctx.h, dq, 8, dq, 8, 256, 1, out, out))  # nctx owns it
    nctx.sync()
    assert L.fa_similarities_topk_dev_noalloc(other.h, dq, 8, dq, 8, 256, 1, out, out) == N.FA_ERR_STATE
    assert b"another context" in L.fa_last_error(other.h)
    third = N.Context(0)
    third.close()  # destroying a context that never claimed the array leaves nctx's claim
    assert L.fa_similarities_topk_dev_noalloc(other.h, dq, 8, dq, 8, 256, 1, out, out) == N.FA_ERR_STATE
    nctx.close()  # the owner goes: the array is free again
    N.check(other.h, L.fa_similarities_topk_dev_noalloc(other.h, dq, 8, dq, 8, 256, 1, out, None))  # indices only
    other.sync()
    idx = np.empty(8, np.int32)
    N.check(other.h, L.fa_memcpy_d2h(other.h, idx.ctypes.data, out, 32))
    assert idx.tolist() == list(range(8))  # each unit row is its own best match
    L.fa_device_free(other.h, dq)
    L.fa_device_free(other.h, out)
    other.close()
