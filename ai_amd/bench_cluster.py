"""Benchmark of the cluster path on device-resident rows (fa_cluster_*_dev).

  python -m ai_amd.bench_cluster                      # 50 000 x 768, k = 40
  python -m ai_amd.bench_cluster --n 200000 --k 256

The workload is the reference's TestNearestSpeed size (cluster_test.go:67-84:
50 000 unit rows of 768 against 40 centres) and KMeans on planted data of the
same size. Rows are generated here (normal, normalised on the device) and
stay in HBM; one JSON line per operation: mean time per call over back-to-back
calls and the algorithmic bytes / flops of the rows pass.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import time

import numpy as np

from . import _native as N


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=50000)
    ap.add_argument("--d", type=int, default=768)
    ap.add_argument("--k", type=int, default=40)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--reps", type=int, default=20)
    a = ap.parse_args()
    n, d, k = a.n, a.d, a.k
    ctx = N.Context(0)
    L = N.lib()
    rng = np.random.default_rng(1)
    # planted rows: k well-separated unit directions plus noise, as the
    # reference's planted() (cluster_test.go:12-26) at k groups
    cd = rng.standard_normal((k, d)).astype(np.float32)
    cd /= np.linalg.norm(cd, axis=1, keepdims=True)
    x = (cd[np.arange(n) % k] + rng.standard_normal((n, d)).astype(np.float32) * (2.4 / np.sqrt(d))).astype(np.float32)
    bufs = {}
    for name, nbytes in (("x", x.nbytes), ("c", k * d * 4), ("idx", n * 4), ("sim", n * 4), ("cent", k * d * 4),
                         ("asg", n * 4), ("sz", k * 4)):
        p = C.c_void_p()
        N.check(ctx.h, L.fa_device_alloc(ctx.h, nbytes, C.byref(p)))
        bufs[name] = p
    N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, bufs["x"], x.ctypes.data, x.nbytes))
    N.check(ctx.h, L.fa_cluster_normalize_dev(ctx.h, bufs["x"], n, d, bufs["x"]))
    c0 = rng.standard_normal((k, d)).astype(np.float32)
    N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, bufs["c"], c0.ctypes.data, c0.nbytes))
    N.check(ctx.h, L.fa_cluster_normalize_dev(ctx.h, bufs["c"], k, d, bufs["c"]))

    def nearest():
        N.check(ctx.h, L.fa_cluster_nearest_dev(ctx.h, bufs["x"], n, bufs["c"], k, d, bufs["idx"], bufs["sim"]))

    it = C.c_int32(0)

    def kmeans():
        N.check(ctx.h, L.fa_cluster_kmeans_dev(ctx.h, bufs["x"], n, d, k, a.iters, C.c_uint64(7), bufs["cent"],
                                               bufs["asg"], bufs["sim"], bufs["sz"], C.byref(it)))

    for name, fn, reps in (("Nearest", nearest, a.reps), ("KMeans", kmeans, max(3, a.reps // 4))):
        fn()
        ctx.sync()
        t = time.perf_counter()
        for _ in range(reps):
            fn()
        ctx.sync()
        us = (time.perf_counter() - t) / reps * 1e6
        rec = {"op": name, "n": n, "d": d, "k": k, "us_per_call": round(us, 1)}
        if name == "Nearest":
            rec["rows_GBps"] = round(n * d * 4 / (us * 1e-6) / 1e9, 1)
            rec["tflops"] = round(2.0 * n * k * d / (us * 1e-6) / 1e12, 2)
        else:
            rec["iterations"] = it.value
            rec["rounds"] = it.value + k - 1  # k-1 seeding passes + Lloyd rounds over the rows
        print(json.dumps(rec), flush=True)
    for p in bufs.values():
        L.fa_device_free(ctx.h, p)
    ctx.close()


if __name__ == "__main__":
    main()
