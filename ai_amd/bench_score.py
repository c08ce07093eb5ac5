"""Benchmark of the C5 scoring step on device-resident data
(fa_similarities_topk_dev): queries x docs^T similarities and the per-query
top-10, ties to the lower index (cluster.Similarities, cluster/cluster.go:
185-190, with the caller's top-k over (*Tensor).Argmax's first-max rule,
tensor/reduce.go:269-297).

  python -m ai_amd.bench_score                     # 256 queries x 100 000 docs x 768, top-10
  python -m ai_amd.bench_score --nq 32 --nd 1000000

The C5 workload: 256 unit queries against a
seed-generated corpus of 100 000 unit rows (normal, then normalised), both
resident in HBM before timing. One JSON line: mean time per call over
back-to-back calls, the product's fp32 flops (2 * nq * nd * d) per second
and the corpus bytes read per second.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import time

import numpy as np

from . import _native as N
from . import synth as S


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--nq", type=int, default=256)
    ap.add_argument("--nd", type=int, default=100000)
    ap.add_argument("--d", type=int, default=768)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--reps", type=int, default=20)
    a = ap.parse_args()
    ctx = N.Context(0)
    L = N.lib()
    q = S.unit_rows(11, "bench_score_q", a.nq, a.d)
    docs = S.unit_rows(5, "corpus", a.nd, a.d)
    dq, dd, di, dv = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
    for p, n in ((dq, q.nbytes), (dd, docs.nbytes), (di, a.nq * a.k * 4), (dv, a.nq * a.k * 4)):
        N.check(ctx.h, L.fa_device_alloc(ctx.h, n, C.byref(p)))
    N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, dq, q.ctypes.data, q.nbytes))
    N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, dd, docs.ctypes.data, docs.nbytes))

    def call():
        N.check(ctx.h, L.fa_similarities_topk_dev(ctx.h, dq, a.nq, dd, a.nd, a.d, a.k, di, dv))

    for _ in range(3):
        call()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(a.reps):
        call()
    ctx.sync()
    dt = (time.perf_counter() - t0) / a.reps
    flops = 2.0 * a.nq * a.nd * a.d
    print(json.dumps({"op": "similarities_topk", "nq": a.nq, "nd": a.nd, "d": a.d, "k": a.k,
                      "us": round(dt * 1e6, 1), "tflops_fp32": round(flops / dt / 1e12, 1),
                      "corpus_GBps": round(docs.nbytes / dt / 1e9, 1)}), flush=True)
    for p in (dq, dd, di, dv):
        L.fa_device_free(ctx.h, p)
    ctx.close()


if __name__ == "__main__":
    main()
