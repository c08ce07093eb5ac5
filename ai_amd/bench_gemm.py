"""GEMM micro-benchmark of fa_matmul_fused_dev (bf16 [n x k] weights).

  python -m ai_amd.bench_gemm                 # the encoder's product shapes
  python -m ai_amd.bench_gemm --shape 32768,768,768 --reps 5 --no-check
  python -m ai_amd.bench_gemm --shape 128,2304,768 --shape 1,768,3072

One JSON line per shape: mean launch time over back-to-back calls, fp32-
equivalent TFLOP/s (2*M*N*K / time) and the max |error| against a float64
product of the same inputs (all rows for M <= 8192, 256 sampled rows above).
The environment selects the kernel: FA_GEMM_XTILE=<tile> forces a split-bf16
tile shape, FA_GEMM_MFMA=f32 runs the fp32-MFMA kernel instead.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import time

import numpy as np

from . import _native as N
from . import synth as S

SHAPES = [(5517, 1280, 768), (5517, 768, 768), (5517, 2304, 768), (5517, 768, 1152),
          (32768, 1280, 768), (32768, 768, 768), (32768, 2304, 768), (32768, 768, 1152)]


def run(shapes, reps: int, check: bool) -> list[dict]:
    ctx = N.Context(0)
    L = N.lib()
    kernel = os.environ.get("FA_GEMM_XTILE", "auto")
    if os.environ.get("FA_GEMM_MFMA") == "f32":
        kernel = "f32-mfma"
    out = []
    for (M, Nn, K) in shapes:
        rng = np.random.default_rng(M + Nn + K)
        a = rng.standard_normal((M, K)).astype(np.float32)
        wb = S.normal_bf16(3, "bench_gemm", 0.05, (Nn, K))
        da, db, dc = C.c_void_p(), C.c_void_p(), C.c_void_p()
        for p, n in ((da, a.nbytes), (db, wb.nbytes), (dc, M * Nn * 4)):
            N.check(ctx.h, L.fa_device_alloc(ctx.h, n, C.byref(p)))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, da, a.ctypes.data, a.nbytes))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, db, wb.ctypes.data, wb.nbytes))

        def call():
            N.check(ctx.h, L.fa_matmul_fused_dev(ctx.h, M, Nn, K, da, K, db, K, N.FA_DT_BF16, N.FA_B_NK, None, dc, Nn))

        call()
        ctx.sync()
        rec = dict(kernel=kernel, M=M, N=Nn, K=K)
        if check:
            c = np.empty((M, Nn), np.float32)
            N.check(ctx.h, L.fa_memcpy_d2h(ctx.h, c.ctypes.data, dc, c.nbytes))
            rows = np.arange(M) if M <= 8192 else rng.choice(M, 256, replace=False)
            want = a[rows].astype(np.float64) @ S.bf16_to_f32(wb).T.astype(np.float64)
            rec["max_abs_err_vs_f64"] = float(np.abs(c[rows] - want).max())
        for _ in range(3):
            call()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            call()
        ctx.sync()
        dt = (time.perf_counter() - t0) / reps
        rec["us"] = round(dt * 1e6, 1)
        rec["tflops_fp32_equiv"] = round(2 * M * Nn * K / dt / 1e12, 1)
        out.append(rec)
        print(json.dumps(rec), flush=True)
        for p in (da, db, dc):
            L.fa_device_free(ctx.h, p)
    ctx.close()
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--shape", action="append",
                    help="M,N,K, repeatable (default: the encoder's product shapes at C2 and M=32768)")
    ap.add_argument("--reps", type=int, default=30)
    ap.add_argument("--no-check", action="store_true", help="skip the float64 comparison")
    a = ap.parse_args()
    shapes = [tuple(int(v) for v in sh.split(",")) for sh in a.shape] if a.shape else SHAPES
    run(shapes, a.reps, not a.no_check)


if __name__ == "__main__":
    main()
