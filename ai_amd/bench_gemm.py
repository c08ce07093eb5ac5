"""GEMM micro-benchmark of fa_matmul_fused_dev (bf16 [n x k] weights).

  python -m ai_amd.bench_gemm                 # the encoder's product shapes
  python -m ai_amd.bench_gemm --shape 32768,768,768 --reps 5 --no-check
  python -m ai_amd.bench_gemm --shape 128,2304,768 --shape 1,768,3072
  python -m ai_amd.bench_gemm --library       # against the vendor bf16 GEMM
  python -m ai_amd.bench_gemm --a-data zeros  # same work on data that draws less power

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


def make_a(rng, M: int, K: int, kind: str) -> np.ndarray:
    """The A operand: normal fp32 values (every split term busy), zeros, or
    bf16-exact values (the mid and lo terms zero). Same MFMA work in every
    case; the time differs only through the power the data draws."""
    if kind == "zeros":
        return np.zeros((M, K), np.float32)
    a = rng.standard_normal((M, K)).astype(np.float32)
    if kind == "bf16":
        a = (a.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    return a


def run(shapes, reps: int, check: bool, a_data: str = "normal") -> list[dict]:
    ctx = N.Context(0)
    L = N.lib()
    kernel = os.environ.get("FA_GEMM_XTILE", "auto")
    if os.environ.get("FA_GEMM_MFMA") == "f32":
        kernel = "f32-mfma"
    out = []
    for (M, Nn, K) in shapes:
        rng = np.random.default_rng(M + Nn + K)
        a = make_a(rng, M, K, a_data)
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
        rec = dict(kernel=kernel, M=M, N=Nn, K=K, a_data=a_data)
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


def dropin(reps: int) -> None:
    """tensor.MatMulFused as the Go drop-in calls it for the GeGLU gate
    (models/gemma/embed.go:227): x [5517 x 768] . W [768 x 1152] with RowScale,
    GELU and Mul, W float32 in the reference's [k x n] layout (and bf16, and
    [n x k]). Host entry point (fa_matmul_fused: copies in and out included,
    as the cgo shim calls it) and device-pointer entry point
    (fa_matmul_fused_dev, operands resident); for float32 weights also the
    strided entry point the Go binding uses (fa_matmul_strided_dev)."""
    ctx = N.Context(0)
    L = N.lib()
    m, k, n = 5517, 768, 1152
    rng = np.random.default_rng(1)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w32 = S.normal_f32(5, "dropin", 0.02, (k, n))
    rs = rng.uniform(0.5, 1.5, m).astype(np.float32)
    mul = rng.standard_normal((m, n)).astype(np.float32)
    c = np.empty((m, n), np.float32)
    for wname, dt, layout, w in (("f32", N.FA_DT_F32, N.FA_B_KN, w32),
                                 ("f32", N.FA_DT_F32, N.FA_B_NK, np.ascontiguousarray(w32.T)),
                                 ("bf16", N.FA_DT_BF16, N.FA_B_KN, S.f32_to_bf16(w32)),
                                 ("bf16", N.FA_DT_BF16, N.FA_B_NK, np.ascontiguousarray(S.f32_to_bf16(w32).T))):
        ldb = w.shape[1]
        e = N.Epilogue()
        e.act = N.FA_ACT_GELU
        e.row_scale = rs.ctypes.data
        e.mul = mul.ctypes.data
        e.ldm = n

        def host():
            N.check(ctx.h, L.fa_matmul_fused(ctx.h, m, n, k, a.ctypes.data, k, w.ctypes.data, ldb, dt, layout,
                                             C.byref(e), c.ctypes.data, n))
        ptrs = {}
        for key, arr in (("a", a), ("w", w), ("rs", rs), ("mul", mul), ("c", c)):
            p = C.c_void_p()
            N.check(ctx.h, L.fa_device_alloc(ctx.h, arr.nbytes, C.byref(p)))
            N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, p, arr.ctypes.data, arr.nbytes))
            ptrs[key] = p
        ed = N.Epilogue()
        ed.act = N.FA_ACT_GELU
        ed.row_scale = ptrs["rs"].value
        ed.mul = ptrs["mul"].value
        ed.ldm = n

        def dev():
            N.check(ctx.h, L.fa_matmul_fused_dev(ctx.h, m, n, k, ptrs["a"], k, ptrs["w"], ldb, dt, layout,
                                                 C.byref(ed), ptrs["c"], n))
        out = dict(op="MatMulFused gate", M=m, K=k, N=n, w=wname, layout="KN" if layout == N.FA_B_KN else "NK")
        for label, fn in (("host_us", host), ("dev_us", dev)):
            for _ in range(3):
                fn()
            ctx.sync()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            ctx.sync()
            out[label] = round((time.perf_counter() - t0) / reps * 1e6, 1)
        out["dev_tflops_fp32_equiv"] = round(2 * m * n * k / (out["dev_us"] * 1e-6) / 1e12, 1)
        if dt == N.FA_DT_F32:
            # the Go binding's route since it takes strided views
            # (fa_matmul_strided_dev): W as a [k x n] array, or the [n x k]
            # array read as its transposed view (row stride 1)
            av, wv = N.Matrix(), N.Matrix()
            av.data, av.rs, av.cs = ptrs["a"].value, k, 1
            wv.data = ptrs["w"].value
            wv.rs, wv.cs = (n, 1) if layout == N.FA_B_KN else (1, k)

            def strided():
                N.check(ctx.h, L.fa_matmul_strided_dev(ctx.h, 0, None, m, n, k, C.byref(av), C.byref(wv),
                                                       C.byref(ed), ptrs["c"]))
            for _ in range(3):
                strided()
            ctx.sync()
            t0 = time.perf_counter()
            for _ in range(reps):
                strided()
            ctx.sync()
            out["strided_dev_us"] = round((time.perf_counter() - t0) / reps * 1e6, 1)
        print(json.dumps(out), flush=True)
        for p in ptrs.values():
            L.fa_device_free(ctx.h, p)
    ctx.close()


def library(shapes, reps: int) -> None:
    """The split product against the vendor bf16 GEMM on the same MFMA work.

    The split-bf16 product A.W (A fp32 = hi + mid + lo, W bf16) is the plain
    bf16 GEMM [A_hi | A_mid | A_lo] (M x 3K) . [W | W | W]^T with fp32
    accumulation. For each shape this times fa_matmul_fused_dev (split
    included, fp32 output) and torch.mm on bf16 operands of that (M, N, 3K)
    shape (hipBLASLt on ROCm; the planes are random here, only the time
    matters): B as the transposed view of an [N x 3K] array (the weights'
    [out, in] layout our kernel reads) with float32 and with bfloat16 output,
    and B as a [3K x N] array with float32 output. Host clock around `reps`
    back-to-back calls each, after a synchronisation."""
    import torch
    ctx = N.Context(0)
    L = N.lib()
    dev = torch.device("cuda")
    for (M, Nn, K) in shapes:
        rng = np.random.default_rng(M + Nn + K)
        a = rng.standard_normal((M, K)).astype(np.float32)
        wb = S.normal_bf16(3, "bench_gemm", 0.05, (Nn, K))
        da, db, dc = C.c_void_p(), C.c_void_p(), C.c_void_p()
        for p, n in ((da, a.nbytes), (db, wb.nbytes), (dc, M * Nn * 4)):
            N.check(ctx.h, L.fa_device_alloc(ctx.h, n, C.byref(p)))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, da, a.ctypes.data, a.nbytes))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, db, wb.ctypes.data, wb.nbytes))

        def ours():
            N.check(ctx.h, L.fa_matmul_fused_dev(ctx.h, M, Nn, K, da, K, db, K, N.FA_DT_BF16, N.FA_B_NK, None, dc, Nn))

        a3 = torch.randn(M, 3 * K, device=dev, dtype=torch.bfloat16)
        w3_nk = torch.randn(Nn, 3 * K, device=dev, dtype=torch.bfloat16)
        w3_kn = torch.randn(3 * K, Nn, device=dev, dtype=torch.bfloat16)
        rec = dict(M=M, N=Nn, K=K, vendor_K=3 * K)
        runs = [("split_kernel_us", ours, ctx.sync),
                ("vendor_nt_f32out_us", lambda: torch.mm(a3, w3_nk.t(), out_dtype=torch.float32), torch.cuda.synchronize),
                ("vendor_nt_bf16out_us", lambda: torch.mm(a3, w3_nk.t()), torch.cuda.synchronize),
                ("vendor_nn_f32out_us", lambda: torch.mm(a3, w3_kn, out_dtype=torch.float32), torch.cuda.synchronize)]
        for label, fn, sync in runs:
            for _ in range(3):
                fn()
            sync()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            sync()
            rec[label] = round((time.perf_counter() - t0) / reps * 1e6, 1)
        # the faster vendor layout with the same (fp32) output as ours
        rec["vendor_bf16_us"] = min(rec["vendor_nt_f32out_us"], rec["vendor_nn_f32out_us"])
        rec["bf16_tflops_split_kernel"] = round(2 * M * Nn * 3 * K / (rec["split_kernel_us"] * 1e-6) / 1e12, 1)
        rec["bf16_tflops_vendor"] = round(2 * M * Nn * 3 * K / (rec["vendor_bf16_us"] * 1e-6) / 1e12, 1)
        print(json.dumps(rec), flush=True)
        for p in (da, db, dc):
            L.fa_device_free(ctx.h, p)
    ctx.close()


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--shape", action="append",
                    help="M,N,K, repeatable (default: the encoder's product shapes at C2 and M=32768)")
    ap.add_argument("--reps", type=int, default=30)
    ap.add_argument("--no-check", action="store_true", help="skip the float64 comparison")
    ap.add_argument("--dropin", action="store_true",
                    help="time the MatMulFused drop-in at the gate shape with float32/bf16 weights in both layouts")
    ap.add_argument("--library", action="store_true",
                    help="time each shape against the vendor bf16 GEMM of the same MFMA work (M x 3K . 3K x N)")
    ap.add_argument("--a-data", default="normal", choices=["normal", "zeros", "bf16"],
                    help="values of A: normal fp32 (default), zeros, or bf16-exact (mid and lo split terms zero)")
    a = ap.parse_args()
    if a.dropin:
        dropin(a.reps)
        return
    shapes = [tuple(int(v) for v in sh.split(",")) for sh in a.shape] if a.shape else SHAPES
    if a.library:
        library(shapes, a.reps)
        return
    run(shapes, a.reps, not a.no_check, a.a_data)


if __name__ == "__main__":
    main()
