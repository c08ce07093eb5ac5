"""Benchmark of the tensor.AttentionScaled drop-in on device-resident data
(fa_attention_dev): softmax(scale * q.k^T + mask) . v per (batch, head)
(tensor/attention.go:67-83).

  python -m ai_amd.bench_attention                          # the reference's [8 x 8 x 512 x 64]
  python -m ai_amd.bench_attention --shape 32,3,256,256 --kv-heads 1 --mask pad
  FA_ATTN_DENSE=0 python -m ai_amd.bench_attention          # the per-row kernel, for comparison

The default shape is the one the reference publishes an attention figure
for (BENCHMARKS.md:73: B=8, H=8, T=S=512, D=64, 763 GFLOPS on a Xeon Gold
6130). q, k, v (and the mask) are resident in HBM before timing. One JSON
line: mean time per call over back-to-back calls and the algorithmic flops
per second, 4 * B * H * T * S * D (the two products; the reference's count).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import time

import numpy as np

from . import _native as N
from . import tensor as T


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", default="8,8,512,64", help="B,H,T,D (S = T)")
    ap.add_argument("--kv-heads", type=int, default=0, help="key/value heads (GQA as head stride 0); 0 = H")
    ap.add_argument("--mask", choices=["none", "pad", "window"], default="none")
    ap.add_argument("--reps", type=int, default=20)
    a = ap.parse_args()
    B, H, Tq, D = (int(x) for x in a.shape.split(","))
    S = Tq
    hkv = a.kv_heads or H
    r = np.random.default_rng(3)
    q = r.standard_normal((B, H, Tq, D)).astype(np.float32)
    k = r.standard_normal((B, hkv, S, D)).astype(np.float32)
    v = r.standard_normal((B, hkv, S, D)).astype(np.float32)
    mask, ms = None, (0, 0, 0, 0)
    if a.mask == "pad":  # [B, 1, 1, S]: lengths S, S/2, S, S/2, ...
        mask = T.PaddingMask([S if b % 2 == 0 else S // 2 for b in range(B)], S)
        ms = (S, 0, 0, 1)
    elif a.mask == "window":  # [T, S] broadcast over batch and head
        mask = T.WindowMask(Tq, 257)
        ms = (0, 0, S, 1)
    ctx = N.Context(0)
    L = N.lib()
    bufs = {}
    for name, arr in (("q", q), ("k", k), ("v", v), ("out", q), ("mask", mask)):
        if arr is None:
            continue
        p = C.c_void_p()
        N.check(ctx.h, L.fa_device_alloc(ctx.h, arr.nbytes, C.byref(p)))
        if name != "out":
            N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, p, arr.ctypes.data, arr.nbytes))
        bufs[name] = p
    st = Tq * D
    kv_sh = 0 if hkv == 1 else st  # head stride 0: the reference's Expand for GQA
    scale = 1.0 / np.sqrt(D)

    def call():
        N.check(ctx.h, L.fa_attention_dev(ctx.h, bufs["q"], bufs["k"], bufs["v"], B, H, Tq, S, D, H * st, st,
                                          hkv * st, kv_sh, hkv * st, kv_sh, bufs.get("mask"), *ms, scale,
                                          bufs["out"]))

    for _ in range(3):
        call()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(a.reps):
        call()
    ctx.sync()
    dt = (time.perf_counter() - t0) / a.reps
    flops = 4.0 * B * H * Tq * S * D
    kernel = "generic" if os.environ.get("FA_ATTN_DENSE", "1").startswith("0") or D not in (64, 128, 256, 512) \
        else "dense_mfma"
    print(json.dumps({"op": "attention", "shape": [B, H, Tq, S, D], "kv_heads": hkv, "mask": a.mask,
                      "kernel": kernel, "us": round(dt * 1e6, 1), "gflops": round(flops / dt / 1e9, 1),
                      "frac_fp32_mfma": round(flops / dt / 157.3e12, 3)}), flush=True)
    for p in bufs.values():
        L.fa_device_free(ctx.h, p)
    ctx.close()


if __name__ == "__main__":
    main()
