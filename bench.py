#!/usr/bin/env python3
"""Throughput of the EmbeddingGemma encoder forward on one MI355X.

One step = one forward pass (token ids -> 768-d L2-normalised embeddings) of
the BASELINE.json workload named by --config (default C2: batch 32 x seq 256,
lengths uniform in [64, 256], Zipf ids), with random-init bf16-resident
weights of the EmbeddingGemma-300M architecture.

Prints ONE JSON line (the driver's contract) with:
  value            sentences/s over the timed steps (whole job, 1 GPU), each
                   step timed as the metric defines t_batch: token ids on the
                   host -> embeddings on the host (fa_gemma_embed_ids: the ids'
                   host-to-device copy, the forward, the embeddings'
                   device-to-host copy and a stream synchronisation per step),
                   as the reference's benchEmbed times Embed host to host
                   (cmd/bench/main.go:350-354)
  device_resident  the same forward with ids already in HBM and the
                   embeddings left there, steps enqueued back to back
                   (fa_gemma_embed_ids_dev): the device-side throughput
  roofline         the dominant kernel (the gate|up GEMM with the GeGLU
                   epilogue) timed with HIP events on the library's stream:
                   algorithmic flops (2*M*N*K) / mean launch duration vs the
                   2.5 PFLOP/s dense bf16 MFMA peak, the unit the split-bf16
                   GEMM runs on (three bf16 products per fp32 multiply-add,
                   so its ceiling is a third of that peak)
  throughput_roofline
                   the timed throughput as a roofline fraction: the forward's
                   algorithmic flops (all GEMMs + attention) per timed step /
                   the timed step, against the bf16 and fp32 MFMA peaks
  cpu_baseline     the CPU oracle (a port of the reference's Go path, the Go
                   toolchain being absent) on a bounded sample of the same
                   workload, on this host's cores
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK = 157.3e12  # MI355X dense fp32 matrix, FLOP/s
BF16_MFMA_PEAK = 2.5e15    # MI355X dense bf16 matrix, FLOP/s
SPLIT_TERMS = 3            # bf16 products per fp32 multiply-add in the split-bf16 GEMM
HBM_PEAK = 8.0e12          # MI355X HBM3E, B/s

METRIC = "sentences/sec @ batch32×seq256 on 1 MI355X; GEMM % of fp32 MFMA peak"

# HBM bytes per launch of the gate|up GEMM at C2, from rocprofv3 FETCH_SIZE
# (KiB, x2.000) + WRITE_SIZE (KiB, x1.000) runs, the factors being what a
# 1 GiB copy kernel reads on the same counters (profiles/
# gemm_gateup_c2_hbm_traffic.md). Re-measured whenever the kernel changes;
# applies to the C2 workload only.
GATEUP_TRAFFIC_C2 = {"bytes": (2 * 30326 + 29578) * 1024, "kernel_rev": "x3-128x256w8-chunkmajor-lds"}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # 50 steps: about 0.26 s of timed work per region at C2, so that one
    # hiccup of the host moves the headline little
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"])
    p.add_argument("--model", default="eg300m", choices=["eg300m", "eg2"],
                   help="eg300m: EmbeddingGemma-300M (the headline); eg2: the EmbeddingGemma 2 text tower at the "
                        "reference's widths (hidden 512, 12 layers, head_dim 256/512, per-layer inputs 512)")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 1 GiB device copy (torch) 3 times: the reference kernel for scaling "
                        "rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    return p.parse_args()


def calibrate_copy() -> None:
    import torch
    n = 1 << 28  # floats: 1 GiB
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": 3}))


def host_cpu() -> dict:
    """This host's CPU model, the logical CPUs this process may run on and the
    physical cores among them (hyperthreads counted once, as the reference's
    topology_linux.go:12-28 counts them)."""
    model, cores = "unknown", set()
    allowed = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    try:
        cpu, phys = None, None
        info = {}
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                cpu = int(v)
            elif k == "model name":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id" and cpu is not None:
                info[cpu] = (phys, v)
        cores = {info[c] for c in allowed if c in info}
    except OSError:
        pass
    return {"cpu_model": model, "logical_cpus": len(allowed),
            "physical_cores": len(cores) if cores else len(allowed)}


def cpu_baseline(batch, budget_s: float, model: str = "eg300m") -> dict:
    """The oracle on consecutive groups of 4 sequences of the workload (each
    padded to its own longest, as the reference's embedBatch pads), until the
    budget is spent. Test infrastructure used as the checker-side baseline.
    OpenMP threads stay at the environment's OMP_NUM_THREADS; they are bound
    close to the launching core (OMP_PROC_BIND=close, set before the oracle
    library starts its runtime)."""
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    from ai_amd import synth as S
    if model == "eg2":
        shape = S.ModelShape2()
        om = O.OracleModel2(shape)
        for name, shp, kind in S.weight_specs2(shape):
            w = S.make_weight(name, shp, kind)
            om.set(name, S.bf16_to_f32(w) if kind == "m" else w)
        om.finalize()
    else:
        om = O.OracleModel(S.ModelShape())
        om.load_synthetic()
    group = 4
    done = tokens = 0
    elapsed = 0.0
    i = 0
    while elapsed < budget_s or done == 0:
        sl = slice(i, i + group)
        L = batch.lengths[sl]
        if L.size == 0:
            i = 0
            continue
        Tm = int(L.max())
        t0 = time.perf_counter()
        om.embed(batch.ids[sl, :Tm], L)
        elapsed += time.perf_counter() - t0
        done += L.size
        tokens += int(L.sum())
        i += group
    om.close()
    threads = O.lib().orc_num_threads()
    hc = host_cpu()
    return {"value": round(done / elapsed, 3), "unit": "sentences/s", "cores": threads, "kind": "port",
            "sample": f"{done} sequences of {batch.name} in groups of {group}, each padded to its group's max "
                      f"length ({tokens} valid tokens, {elapsed:.1f} s, {O.isa()}, OMP threads {threads})",
            "tokens_per_s": round(tokens / elapsed, 1), "threads": threads, "isa": O.isa(),
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"), "omp_places": os.environ.get("OMP_PLACES"), **hc}


def main():
    a = parse()
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {a.gpus}); data-parallel sharding over "
              f"sentences is not run", file=sys.stderr)
        sys.exit(2)
    from ai_amd import _native as N
    from ai_amd import gemma as G
    from ai_amd import synth as S

    ctx = N.Context(0)
    shape = S.ModelShape2() if a.model == "eg2" else S.ModelShape()
    model = G.Model(shape, ctx)
    model.load_synthetic()
    batch = S.make_batch(a.config, with_corpus=False)
    B, T = batch.B, batch.T
    # inputs resident in HBM before timing
    import ctypes as C
    d_ids, d_out = C.c_void_p(), C.c_void_p()
    N.check(ctx.h, N.lib().fa_device_alloc(ctx.h, batch.ids.nbytes, C.byref(d_ids)))
    N.check(ctx.h, N.lib().fa_device_alloc(ctx.h, B * model.Dim() * 4, C.byref(d_out)))
    N.check(ctx.h, N.lib().fa_memcpy_h2d(ctx.h, d_ids, batch.ids.ctypes.data, batch.ids.nbytes))

    def step():
        model.embed_ids_dev(d_ids.value, batch.lengths, B, T, d_out.value)

    # host to host: ids [B, T] and lengths on the host, embeddings back on the
    # host, one synchronisation per step (inside fa_gemma_embed_ids)
    h_out = np.empty((B, model.Dim()), np.float32)
    ids_c = np.ascontiguousarray(batch.ids, np.int32)
    lens_c = np.ascontiguousarray(batch.lengths, np.int32)

    def host_step():
        N.check(ctx.h, N.lib().fa_gemma_embed_ids(model.h, ids_c.ctypes.data, lens_c.ctypes.data, B, T, 0,
                                                  h_out.ctypes.data))

    def timed(fn, steps):
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        ctx.sync()
        return time.perf_counter() - t0

    # the device-resident forward first (ids in HBM, embeddings left there, no
    # per-step synchronisation): three regions of K steps after the warm-up
    for _ in range(a.warmup):
        step()
    dev_runs = [timed(step, a.steps) / a.steps * 1e3 for _ in range(3)]
    dev_med = sorted(dev_runs)[1]

    # the headline: W warm-up steps, then exactly K host-to-host steps
    for _ in range(a.warmup):
        host_step()
    ctx.sync()
    elapsed = timed(host_step, a.steps)
    ms_per_step = elapsed / a.steps * 1e3
    sent_s = B * a.steps / elapsed
    tok_s = batch.tokens * a.steps / elapsed

    # Two more timed regions of the same K steps: min / median over three runs
    # (the reference's protocol, cmd/bench/main.go:46-66); the headline value
    # stays the first region above.
    runs = [ms_per_step] + [timed(host_step, a.steps) / a.steps * 1e3 for _ in range(2)]

    # Second pass over the same steps with every launch bracketed by HIP events.
    model.set_profiling(True)
    model.reset_stats()
    t1 = time.perf_counter()
    for _ in range(a.steps):
        step()
    ctx.sync()
    prof_ms = (time.perf_counter() - t1) / a.steps * 1e3
    stats = model.kernel_stats()
    model.set_profiling(False)

    def kstat(name):
        s = stats[name]
        avg_ms = s["ms"] / max(1, s["launches"])
        per = s["flops"] / max(1, s["launches"])
        perb = s["bytes"] / max(1, s["launches"])
        return s, avg_ms, per, perb

    gs, g_ms, g_flops, _ = kstat("gemm_gateup")
    achieved = g_flops / (g_ms * 1e-3) if g_ms > 0 else 0.0
    roofline = {"kernel": "gemm_x3_kernel split-bf16, GeGLU epilogue (gate|up, M=%d N=%d K=%d)"
                          % (batch.tokens, 2 * shape.intermediate_size, shape.hidden_size),
                "bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": BF16_MFMA_PEAK / 1e12,
                "unit": "TFLOP/s", "frac": round(achieved / BF16_MFMA_PEAK, 4),
                "traffic": GATEUP_TRAFFIC_C2["bytes"] if a.config == "C2" and a.model == "eg300m" else None,
                "launch_ms": round(g_ms, 4), "flops_per_launch": g_flops,
                "mfma_flops_per_launch": SPLIT_TERMS * g_flops,
                "mfma_frac": round(SPLIT_TERMS * achieved / BF16_MFMA_PEAK, 4),
                "ceiling_frac": round(1 / SPLIT_TERMS, 4)}
    kernels = {}
    gemm_fl = gemm_ms = 0.0
    for name in N.KERNEL_KINDS:
        s, avg_ms, per, perb = kstat(name)
        if s["launches"] == 0:
            continue
        e = {"launches_per_step": s["launches"] / a.steps, "ms_per_step": round(s["ms"] / a.steps, 4)}
        if s["flops"]:
            e["tflops"] = round(s["flops"] / (s["ms"] * 1e-3) / 1e12, 2)
            e["frac_fp32_mfma"] = round(s["flops"] / (s["ms"] * 1e-3) / FP32_MFMA_PEAK, 4)
        if s["bytes"]:
            e["GBps"] = round(s["bytes"] / (s["ms"] * 1e-3) / 1e9, 1)
            e["frac_hbm"] = round(s["bytes"] / (s["ms"] * 1e-3) / HBM_PEAK, 4)
        kernels[name] = e
        if name.startswith("gemm"):
            gemm_fl += s["flops"]
            gemm_ms += s["ms"]
    gemm_all = {"tflops": round(gemm_fl / (gemm_ms * 1e-3) / 1e12, 2) if gemm_ms else 0,
                "frac_fp32_mfma": round(gemm_fl / (gemm_ms * 1e-3) / FP32_MFMA_PEAK, 4) if gemm_ms else 0,
                "ms_per_step": round(gemm_ms / a.steps, 3)}
    # The timed throughput (sentences/s and tokens/s are one measurement) as
    # a roofline fraction: the forward's algorithmic flops (every GEMM and
    # the attention, as counted per launch in the event pass) per timed step
    # over the timed step.
    step_fl = sum(stats[n]["flops"] for n in N.KERNEL_KINDS) / a.steps
    throughput_roofline = {"flops_per_step": step_fl,
                           "tflops": round(step_fl / (ms_per_step * 1e-3) / 1e12, 2),
                           "frac_bf16_mfma": round(step_fl / (ms_per_step * 1e-3) / BF16_MFMA_PEAK, 4),
                           "frac_fp32_mfma": round(step_fl / (ms_per_step * 1e-3) / FP32_MFMA_PEAK, 4)}

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(batch, a.cpu_seconds, a.model)

    out = {
        "metric": METRIC,
        "value": round(sent_s, 2),
        "unit": "sentences/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init bf16 weights N(0,0.02), Zipf(1.1) token ids; seeded)",
        "config": {"workload": f"{a.config}: "
                               + ("EmbeddingGemma 2 text tower" if a.model == "eg2" else "EmbeddingGemma-300M encoder")
                               + f" forward, batch {B} x seq {T}, "
                               f"lengths {int(batch.lengths.min())}..{int(batch.lengths.max())}",
                   "batch": B, "seq_len": T, "valid_tokens": batch.tokens},
        "tokens_per_s": round(tok_s, 1),
        "runs_ms_per_step": {"all": [round(r, 3) for r in runs], "min": round(min(runs), 3),
                             "median": round(sorted(runs)[1], 3)},
        "timing": "host ids -> host embeddings per step (fa_gemma_embed_ids, synchronised every step)",
        "device_resident": {"sentences_per_s": round(B / (dev_med * 1e-3), 1),
                            "tokens_per_s": round(batch.tokens / (dev_med * 1e-3), 1),
                            "ms_per_step": {"all": [round(r, 3) for r in dev_runs], "median": round(dev_med, 3)},
                            "note": "ids resident in HBM, embeddings left in HBM, steps enqueued back to back"},
        "roofline": roofline,
        "throughput_roofline": throughput_roofline,
        "gemm_all": gemm_all,
        "kernels": kernels,
        "profiled_ms_per_step": round(prof_ms, 3),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    N.lib().fa_device_free(ctx.h, d_ids)
    N.lib().fa_device_free(ctx.h, d_out)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
