"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "Q4_K matvec GB/s (% HBM peak) @14336x4096"): one step = one batch-1
Q4_K matvec over a 14336x4096 weight (33,030,144 B) with fp32 activations, weights already resident
in HBM. Weight copies are rotated so the streamed footprint exceeds 512 MB and the 256 MB Infinity
Cache cannot serve them. `value` = algorithmic bytes (weights + x + y) per step / measured time.

Secondary lines (same JSON object, "secondary"): the other BASELINE configs timed the same way.
The CPU baseline times the oracle (a C restatement of the reference's cpu_ref::matvec) on a bounded
sample of the same workload on the host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 600 << 20  # > 2x the 256 MB Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Matrix:
    """A quantized matrix replicated `copies` times in HBM (rotated per step)."""

    def __init__(self, ty, rows, cols, seed, min_bytes=ROTATE_BYTES):
        import torch
        import lastengine_amd as le
        self.ty, self.rows, self.cols = ty, rows, cols
        src = le.fill_normal(rows * cols, seed, std=0.02).reshape(rows, cols)
        self.host = le.quantize_rows(ty, src)
        self.nbytes = self.host.nbytes
        self.copies = max(1, -(-min_bytes // self.nbytes))
        first = torch.from_numpy(self.host).cuda()
        self.bufs = [first] + [first.clone() for _ in range(self.copies - 1)]

    def __getitem__(self, i):
        return self.bufs[i % self.copies]


def time_steps(step, steps, warmup):
    """Run `step(i)` warmup times, then time `steps` calls between events on the current stream
    (the stream the library launches on). Returns ms per step."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        step(warmup + i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def bench_matvec(eng, ty, rows, cols, steps, warmup, seed=1):
    import torch
    import lastengine_amd as le
    m = Matrix(ty, rows, cols, seed)
    x = torch.from_numpy(le.fill_normal(cols, seed + 1)).cuda()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ms = time_steps(lambda i: eng.mv(ty, m[i], x, y, rows, cols), steps, warmup)
    alg = m.nbytes + 4 * cols + 4 * rows
    return {"ms": ms, "us": ms * 1e3, "bytes": alg, "gbs": alg / (ms * 1e-3) / 1e9}, m


def bench_gemm(eng, ty, rows, cols, mtok, steps, warmup, seed=3):
    import torch
    import lastengine_amd as le
    m = Matrix(ty, rows, cols, seed)
    x = torch.from_numpy(le.fill_normal(mtok * cols, seed + 1)).cuda()
    y = torch.empty(mtok * rows, dtype=torch.float32, device="cuda")
    ms = time_steps(lambda i: eng.gemm(ty, m[i], x, mtok, y, rows, cols), steps, warmup)
    flops = 2.0 * mtok * rows * cols
    alg = m.nbytes + 4 * mtok * (cols + rows)
    return {"m": mtok, "us": ms * 1e3, "gbs": alg / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12}


def cpu_baseline(ty, host_q, rows, cols, budget_s=2.0):
    """Oracle matvec (C restatement of cpu_ref::matvec) on the host cores, bounded sample."""
    import lastengine_amd as le
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    x = le.fill_normal(cols, 2)
    oracle.matvec(ty, host_q, rows, cols, x, nthreads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.matvec(ty, host_q, rows, cols, x, nthreads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and reps >= 3:
            break
    per = el / reps
    gbs = (host_q.nbytes + 4 * cols + 4 * rows) / per / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": "%d full %dx%d Q4_K matvecs (oracle, %d threads), %.1f ms each" % (reps, rows, cols, threads,
                                                                                     per * 1e3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box here has one "
              "GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import lastengine_amd as le

    eng = le.Engine()
    props = torch.cuda.get_device_properties(0)
    log("device:", props.name, getattr(props, "gcnArchName", ""), "CUs", props.multi_processor_count)

    rows, cols = 14336, 4096
    head, m = bench_matvec(eng, le.Q4_K, rows, cols, args.steps, args.warmup)
    log("headline Q4_K %dx%d: %.2f us, %.1f GB/s" % (rows, cols, head["us"], head["gbs"]))

    out = {
        "metric": "Q4_K matvec GB/s (% HBM peak) @14336x4096; MoE layer us/token decode",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x fp32 activations, fp32 accumulate",
        "data": "synthetic: seeded N(0,0.02) weights quantized by this repo's Q4_K quantizer, N(0,1) activations",
        "config": {"workload": "Q4_K batch-1 matvec 14336x4096 (gate/up of a Llama-3-8B layer)", "rows": rows,
                   "cols": cols, "weight_bytes": m.nbytes, "rotated_copies": m.copies,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "le_mv_12_g8_t1", "achieved": round(head["gbs"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None},
    }

    if not args.no_secondary:
        sec = {}
        steps2 = max(50, args.steps // 4)
        for name, ty, r, c in [("cfg1_q4k_4096x4096", le.Q4_K, 4096, 4096),
                               ("q6k_4096x14336", le.Q6_K, 4096, 14336),
                               ("q8_0_head_32000x4096", le.Q8_0, 32000, 4096),
                               ("iq2xxs_14336x4096", le.IQ2_XXS, 14336, 4096),
                               ("iq3xxs_4096x14336", le.IQ3_XXS, 4096, 14336)]:
            r_, _ = bench_matvec(eng, ty, r, c, steps2, args.warmup // 4)
            sec[name] = {"us": round(r_["us"], 3), "GB/s": round(r_["gbs"], 1),
                         "frac_hbm": round(r_["gbs"] / HBM_PEAK_GBS, 4)}
            log(name, sec[name])
            torch.cuda.empty_cache()
        for mt in (4, 8, 16, 64, 512):
            g = bench_gemm(eng, le.Q4_K, 14336, 4096, mt, max(20, steps2 // (1 + mt // 16)), 5)
            sec["gemm_q4k_14336x4096_m%d" % mt] = {"us": round(g["us"], 2), "GB/s": round(g["gbs"], 1),
                                                  "TFLOP/s": round(g["tflops"], 2)}
            log("gemm m=%d" % mt, sec["gemm_q4k_14336x4096_m%d" % mt])
        out["secondary"] = sec

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(le.Q4_K, m.host, rows, cols)
        log("cpu baseline", out["cpu_baseline"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
