"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "Q4_K matvec GB/s (% HBM peak) @14336x4096; MoE layer us/token
decode"): one step = one batch-1 Q4_K matvec over a 14336x4096 weight (33,030,144 B) with fp32
activations, weights resident in HBM. Copies of the weight are rotated so the streamed footprint
exceeds 512 MB and the 256 MB Infinity Cache cannot serve repeats. The steps are recorded once into
a HIP graph (one launch per weight copy) and the graph is replayed; HIP events on that stream
bracket every timed replay, at least 200 launches are timed whatever --steps says, and the
median per-launch time over the replays is reported. `value` = algorithmic bytes (weights + x + y)
per step / median time per step.

Secondary measurements (same JSON object, "secondary"): the MoE expert layer (config 4) in
us/token at 1 and 8 tokens, the Llama-3-8B layer matvecs and Q8_0 head (config 2), the IQ2_XXS /
IQ3_XXS matvecs (config 5), Q4_K 4096x4096 (config 1), the small-M GEMM (config 3) and the
prefill-shaped GEMMs of the other types, and the streaming-read ceiling of this part at 33 MB and
9.4 MB (a bare read of that many bytes, the practical bound of the matvecs).
The CPU baseline times the oracle (a C restatement of the reference's cpu_ref::matvec) on a
bounded sample of the headline workload on the host's cores.

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


def device_copies(host, min_bytes=ROTATE_BYTES):
    import torch
    first = torch.from_numpy(np.ascontiguousarray(host)).cuda()
    n = max(1, -(-min_bytes // first.numel()))
    return [first] + [first.clone() for _ in range(n - 1)]


def quantized(ty, rows, cols, seed):
    import lastengine_amd as le
    if ty not in le.TYPES.values():
        return synthetic_blocks(ty, rows, cols, seed)
    return le.quantize_rows(ty, le.fill_normal(rows * cols, seed, std=0.02).reshape(rows, cols))


# f16 super-block scale fields per type (block bytes, offsets): Q4_0, Q3_K, Q5_K, IQ2_S
_SCALE_FIELDS = {2: (18, [0]), 11: (110, [108]), 13: (176, [0, 2]), 22: (82, [0])}


def synthetic_blocks(ty, rows, cols, seed):
    """Seeded block bytes for the types this build has no quantizer for (Q4_0, Q3_K, Q5_K, IQ2_S):
    uniform random codes with the f16 scale fields set to finite values in [-0.01, 0.01]."""
    import lastengine_amd as le
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(rows, le.row_bytes(ty, cols)), dtype=np.uint8)
    bb, offs = _SCALE_FIELDS[ty]
    blk = q.reshape(rows, -1, bb)
    for o in offs:
        blk[:, :, o:o + 2] = rng.uniform(-0.01, 0.01, size=blk.shape[:2]).astype(np.float16).view(np.uint8).reshape(
            blk.shape[0], blk.shape[1], 2)
    return q


MIN_TIMED_LAUNCHES = 200


def graph_time(record, n_launch, steps, warmup, min_launches=MIN_TIMED_LAUNCHES):
    """Capture record() (n_launch steps) into a HIP graph, replay it, and time each replay with HIP
    events on the replay stream. At least max(steps, min_launches) steps are timed; returns the
    median per-step time over the replays in ms (plus mean/min/max and counts in .stats)."""
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        record()  # eager warm-up outside capture (loads code objects)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        record()
    for _ in range(max(1, -(-warmup // n_launch))):
        g.replay()
    torch.cuda.synchronize()
    reps = max(3, -(-max(steps, min_launches) // n_launch))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for r in range(reps):
        g.replay()
        evs[r + 1].record()
    torch.cuda.synchronize()
    per = sorted(evs[r].elapsed_time(evs[r + 1]) / n_launch for r in range(reps))
    med = per[len(per) // 2] if len(per) % 2 else 0.5 * (per[len(per) // 2 - 1] + per[len(per) // 2])
    graph_time.stats = {"replays": reps, "launches_per_replay": n_launch, "timed_launches": reps * n_launch,
                        "median_us": round(med * 1e3, 3), "mean_us": round(sum(per) / reps * 1e3, 3),
                        "min_us": round(per[0] * 1e3, 3), "max_us": round(per[-1] * 1e3, 3)}
    return med


def bench_matvec(eng, ty, rows, cols, steps, warmup, seed=1):
    import torch
    import lastengine_amd as le
    host = quantized(ty, rows, cols, seed)
    bufs = device_copies(host)
    x = torch.from_numpy(le.fill_normal(cols, seed + 1)).cuda()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")

    def record():
        for b in bufs:
            eng.mv(ty, b, x, y, rows, cols)
    ms = graph_time(record, len(bufs), steps, warmup)
    alg = host.nbytes + 4 * cols + 4 * rows
    return {"us": ms * 1e3, "ms": ms, "bytes": alg, "gbs": alg / (ms * 1e-3) / 1e9, "copies": len(bufs),
            "timing": dict(graph_time.stats)}, host


def bench_matvec_q8(eng, ty, rows, cols, steps, warmup, seed=1):
    """int8 activation mode: le_matvec_q8 on activations quantize_x'd once (the reference's
    matvec_<ty> launch), and le_quant_x alone."""
    import torch
    import lastengine_amd as le
    host = quantized(ty, rows, cols, seed)
    bufs = device_copies(host)
    x = torch.from_numpy(le.fill_normal(cols, seed + 1)).cuda()
    xq = torch.empty(cols, dtype=torch.int8, device="cuda")
    xd = torch.empty(cols // 32, dtype=torch.float32, device="cuda")
    xs = torch.empty(cols // 32, dtype=torch.int32, device="cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    eng.quant_x(x, xq, xd, xs, cols // 32)

    def record():
        for b in bufs:
            eng.mv_q8(ty, None, xq, xd, xs, y, rows, cols, 0, 1, w=b)
    ms = graph_time(record, len(bufs), steps, warmup)

    def record_qx():
        for _ in range(20):
            eng.quant_x(x, xq, xd, xs, cols // 32)
    msq = graph_time(record_qx, 20, steps, warmup)
    alg = host.nbytes + cols + 8 * (cols // 32) + 4 * rows
    gbs = alg / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "quant_x_us": round(msq * 1e3, 3)}


def bench_layer(eng, mats, steps, warmup):
    """One step = every matvec of `mats` [(name, ty, rows, cols)] in sequence."""
    import torch
    import lastengine_amd as le
    hosts = [quantized(ty, r, c, 50 + i) for i, (_, ty, r, c) in enumerate(mats)]
    total = sum(h.nbytes for h in hosts)
    ncopy = max(1, -(-ROTATE_BYTES // total))
    devs = [device_copies(h, min_bytes=ncopy * h.nbytes) for h in hosts]
    xs = {c: torch.from_numpy(le.fill_normal(c, c)).cuda() for (_, _, _, c) in mats}
    ys = [torch.empty(r, dtype=torch.float32, device="cuda") for (_, _, r, _) in mats]

    # "qkv": q, k and v (same input) as one matvec over a pointer table of 1024-row slots: q's four
    # row blocks, then k and v, outputs [q | k | v] (Gpu::mv_ptrs, src/gpu.rs:228-237)
    tabs = {}
    for i, (name, ty, r, c) in enumerate(mats):
        if name == "qkv":
            rb = le.row_bytes(ty, c)
            assert r % 1024 == 0
            tabs[i] = []
            for k in range(ncopy):
                base = devs[i][k].data_ptr()
                tabs[i].append(torch.tensor([base + j * 1024 * rb for j in range(r // 1024)], dtype=torch.int64, device="cuda"))

    def record():
        for k in range(ncopy):
            for i, (name, ty, r, c) in enumerate(mats):
                if name == "down_swiglu":  # SwiGLU of the previous (gate | up) output fused into the down matvec
                    eng.mv_swiglu(ty, devs[i][k], ys[i - 1], ys[i], r, c)
                elif name == "qkv":
                    eng.mv_ptrs(ty, tabs[i][k], xs[c], ys[i], 1024, c, 0, r // 1024)
                else:
                    eng.mv(ty, devs[i][k], xs[c], ys[i], r, c)
    ms = graph_time(record, ncopy, steps, warmup, min_launches=40)
    alg = total + sum(4 * (r + c) for (_, _, r, c) in mats)
    return {"us": round(ms * 1e3, 3), "GB/s": round(alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "weight_bytes": total}


def bench_gemm(eng, ty, rows, cols, mtok, steps, warmup, seed=3):
    import torch
    import lastengine_amd as le
    host = quantized(ty, rows, cols, seed)
    bufs = device_copies(host)
    x = torch.from_numpy(le.fill_normal(mtok * cols, seed + 1)).cuda()
    y = torch.empty(mtok * rows, dtype=torch.float32, device="cuda")
    ws = torch.empty(max(16, eng.gemm_workspace_size_rows(ty, mtok, rows, cols)), dtype=torch.uint8, device="cuda")

    def record():
        for b in bufs:
            eng.gemm(ty, b, x, mtok, y, rows, cols, ws=ws)
    ms = graph_time(record, len(bufs), steps, warmup, min_launches=20)
    alg = host.nbytes + 4 * mtok * (cols + rows)
    return {"us": round(ms * 1e3, 2), "GB/s": round(alg / (ms * 1e-3) / 1e9, 1),
            "TFLOP/s": round(2.0 * mtok * rows * cols / (ms * 1e-3) / 1e12, 2)}


def unique_experts(logits, k):
    top = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    return len(np.unique(top))


def bench_moe(eng, n_tok, steps, warmup, n_exp=128, k=8, hidden=2048, ff=768, copies=4, variants=8):
    """Config 4: Qwen3-30B-A3B expert layer. Rotates `copies` full expert sets (each 392 MB) and
    `variants` router-logit draws so repeated steps stream different experts."""
    import torch
    import lastengine_amd as le
    tg, td = le.Q4_K, le.Q6_K
    g = quantized(tg, n_exp * ff, hidden, 201)
    u = quantized(tg, n_exp * ff, hidden, 202)
    d = quantized(td, n_exp * hidden, ff, 203)
    per_expert = (g.nbytes + u.nbytes + d.nbytes) // n_exp
    sets = []
    for c in range(copies):
        if c == 0:
            sets.append(tuple(torch.from_numpy(a).cuda() for a in (g, u, d)))
        else:
            sets.append(tuple(t.clone() for t in sets[0]))
    del g, u, d
    lgs = [le.fill_normal(n_tok * n_exp, 300 + i).reshape(n_tok, n_exp) for i in range(variants)]
    dlg = [torch.from_numpy(l).cuda() for l in lgs]
    h = torch.from_numpy(le.fill_normal(n_tok * hidden, 299)).cuda()
    out = torch.empty(n_tok * hidden, dtype=torch.float32, device="cuda")
    nws = eng.moe_workspace_size(n_tok, k, ff)
    if n_tok >= 11:  # room for the grouped form, which takes 11 tokens and more
        nws = max(nws, eng.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    n_launch = copies * variants

    def record():
        for i in range(n_launch):
            gs, us_, ds = sets[i % copies]
            eng.moe(tg, tg, td, gs, us_, ds, n_exp, k, hidden, ff, dlg[i % variants], h, n_tok, out, ws=ws)
    ms = graph_time(record, n_launch, steps, warmup, min_launches=64)
    uniq = float(np.mean([unique_experts(l, k) for l in lgs]))
    wbytes = uniq * per_expert
    res = {"n_tok": n_tok, "us_per_layer": round(ms * 1e3, 3), "us_per_token": round(ms * 1e3 / n_tok, 3),
           "unique_experts": uniq, "weight_bytes": int(wbytes), "GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
           "roofline_us": round(wbytes / (HBM_PEAK_GBS * 1e9) * 1e6, 3)}
    res["x_roofline"] = round(res["us_per_layer"] / res["roofline_us"], 2)
    del sets
    torch.cuda.empty_cache()
    return res


def bench_moe_prefill(eng, n_tok, steps, warmup, n_exp=128, k=8, hidden=2048, ff=768, copies=2):
    """Config 4's expert layer at prefill sizes (grouped matrix-core form): us per layer, tokens/s
    and TFLOP/s over the routed gate/up/down products; `copies` expert sets rotated."""
    import torch
    import lastengine_amd as le
    g = quantized(le.Q4_K, n_exp * ff, hidden, 201)
    u = quantized(le.Q4_K, n_exp * ff, hidden, 202)
    d = quantized(le.Q6_K, n_exp * hidden, ff, 203)
    sets = [tuple(torch.from_numpy(a).cuda() for a in (g, u, d))]
    sets += [tuple(t.clone() for t in sets[0]) for _ in range(copies - 1)]
    del g, u, d
    lg = torch.from_numpy(le.fill_normal(n_tok * n_exp, 400).reshape(n_tok, n_exp)).cuda()
    h = torch.from_numpy(le.fill_normal(n_tok * hidden, 401)).cuda()
    out = torch.empty(n_tok * hidden, dtype=torch.float32, device="cuda")
    nws = max(eng.moe_workspace_size(n_tok, k, ff), eng.moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")

    def record():
        for gs, us_, ds in sets:
            eng.moe(le.Q4_K, le.Q4_K, le.Q6_K, gs, us_, ds, n_exp, k, hidden, ff, lg, h, n_tok, out, ws=ws)
    ms = graph_time(record, copies, steps, warmup, min_launches=8)
    flops = 2.0 * n_tok * k * 3 * hidden * ff
    del sets
    torch.cuda.empty_cache()
    return {"n_tok": n_tok, "us_per_layer": round(ms * 1e3, 2), "tok_per_s": round(n_tok / (ms * 1e-3), 0),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2)}


def host_cpu():
    """(CPU model, logical cores the OS reports)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, os.cpu_count() or 1


# Host threads for the CPU baseline: the CPU share of one GPU on the benchmark boxes (16), or fewer
# where the host has fewer cores.
CPU_THREADS = 16


def cpu_baseline(ty, host_q, rows, cols, budget_s=10.0):
    """Oracle matvec (C restatement of cpu_ref::matvec) on the host cores, bounded sample."""
    import lastengine_amd as le
    import oracle
    model, nproc = host_cpu()
    threads = max(1, min(CPU_THREADS, nproc))
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
            "host_nproc": nproc, "host_cpu": model,
            "sample": "%d full %dx%d Q4_K matvecs by the oracle (rows split over %d threads: the CPU share of one "
                      "GPU on the box, of %d logical cores), %.1f ms each" % (reps, rows, cols, threads, nproc, per * 1e3)}


def bench_stream_read(eng, size, steps, warmup):
    """Practical HBM read ceiling at `size` bytes: le_stream_read over rotated buffers (the best of
    the probe's load forms measured for that size), same graph timing as the matvecs."""
    import torch
    n = max(1, -(-ROTATE_BYTES // size))
    bufs = [torch.ones(size // 4, dtype=torch.int32, device="cuda") for _ in range(n)]
    sink = torch.empty(eng.stream_read_sink_bytes() // 4 * 16, dtype=torch.int32, device="cuda")
    best = None
    for opts in ({"rd_u": 4, "rd_blocks_per_cu": 1, "rd_block": 512}, {"rd_u": 1, "rd_blocks_per_cu": 2, "rd_block": 512}):
        for k, v in opts.items():
            eng.set_option(k, v)

        def record():
            for b in bufs:
                eng.stream_read(b, size, sink)
        ms = graph_time(record, len(bufs), steps, warmup)
        if best is None or ms < best[0]:
            best = (ms, opts)
    for k, v in {"rd_u": 4, "rd_blocks_per_cu": 1, "rd_block": 512}.items():
        eng.set_option(k, v)
    del bufs
    torch.cuda.empty_cache()
    gbs = size / (best[0] * 1e-3) / 1e9
    return {"bytes": size, "us": round(best[0] * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "load_form": best[1]}


PROBES = {
    # name: (kind, type, rows, cols, tokens)
    "headline": ("mv", "Q4_K", 14336, 4096, 1),
    "config1": ("mv", "Q4_K", 4096, 4096, 1),
    "q6k_down": ("mv", "Q6_K", 4096, 14336, 1),
    "q8_0_head": ("mv", "Q8_0", 32000, 4096, 1),
    "iq2xxs": ("mv", "IQ2_XXS", 14336, 4096, 1),
    "iq3xxs": ("mv", "IQ3_XXS", 4096, 14336, 1),
    "gemm_m64": ("gemm", "Q4_K", 14336, 4096, 64),
    "gemm_m512": ("gemm", "Q4_K", 14336, 4096, 512),
    "gemm_q6k_m512": ("gemm", "Q6_K", 4096, 14336, 512),
    "moe_ntok1": ("moe", None, 0, 0, 1),
    "moe_ntok8": ("moe", None, 0, 0, 8),
    "moe_prefill64": ("moe", None, 0, 0, 64),
    "gemm_m8": ("gemm", "Q4_K", 14336, 4096, 8),
    "gemm_m16": ("gemm", "Q4_K", 14336, 4096, 16),
    "q4_0": ("mv", "Q4_0", 14336, 4096, 1),
    "q3_k": ("mv", "Q3_K", 14336, 4096, 1),
    "q5_k": ("mv", "Q5_K", 14336, 4096, 1),
    "iq2_s": ("mv", "IQ2_S", 14336, 4096, 1),
    "gemm_q5k_m512": ("gemm", "Q5_K", 14336, 4096, 512),
    "gemm_iq2s_m512": ("gemm", "IQ2_S", 14336, 4096, 512),
}


def probe(eng, name, launches=100, copy_bytes=256 << 20):
    """Workload for rocprofv3 --pmc passes: `launches` eager launches of one workload of PROBES over
    rotated weight copies, then 10 copies of a `copy_bytes` buffer (torch's elementwise copy kernel)
    whose FETCH_SIZE / WRITE_SIZE per dispatch calibrate the counters against known traffic."""
    import torch
    import lastengine_amd as le
    kind, tname, rows, cols, mtok = PROBES[name]
    wbytes = 0
    if kind == "moe":
        n_exp, k, hidden, ff = 128, 8, 2048, 768
        g = quantized(le.Q4_K, n_exp * ff, hidden, 201)
        u = quantized(le.Q4_K, n_exp * ff, hidden, 202)
        d = quantized(le.Q6_K, n_exp * hidden, ff, 203)
        dg, du, dd = (torch.from_numpy(a).cuda() for a in (g, u, d))
        lgs = [torch.from_numpy(le.fill_normal(mtok * n_exp, 300 + i)).cuda() for i in range(8)]
        h = torch.from_numpy(le.fill_normal(mtok * hidden, 299)).cuda()
        out = torch.empty(mtok * hidden, dtype=torch.float32, device="cuda")
        nws = eng.moe_workspace_size(mtok, k, ff)
        if mtok > 8:  # the grouped (prefill) form: le_moe_route_tok, le_moe_group, le_gqg_*
            nws = max(nws, eng.moe_prefill_workspace_size(mtok, k, n_exp, hidden, ff))
        ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
        for i in range(launches):
            eng.moe(le.Q4_K, le.Q4_K, le.Q6_K, dg, du, dd, n_exp, k, hidden, ff, lgs[i % 8], h, mtok, out, ws=ws)
    else:
        ty = le.MV_TYPES[tname]
        host = quantized(ty, rows, cols, 1)
        wbytes = int(host.nbytes)
        bufs = device_copies(host)
        x = torch.from_numpy(le.fill_normal(mtok * cols, 2)).cuda()
        y = torch.empty(mtok * rows, dtype=torch.float32, device="cuda")
        if kind == "gemm":
            ws = torch.empty(max(16, eng.gemm_workspace_size_rows(ty, mtok, rows, cols)), dtype=torch.uint8, device="cuda")
        for i in range(launches):
            if kind == "mv":
                eng.mv(ty, bufs[i % len(bufs)], x, y, rows, cols)
            else:
                eng.gemm(ty, bufs[i % len(bufs)], x, mtok, y, rows, cols, ws=ws)
    src = torch.ones(copy_bytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": name, "launches": launches, "copy_bytes": copy_bytes, "weight_bytes": wbytes}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe", nargs="?", const="headline", choices=sorted(PROBES),
                    help="counter-pass workload: eager launches of one workload plus a 256 MiB copy kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import lastengine_amd as le

    eng = le.Engine()
    props = torch.cuda.get_device_properties(0)
    log("device:", props.name, getattr(props, "gcnArchName", ""), "CUs", props.multi_processor_count)

    rows, cols = 14336, 4096
    if args.probe:
        probe(eng, args.probe)
        return
    head, host = bench_matvec(eng, le.Q4_K, rows, cols, args.steps, args.warmup)
    log("headline Q4_K %dx%d: %.3f us, %.1f GB/s" % (rows, cols, head["us"], head["gbs"]))

    out = {
        "metric": "Q4_K matvec GB/s (% HBM peak) @14336x4096; MoE layer us/token decode",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "timing": dict(head["timing"], note="value and ms_per_step are the median over the timed graph replays"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k",
        "data": "synthetic: seeded N(0,0.02) weights quantized by this repo's quantizer, N(0,1) activations",
        "config": {"workload": "Q4_K batch-1 matvec 14336x4096 (config 2 gate/up shape)", "rows": rows,
                   "cols": cols, "weight_bytes": int(host.nbytes), "rotated_copies": head["copies"],
                   "activations": "fp32 in, fp32 out, fp32 accumulation"},
        "roofline": {"bound": "hbm", "kernel": "le_ms_12_p2_w4", "achieved": round(head["gbs"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None},
    }
    tr = os.path.join(REPO, "profiles", "traffic_le_ms_12_14336x4096.json")
    if os.path.exists(tr):  # from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this workload
        out["roofline"]["traffic"] = json.load(open(tr)).get("hbm_bytes_per_launch")
        out["roofline"]["traffic_source"] = "profiles/traffic_le_ms_12_14336x4096.md"

    if not args.no_secondary:
        sec = {}
        steps2 = max(100, args.steps // 4)
        for nt in (1, 8, 16):
            r = bench_moe(eng, nt, max(64, steps2 // 4) if nt <= 8 else 16, 32 if nt <= 8 else 4)
            sec["moe_config4_ntok%d" % nt] = r
            log("moe", r)
        for nt in (64, 512, 2048):
            r = bench_moe_prefill(eng, nt, 16, 4)
            sec["moe_config4_prefill_ntok%d" % nt] = r
            log("moe prefill", r)
        r, _ = bench_matvec(eng, le.Q4_K, 4096, 4096, steps2, args.warmup // 4)
        sec["config1_q4k_4096x4096"] = {"us": round(r["us"], 3), "GB/s": round(r["gbs"], 1),
                                        "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        log("config1", sec["config1_q4k_4096x4096"])
        # the reference's dense decode layer: q, k, v (src/gpu/dense.rs:284), o, gate and up as one
        # matrix of concatenated rows (:67-73,309), then down on silu(gate) * up formed inside the
        # down matvec (swiglu_gu + quant_x + matvec_14 in the reference, :310-312)
        # q, k and v read the same input, so they run as one matvec over a pointer table of 1024-row
        # slots (q's four row blocks, k, v; weights as separate tensors, as in the GGUF file)
        layer = [("qkv", le.Q4_K, 6144, 4096), ("wo", le.Q4_K, 4096, 4096), ("gate_up", le.Q4_K, 28672, 4096), ("down_swiglu", le.Q6_K, 4096, 14336)]
        sec["config2_llama3_8b_layer"] = bench_layer(eng, layer, max(40, steps2 // 8), 8)
        log("config2 layer", sec["config2_llama3_8b_layer"])
        sec["config2_q8_0_head_32000x4096"] = bench_layer(eng, [("head", le.Q8_0, 32000, 4096)], max(40, steps2 // 8), 8)
        log("config2 head", sec["config2_q8_0_head_32000x4096"])
        for name, ty, r_, c_ in [("q6k_down_4096x14336", le.Q6_K, 4096, 14336),
                                 ("iq2xxs_14336x4096", le.IQ2_XXS, 14336, 4096),
                                 ("iq3xxs_4096x14336", le.IQ3_XXS, 4096, 14336)]:
            r, _ = bench_matvec(eng, ty, r_, c_, steps2, args.warmup // 4)
            sec[name] = {"us": round(r["us"], 3), "GB/s": round(r["gbs"], 1), "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
            log(name, sec[name])
            torch.cuda.empty_cache()
        for name, ty in [("q4_0", le.Q4_0), ("q3_k", le.Q3_K), ("q5_k", le.Q5_K), ("iq2_s", le.IQ2_S)]:
            r, _ = bench_matvec(eng, ty, 14336, 4096, steps2, args.warmup // 4)
            sec["%s_14336x4096" % name] = {"us": round(r["us"], 3), "GB/s": round(r["gbs"], 1),
                                          "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
            log(name, sec["%s_14336x4096" % name])
            torch.cuda.empty_cache()
        for name, ty, r_, c_ in [("q4k_14336x4096", le.Q4_K, 14336, 4096), ("q6k_4096x14336", le.Q6_K, 4096, 14336)]:
            sec["int8_mode_" + name] = bench_matvec_q8(eng, ty, r_, c_, steps2, args.warmup // 4)
            log("int8 mode", name, sec["int8_mode_" + name])
            torch.cuda.empty_cache()
        sec["config5_iq_gate_up_down"] = bench_layer(
            eng, [("gate", le.IQ2_XXS, 14336, 4096), ("up", le.IQ2_XXS, 14336, 4096), ("down", le.IQ3_XXS, 4096, 14336)],
            max(40, steps2 // 8), 8)
        log("config5", sec["config5_iq_gate_up_down"])
        for mt in (4, 8, 16, 64, 512):
            g = bench_gemm(eng, le.Q4_K, 14336, 4096, mt, max(20, steps2 // (1 + mt // 8)), 4)
            sec["config3_gemm_q4k_14336x4096_m%d" % mt] = g
            log("gemm m=%d" % mt, g)
            torch.cuda.empty_cache()
        # prefill-shaped GEMMs of the other types (config 2 down / head, config 5 shapes)
        for tname, ty, r_, c_, mts in [("q6k_down_4096x14336", le.Q6_K, 4096, 14336, (17, 64, 512)),
                                      ("q8_0_head_32000x4096", le.Q8_0, 32000, 4096, (64, 512)),
                                      ("iq2xxs_14336x4096", le.IQ2_XXS, 14336, 4096, (64, 512)),
                                      ("iq3xxs_4096x14336", le.IQ3_XXS, 4096, 14336, (64, 512)),
                                      ("q4_0_14336x4096", le.Q4_0, 14336, 4096, (64, 512)),
                                      ("q3_k_14336x4096", le.Q3_K, 14336, 4096, (64, 512)),
                                      ("q5_k_14336x4096", le.Q5_K, 14336, 4096, (64, 512)),
                                      ("iq2_s_14336x4096", le.IQ2_S, 14336, 4096, (64, 512))]:
            for mt in mts:
                g = bench_gemm(eng, ty, r_, c_, mt, max(20, steps2 // (1 + mt // 8)), 4)
                sec["gemm_%s_m%d" % (tname, mt)] = g
                log("gemm %s m=%d" % (tname, mt), g)
                torch.cuda.empty_cache()
        for size in (536870912, 33030144, 9437184):
            sec["stream_read_ceiling_%dB" % size] = bench_stream_read(eng, size, steps2, 20)
            log("stream read", size, sec["stream_read_ceiling_%dB" % size])
        out["secondary"] = sec
        ceil = sec.get("stream_read_ceiling_33030144B")
        if ceil:
            out["roofline"]["read_ceiling_GBs"] = ceil["GB/s"]
            out["roofline"]["frac_of_read_ceiling"] = round(head["gbs"] / ceil["GB/s"], 4)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(le.Q4_K, host, rows, cols)
        log("cpu baseline", out["cpu_baseline"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
