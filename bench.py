"""Benchmark of the MI355X quantized matrix-multiply path (one GPU).

Headline workload: Q4_K dequant-GEMV, W 17408 x 5120 (N(0, 0.02), seed 2,
quantized by this repo's quantizer), x one row of 5120 fp32 (N(0, 1), seed 1002), y fp32.
One step = one GEMV over one weight copy. The weights rotate over enough copies (>= 512 MB)
that the 256 MB MALL cannot serve repeated reads; inputs are resident in HBM before timing.

`value` = algorithmic bytes per step (stored W + 4 M K + 4 M N) / time per step, in GB/s.
Also reported on the same line: the Q6_K GEMVs (config 3), the fused gate/up Q4_K GEMM at
M = 512 (config 4) in TFLOP/s, the roofline of the headline kernel, and the CPU oracle
(a port of the reference's cpu::matmul) timed on the host cores on the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 512 << 20


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def make_weights(hl, t, rows, cols, seed, outliers=0.0):
    w = hl.fill_normal(seed, rows * cols, 0.0, 0.02).reshape(rows, cols)
    if outliers:
        k = max(1, int(round(cols * outliers)))
        w[:, np.random.default_rng(seed + 7).choice(cols, size=k, replace=False)] *= 8.0
    return hl.quantize(t, w.reshape(-1))


def device_copies(hl, torch, t, wq, rows, cols, min_bytes=MALL_BYTES):
    """SLAB images on the device, enough copies to exceed `min_bytes` in total."""
    one = torch.empty(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device="cuda")
    src = torch.from_numpy(wq).to("cuda")
    hl.repack_slab(t, src, rows, cols, one)
    del src
    n = max(2, math.ceil(min_bytes / one.numel()) + 1)
    copies = [one] + [one.clone() for _ in range(n - 1)]
    torch.cuda.synchronize()
    return copies


WINDOW_MS = 150.0  # wall time each extra workload is replayed for, split into SAMPLES samples
SAMPLES = 5


def _warm_graph(torch, launch, indices):
    """Eager warm-up over the weight copies on a side stream (also loads the code objects and
    creates the library's per-stream workspace there), then a HIP graph of launch(i) for i in
    indices captured on that stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in sorted(set(indices)):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in indices:
            launch(i)
    return g


def time_exact(torch, launch, n_copies, steps, warmup):
    """The headline's timing: `warmup` untimed steps, then exactly `steps` steps (one launch
    over the next weight copy each) in one graph replay, bracketed by a synchronize and HIP
    events on the stream the graph replays on. Returns ms per step."""
    gk = _warm_graph(torch, launch, [i % n_copies for i in range(steps)])
    if warmup > 0:
        gw = _warm_graph(torch, launch, [i % n_copies for i in range(warmup)])
        gw.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    gk.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_window(torch, launch, n_copies, min_ms=WINDOW_MS, samples=SAMPLES):
    """Replays of one pass over the weight copies for at least min_ms of GPU time, in `samples`
    samples bracketed by HIP events; returns (median ms per step, the samples, steps timed)."""
    g = _warm_graph(torch, launch, list(range(n_copies)))
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    pass_ms = max(e0.elapsed_time(e1), 1e-3)
    reps = max(1, math.ceil(min_ms / samples / pass_ms))
    per = []
    for _ in range(samples):
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / (reps * n_copies))
    return sorted(per)[len(per) // 2], per, samples * reps * n_copies


def time_per_launch(torch, launch, n_copies, iters):
    """Events around each single eager launch (the kernel's own duration plus event overhead)."""
    cur = torch.cuda.current_stream()
    pairs = []
    for k in range(iters):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur)
        launch(k % n_copies)
        b.record(cur)
        pairs.append((a, b))
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in pairs)
    return ts[len(ts) // 2], sum(ts) / len(ts)


def gemv_case(hl, torch, t, rows, cols, m, seed, steps=0, warmup=0, outliers=0.0, norm=False, exact_steps=False,
              variant=0):
    wq = make_weights(hl, t, rows, cols, seed, outliers)
    copies = device_copies(hl, torch, t, wq, rows, cols)
    x = torch.from_numpy(hl.fill_normal(seed + 1000, m * cols).reshape(m, cols)).to("cuda")
    y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
    nw = torch.from_numpy(hl.fill_normal(seed + 2000, cols, 1.0, 0.1)).to("cuda") if norm else None

    def launch(i):
        hl.gemv(t, copies[i], x, y, rows, cols, m, norm_w=nw, variant=variant)

    ms, samples, n = time_window(torch, launch, len(copies))
    r = {"ms": ms, "samples_us": [round(v * 1e3, 3) for v in samples], "steps": n}
    if exact_steps:  # the headline: exactly `steps` timed steps after `warmup`
        r["exact_ms"] = time_exact(torch, launch, len(copies), steps, warmup)
        med, mean = time_per_launch(torch, launch, len(copies), 200)
        r.update(event_median_us=med * 1e3, event_mean_us=mean * 1e3)
    algo = len(wq) + 4 * m * cols + 4 * m * rows + (4 * cols if norm else 0)
    del copies
    torch.cuda.empty_cache()
    r.update(bytes=algo, gbs=algo / (ms * 1e-3) / 1e9, wq=wq, x=x.cpu().numpy())
    return r


def lm_head_case(hl, torch, t, rows, cols, m, seed, outliers=0.0):
    """The LM head (halo_mi_lm_head): the gemv over the vocabulary with the argmax fused into
    its epilogue, the logits not kept. Same bytes as the plain GEMV plus 12 B of result words
    per vector."""
    wq = make_weights(hl, t, rows, cols, seed, outliers)
    copies = device_copies(hl, torch, t, wq, rows, cols)
    x = torch.from_numpy(hl.fill_normal(seed + 1000, m * cols).reshape(m, cols)).to("cuda")
    res = torch.empty((m, 3), dtype=torch.int32, device="cuda")

    def launch(i):
        hl.lm_head(t, copies[i], x, res, rows, cols, m)

    ms, samples, n = time_window(torch, launch, len(copies))
    algo = len(wq) + 4 * m * cols + 12 * m
    del copies
    torch.cuda.empty_cache()
    return {"bytes": algo, "ms": ms, "steps": n, "gbs": algo / (ms * 1e-3) / 1e9}


def gemm_case(hl, torch, t, rows, cols, m, seed, variant=0):
    wg = make_weights(hl, t, rows, cols, seed)
    wu = make_weights(hl, t, rows, cols, seed + 40)
    cg = device_copies(hl, torch, t, wg, rows, cols, MALL_BYTES // 2)
    cu = device_copies(hl, torch, t, wu, rows, cols, MALL_BYTES // 2)
    n = min(len(cg), len(cu))
    x = torch.from_numpy(hl.fill_normal(seed + 1000, m * cols).reshape(m, cols)).to("cuda")
    out = torch.empty((m, rows), dtype=torch.float32, device="cuda")

    def launch(i):
        hl.gate_up_swiglu(t, cg[i], cu[i], x, out, rows, cols, m, variant=variant)

    ms, samples, nsteps = time_window(torch, launch, n)
    flops = 4.0 * m * rows * cols
    del cg, cu
    torch.cuda.empty_cache()
    return {"flops": flops, "ms": ms, "steps": nsteps, "tflops": flops / (ms * 1e-3) / 1e12,
            "samples_us": [round(v * 1e3, 3) for v in samples]}


# name -> (kind, type, rows, cols, M, seed): the workloads of the extra figures
WORKLOADS = {
    "q4k_gemv_17408x5120_m1": ("gemv", "Q4_K", 17408, 5120, 1, 2),
    "q4k_gemv_17408x5120_m4": ("gemv", "Q4_K", 17408, 5120, 4, 2),
    "q6k_gemv_5120x17408_m1": ("gemv", "Q6_K", 5120, 17408, 1, 3),
    "q6k_gemv_5120x17408_m4": ("gemv", "Q6_K", 5120, 17408, 4, 3),
    "q4k_gate_up_swiglu_m2": ("gemm", "Q4_K", 17408, 5120, 2, 4),
    "q4k_gate_up_swiglu_m8": ("gemm", "Q4_K", 17408, 5120, 8, 4),
    "q4k_gate_up_swiglu_m64": ("gemm", "Q4_K", 17408, 5120, 64, 4),
    "q4k_gate_up_swiglu_m512": ("gemm", "Q4_K", 17408, 5120, 512, 4),
    "q4k_gemv_norm_17408x5120_m1": ("gemv_norm", "Q4_K", 17408, 5120, 1, 2),
    "q5k_gemv_17408x5120_m1": ("gemv", "Q5_K", 17408, 5120, 1, 6),
    "iq4xs_gemv_17408x5120_m1": ("gemv", "IQ4_XS", 17408, 5120, 1, 7),
    "q5k_gate_up_swiglu_m512": ("gemm", "Q5_K", 17408, 5120, 512, 6),
    "iq4xs_gate_up_swiglu_m512": ("gemm", "IQ4_XS", 17408, 5120, 512, 7),
    "upload_q4k_17408x5120": ("upload", "Q4_K", 17408, 5120, 0, 2),
    "model_upload_64_layers": ("model_upload", None, 0, 0, 64, 9),
    "q6k_lm_head_151936x5120_m1": ("head", "Q6_K", 151936, 5120, 1, 3),
    "q6k_lm_head_248320x5120_m1": ("head", "Q6_K", 248320, 5120, 1, 8),
    "hybrid_layer_m1": ("layer", None, 0, 0, 1, 5),
    "hybrid_layer_m4": ("layer", None, 0, 0, 4, 5),
    "hybrid_layer_m512": ("layer", None, 0, 0, 512, 5),
    "hybrid_layer_m1_qk_fused": ("layer_qk", None, 0, 0, 1, 5),
    "hybrid_layer_m1_qkv_group": ("layer_qkv", None, 0, 0, 1, 5),
    "hybrid_layer_m1_qk_fused_qkv_group": ("layer_qk_qkv", None, 0, 0, 1, 5),
    "hybrid_layer_m4_qkv_group": ("layer_qkv", None, 0, 0, 4, 5),
    "hybrid_layer_m512_qkv_group": ("layer_qkv", None, 0, 0, 512, 5),
    "q4k_gemv_17408x5120_m8": ("gemv", "Q4_K", 17408, 5120, 8, 2),
    "q6k_gemv_151936x5120_m1": ("gemv", "Q6_K", 151936, 5120, 1, 3),
    "q4k_gate_up_swiglu_m4": ("gemm", "Q4_K", 17408, 5120, 4, 4),
    "read_floor_50MB": ("read_floor", None, 17408 * 2880, 0, 0, 0),
    "read_floor_73MB": ("read_floor", None, 5120 * 14280, 0, 0, 0),
}

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_17408x5120_m1_traffic.json")


def measured_traffic():
    """HBM bytes per launch of the headline kernel, from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary written by `python -m halo_amd.profiling traffic` (None when it is absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return {"traffic_bytes": round(t["traffic_bytes"]), "source": os.path.relpath(TRAFFIC_FILE, ROOT)}


# one synthetic Q4_K_M-mixed hybrid layer, hidden 5120: (name, type, rows, cols)
LAYER = [
    ("gdn_in", "Q4_K", 12288, 5120),
    ("gdn_out", "Q4_K", 5120, 6144),
    ("q", "Q4_K", 6144, 5120),
    ("k", "Q4_K", 1024, 5120),
    ("v", "Q6_K", 1024, 5120),
    ("o", "Q4_K", 5120, 6144),
    ("gate_up", "Q4_K", 17408, 5120),  # two matrices, one fused gate/up/SwiGLU call
    ("down", "Q6_K", 5120, 17408),
]


def upload_case(hl, torch, t, rows, cols, seed, reps=10):
    """North-star part (c): GGUF rows -> SLAB image. The device repack (GGUF bytes already in
    HBM; reads and writes the matrix once: 2 x bytes of traffic) and the host upload from
    pinned memory through halo_mi_upload_slab (PCIe-inclusive; never the headline value)."""
    wq = make_weights(hl, t, rows, cols, seed)
    nbytes = len(wq)
    src = torch.from_numpy(wq).to("cuda")
    dst = torch.empty(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device="cuda")
    hl.repack_slab(t, src, rows, cols, dst)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        hl.repack_slab(t, src, rows, cols, dst)
    e1.record()
    torch.cuda.synchronize()
    repack_ms = e0.elapsed_time(e1) / reps
    pinned = torch.from_numpy(wq).pin_memory()
    host = pinned.numpy()
    hl.upload_slab(t, host, rows, cols, dst)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        hl.upload_slab(t, host, rows, cols, dst)
    torch.cuda.synchronize()
    upload_ms = (time.perf_counter() - t0) * 1e3 / reps
    # pageable host memory, as from an mmap'd GGUF file
    t0 = time.perf_counter()
    for _ in range(reps):
        hl.upload_slab(t, wq, rows, cols, dst)
    torch.cuda.synchronize()
    pageable_ms = (time.perf_counter() - t0) * 1e3 / reps
    del src, dst, pinned
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "repack_us": repack_ms * 1e3, "repack_gbs": 2 * nbytes / (repack_ms * 1e-3) / 1e9,
            "upload_ms": upload_ms, "upload_gbs": nbytes / (upload_ms * 1e-3) / 1e9,
            "pageable_ms": pageable_ms, "pageable_gbs": nbytes / (pageable_ms * 1e-3) / 1e9}


def model_upload_case(hl, torch, layers=64, seed=9):
    """Row (f3): a model-scale load. `layers` copies of the config-5 layer (269 MB each, so 64
    layers are 17.2 GB) from pageable host memory into SLAB images in one device arena with one
    halo_mi_upload_tensors call; q|k and gate|up are uploaded as row-fused projections (the
    pair kernel takes the up half at the gate half's end). Host bytes are random: the upload
    moves bytes and does not read them. PCIe-inclusive, so never a headline value."""
    rng = np.random.default_rng(seed)
    plan = [("gdn_in", ["gdn_in"]), ("gdn_out", ["gdn_out"]), ("qk", ["q", "k"]), ("v", ["v"]), ("o", ["o"]),
            ("gate_up", ["gate_up", "gate_up"]), ("down", ["down"])]
    spec = {name: (int(getattr(hl.DType, tn)), rows, cols) for name, tn, rows, cols in LAYER}
    src = {name: rng.integers(0, 256, size=rows * hl.row_bytes(t, cols), dtype=np.uint8)
           for name, (t, rows, cols) in spec.items()}
    per_layer, offs = 0, []
    for fused, parts in plan:
        t, _, cols = spec[parts[0]]
        rows = sum(spec[p][1] for p in parts)
        offs.append((fused, t, cols, parts, per_layer))
        per_layer += hl.slab_bytes(t, rows, cols)
    arena = torch.empty(per_layer * layers, dtype=torch.uint8, device="cuda")
    base = arena.data_ptr()
    tensors = [(t, cols, [(src[p], spec[p][1]) for p in parts], base + l * per_layer + off)
               for l in range(layers) for (fused, t, cols, parts, off) in offs]
    nbytes = layers * sum(len(src[p]) for _, parts in plan for p in parts)
    hl.upload_tensors(tensors[:len(plan)])  # warm-up: page-in of the sources, the first pinned buffers
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hl.upload_tensors(tensors)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    del arena
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "s": sec, "gbs": nbytes / sec / 1e9, "tensors": len(tensors)}


def layer_case(hl, torch, m, seed=5, fuse_qk=False, group_qkv=False):
    """All matmuls of one config-5 layer as one step (the fused gate/up pair is one call), over
    enough copies of the layer's weights that the MALL cannot serve repeats. fuse_qk: q and k
    (both Q4_K, 5120 columns) as one row-fused 7168-row matrix, one GEMV instead of two (the
    reference's try_make_fused; v is Q6_K, so it stays apart). group_qkv: q (or q|k), k and v
    in one grouped call (two weight types): halo_mi_gemv_group up to 8 vectors, the grouped bf16
    GEMM halo_mi_gemm_group above."""
    layer = LAYER
    if fuse_qk:
        layer = [(n, tn, r, c) for n, tn, r, c in LAYER if n not in ("q", "k")]
        layer.insert(2, ("qk", "Q4_K", 6144 + 1024, 5120))
    mats = []
    one_copy = 0
    for i, (name, tn, rows, cols) in enumerate(layer):
        t = int(getattr(hl.DType, tn))
        ws = [make_weights(hl, t, rows, cols, seed * 100 + 10 * i + j) for j in range(2 if name == "gate_up" else 1)]
        dev = []
        for wq in ws:
            d = torch.empty(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device="cuda")
            hl.repack_slab(t, torch.from_numpy(wq).to("cuda"), rows, cols, d)
            dev.append(d)
            one_copy += d.numel()
        mats.append((name, t, rows, cols, dev, sum(len(w) for w in ws)))
    n_copies = max(2, math.ceil(MALL_BYTES / one_copy) + 1)
    copies = [mats] + [[(n, t, r, c, [d.clone() for d in dv], wb) for (n, t, r, c, dv, wb) in mats] for _ in range(n_copies - 1)]
    xs = {c: torch.from_numpy(hl.fill_normal(seed + 1000 + c, m * c).reshape(m, c)).to("cuda") for c in {5120, 6144, 17408}}
    ys = {name: torch.empty((m, rows), dtype=torch.float32, device="cuda") for name, _, rows, _, _, _ in mats}

    def launch(i):
        group = []
        for name, t, rows, cols, dev, _ in copies[i]:
            if name == "gate_up":
                hl.gate_up_swiglu(t, dev[0], dev[1], xs[cols], ys[name], rows, cols, m)
            elif group_qkv and name in ("q", "k", "qk", "v"):
                group.append((t, dev[0], rows, ys[name]))
            else:
                hl.gemv(t, dev[0], xs[cols], ys[name], rows, cols, m)
        if group:
            (hl.gemm_group if m > 8 else hl.gemv_group)(group, xs[5120], 5120, m)

    ms, samples, nsteps = time_window(torch, launch, n_copies)
    algo = sum(wb + 4 * m * cols + 4 * m * rows for name, _, rows, cols, _, wb in mats)
    flops = sum((4.0 if name == "gate_up" else 2.0) * m * rows * cols for name, _, rows, cols, _, _ in mats)
    del copies, mats
    torch.cuda.empty_cache()
    return {"ms": ms, "steps": nsteps, "bytes": algo, "gbs": algo / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12}


def read_floor_case(hl, torch, nbytes, min_bytes=MALL_BYTES):
    """The single-launch read floor of `nbytes`: halo_mi_stream_read (a plain read-only stream,
    nothing computed or written) over enough copies that the MALL cannot serve repeats; the
    best of a sweep of launch shapes (workgroups per CU x loads in flight per thread)."""
    n = max(2, math.ceil(min_bytes / nbytes) + 1)
    bufs = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(n)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(cus * 64 * 256, dtype=torch.int32, device="cuda")
    best = None
    for per_cu in (4, 8, 16, 32):
        for unroll in (4, 8, 16):
            wgs = cus * per_cu

            def launch(i, wgs=wgs, unroll=unroll):
                hl.stream_read(bufs[i], nbytes, wgs, unroll, sink)

            ms, _, _ = time_window(torch, launch, n, min_ms=30.0, samples=3)
            if best is None or ms < best[0]:
                best = (ms, per_cu, unroll, launch)
    ms, samples, _ = time_window(torch, best[3], n)
    del bufs
    torch.cuda.empty_cache()
    return {"us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9, "workgroups_per_cu": best[1], "loads_in_flight": best[2],
            "samples_us": [round(v * 1e3, 3) for v in samples]}


def cpu_baseline(t, wq, rows, cols, x, seconds, threads=0):
    """The oracle (a C port of the reference's cpu::matmul) on `threads` host cores (0 = all),
    best of N after one warm-up, for about `seconds` of CPU time."""
    from oracle import oracle as orc

    threads = threads or orc.default_threads()
    orc.matmul(t, wq, rows, cols, x, threads=threads)
    best, spent, runs = float("inf"), 0.0, 0
    while runs == 0 or (spent < seconds and runs < 1000):
        t0 = time.perf_counter()
        orc.matmul(t, wq, rows, cols, x, threads=threads)
        dt = time.perf_counter() - t0
        best, spent, runs = min(best, dt), spent + dt, runs + 1
    algo = len(wq) + 4 * x.size + 4 * x.shape[0] * rows
    return {"value": round(algo / best / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"full Q4_K {rows}x{cols} M={x.shape[0]} GEMV, best of {runs} runs after 1 warm-up "
                      f"({spent:.1f} s total), oracle/oracle.c built -O2 -ffp-contract=off",
            "ms_per_call": round(best * 1e3, 3)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed steps of the headline workload (exactly)")
    ap.add_argument("--warmup", type=int, default=200, help="untimed steps before them")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--only", choices=sorted(WORKLOADS),
                    help="run one workload alone and print its figures (for profiling); no headline line")
    ap.add_argument("--variant", type=int, default=0, help="kernel variant id for --only gemv / gemm workloads "
                    "(halo_mi_gemv_params::variant; 0 = the default choice)")
    ap.add_argument("--rows", type=int, default=0, help="--only gemv / gemm workloads: rows instead of the workload's")
    ap.add_argument("--m", type=int, default=0, help="--only gemv / gemm workloads: vectors instead of the workload's")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after the benchmark, copy a buffer of this many MiB 4 times (a plain copy kernel of "
                         "known size, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1).",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch

    import halo_amd as hl

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    hl.lib()
    Q4_K, Q6_K = int(hl.DType.Q4_K), int(hl.DType.Q6_K)
    if args.only:
        kind, t, rows, cols, m, seed = WORKLOADS[args.only]
        log(f"only {args.only}")
        if kind == "upload":
            r = upload_case(hl, torch, int(getattr(hl.DType, t)), rows, cols, seed)
            print(json.dumps({"workload": args.only, **{k: round(v, 3) for k, v in r.items()}}), flush=True)
            return 0
        if kind == "model_upload":
            r = model_upload_case(hl, torch, m, seed)
            print(json.dumps({"workload": args.only, "GB": round(r["bytes"] / 1e9, 2), "s": round(r["s"], 3),
                              "GB/s": round(r["gbs"], 1)}), flush=True)
            return 0
        if kind == "read_floor":
            r = read_floor_case(hl, torch, rows)
            print(json.dumps({"workload": args.only, **{k: v for k, v in r.items()}}), flush=True)
            return 0
        if kind.startswith("layer"):
            r = layer_case(hl, torch, m, seed, fuse_qk="qk" in kind.split("_")[1:], group_qkv=kind.endswith("qkv"))
            print(json.dumps({"workload": args.only, "us_per_layer": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                              "TFLOP/s": round(r["tflops"], 2)}), flush=True)
            return 0
        t = int(getattr(hl.DType, t))
        rows = args.rows or rows
        m = args.m or m
        if kind == "head":
            r = lm_head_case(hl, torch, t, rows, cols, m, seed, outliers=0.01)
            print(json.dumps({"workload": args.only, "GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3)}), flush=True)
            return 0
        if kind in ("gemv", "gemv_norm"):
            r = gemv_case(hl, torch, t, rows, cols, m, seed, norm=kind == "gemv_norm",
                          outliers=0.01 if rows == 151936 else 0.0, variant=args.variant)
            out = {"workload": args.only, "GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3)}
        else:
            r = gemm_case(hl, torch, t, rows, cols, m, seed, variant=args.variant)
            out = {"workload": args.only, "TFLOP/s": round(r["tflops"], 2), "us": round(r["ms"] * 1e3, 3)}
        print(json.dumps(out), flush=True)
        return 0

    def gemv_fig(r):
        return {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 2), "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}

    def gemm_fig(r):
        return {"TFLOP/s": round(r["tflops"], 2), "us": round(r["ms"] * 1e3, 2),
                "frac_bf16_peak": round(r["tflops"] / BF16_PEAK_TFLOPS, 4)}

    log(f"config 2: Q4_K GEMV 17408x5120 M=1 ({args.warmup} warm-up steps, {args.steps} timed steps)")
    head = gemv_case(hl, torch, Q4_K, 17408, 5120, 1, 2, args.steps, args.warmup, exact_steps=True)
    # average launch duration: HIP events around the timed region, on the stream the graph (and
    # so the kernels) runs on, divided by the launches in it
    kernel_us = head["exact_ms"] * 1e3
    achieved = head["bytes"] / (kernel_us * 1e-6) / 1e9
    traffic = measured_traffic()
    log("read floor: one read-only stream over the headline's 50 MB of weights")
    floor = read_floor_case(hl, torch, hl.slab_bytes(Q4_K, 17408, 5120))
    extra = {"q4k_gemv_17408x5120_m1_window": {**gemv_fig(head), "samples_us": head["samples_us"],
                                                "note": f"median of {SAMPLES} samples over {WINDOW_MS:.0f} ms of replays"}}
    if not args.no_extra:
        log("read floor of the 73 MB Q6_K 5120x17408 matrix")
        r = read_floor_case(hl, torch, hl.slab_bytes(Q6_K, 5120, 17408))
        extra["read_floor_73MB"] = {"us": round(r["us"], 2), "GB/s": round(r["gbs"], 1), "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        log("config 2 with the fused RMS-norm prologue (norm_w): Q4_K GEMV M=1")
        extra["q4k_gemv_norm_17408x5120_m1"] = gemv_fig(gemv_case(hl, torch, Q4_K, 17408, 5120, 1, 2, norm=True))
        log("config 2: Q4_K GEMV M=4")
        extra["q4k_gemv_17408x5120_m4"] = gemv_fig(gemv_case(hl, torch, Q4_K, 17408, 5120, 4, 2))
        for m in (1, 2, 3, 4):
            log(f"config 3: Q6_K GEMV 5120x17408 M={m}")
            extra[f"q6k_gemv_5120x17408_m{m}"] = gemv_fig(gemv_case(hl, torch, Q6_K, 5120, 17408, m, 3))
        for m in (1, 4):
            log(f"config 3: Q6_K GEMV 151936x5120 M={m} (1% outlier columns)")
            extra[f"q6k_gemv_151936x5120_m{m}"] = gemv_fig(gemv_case(hl, torch, Q6_K, 151936, 5120, m, 3, outliers=0.01))
        for name, tn, seed in (("q5k", "Q5_K", 6), ("iq4xs", "IQ4_XS", 7)):
            log(f"the UD pack's other formats: {tn} GEMV 17408x5120 M=1 and gate/up M=512")
            tt = int(getattr(hl.DType, tn))
            extra[f"{name}_gemv_17408x5120_m1"] = gemv_fig(gemv_case(hl, torch, tt, 17408, 5120, 1, seed))
            extra[f"{name}_gate_up_swiglu_m512"] = gemm_fig(gemm_case(hl, torch, tt, 17408, 5120, 512, seed))
        log("LM head: Q6_K 151936x5120 M=1 with the fused argmax (no logits kept)")
        r = lm_head_case(hl, torch, Q6_K, 151936, 5120, 1, 3, outliers=0.01)
        extra["q6k_lm_head_151936x5120_m1"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 2),
                                               "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        log("LM head at the model's own vocabulary: Q6_K 248320x5120 M=1 (1.04 GB), fused argmax")
        r = lm_head_case(hl, torch, Q6_K, 248320, 5120, 1, 8, outliers=0.01)
        extra["q6k_lm_head_248320x5120_m1"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 2),
                                               "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        log("part (c): GGUF -> SLAB repack and host upload, Q4_K 17408x5120")
        r = upload_case(hl, torch, Q4_K, 17408, 5120, 2)
        extra["q4k_17408x5120_repack_device"] = {"us": round(r["repack_us"], 2), "GB/s": round(r["repack_gbs"], 1),
                                                  "note": "reads + writes the 50 MB matrix once"}
        extra["q4k_17408x5120_upload_from_pinned_host"] = {"ms": round(r["upload_ms"], 3), "GB/s": round(r["upload_gbs"], 1),
                                                           "note": "PCIe-inclusive, 64 MiB chunks through one staging buffer"}
        extra["q4k_17408x5120_upload_from_pageable_host"] = {"ms": round(r["pageable_ms"], 3),
                                                             "GB/s": round(r["pageable_gbs"], 1),
                                                             "note": "as from an mmap'd GGUF file"}
        log("row (f3): model-scale upload, 64 config-5 layers (17.2 GB) with row-fused q|k and gate|up")
        r = model_upload_case(hl, torch, 64)
        extra["model_upload_64_layers_pageable"] = {"GB": round(r["bytes"] / 1e9, 2), "s": round(r["s"], 3),
                                                    "GB/s": round(r["gbs"], 1), "tensors": r["tensors"],
                                                    "note": "host -> SLAB, PCIe-inclusive, one upload_tensors call"}
        log("config 1 on the GPU: Q4_0 GEMV 4096x4096 M=1")
        extra["q4_0_gemv_4096x4096_m1"] = gemv_fig(gemv_case(hl, torch, int(hl.DType.Q4_0), 4096, 4096, 1, 0))
        for m in (1, 4, 512):
            log(f"config 5: hybrid layer (8 matmuls, 269 MB of weights) M={m}")
            r = layer_case(hl, torch, m)
            extra[f"hybrid_layer_m{m}"] = {"us_per_layer": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                                           "TFLOP/s": round(r["tflops"], 2)}
        for m in (1, 4, 512):
            if m != 512:
                log(f"config 5 with q|k row-fused (one GEMV for both) M={m}")
                r = layer_case(hl, torch, m, fuse_qk=True)
                extra[f"hybrid_layer_m{m}_qk_fused"] = {"us_per_layer": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                                                        "TFLOP/s": round(r["tflops"], 2)}
            log(f"config 5 with q, k, v in one grouped launch M={m}")
            r = layer_case(hl, torch, m, group_qkv=True)
            extra[f"hybrid_layer_m{m}_qkv_group"] = {"us_per_layer": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                                                     "TFLOP/s": round(r["tflops"], 2)}
        for m in (1, 2, 4, 8):
            # what the Backend adapter runs for decode and MTP verify (GemvArgs::allow_gemm off),
            # every row bitwise its own n_vec == 1 row: the slab GEMV (MiOptions default,
            # variant 2), or the exact GEMM with its K split fixed by the shape
            # (BatchInvariantKernel::Exact, variant 9)
            for fam, v in (("gemv", 2), ("exact", 9)):
                log(f"decode / MTP verify, batch-invariant family {fam} (variant {v}) M={m}")
                extra[f"q4k_gemv_17408x5120_m{m}_allow_gemm_off_{fam}"] = gemv_fig(
                    gemv_case(hl, torch, Q4_K, 17408, 5120, m, 2, variant=v))
                extra[f"q6k_gemv_5120x17408_m{m}_allow_gemm_off_{fam}"] = gemv_fig(
                    gemv_case(hl, torch, Q6_K, 5120, 17408, m, 3, variant=v))
                r = gemm_case(hl, torch, Q4_K, 17408, 5120, m, 4, variant=v)
                extra[f"q4k_gate_up_swiglu_m{m}_allow_gemm_off_{fam}"] = {
                    **gemm_fig(r), "weights_GB/s": round(2 * 17408 * 2880 / (r["ms"] * 1e-3) / 1e9, 1)}
        for m in (2, 4, 8, 64, 512):
            log(f"config 4: Q4_K gate/up + SwiGLU M={m}")
            r = gemm_case(hl, torch, Q4_K, 17408, 5120, m, 4)
            extra[f"q4k_gate_up_swiglu_m{m}"] = {**gemm_fig(r), "weights_GB/s": round(2 * 17408 * 2880 / (r["ms"] * 1e-3) / 1e9, 1),
                                                 "samples_us": r["samples_us"]}
    log("cpu baseline (all host threads, then one)")
    cpu = cpu_baseline(Q4_K, head["wq"], 17408, 5120, head["x"], args.cpu_seconds)
    one = cpu_baseline(Q4_K, head["wq"], 17408, 5120, head["x"], min(5.0, args.cpu_seconds), threads=1)
    cpu["one_thread"] = {k: one[k] for k in ("value", "unit", "cores", "ms_per_call", "sample")}

    line = {
        "metric": "Q4_K GEMV GB/s at M=1 (17408x5120, BASELINE config 2)",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["exact_ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: N(0,0.02) weights quantized to Q4_K by this repo's quantizer, N(0,1) x",
        "config": {"workload": "Q4_K dequant-GEMV 17408x5120 M=1 (config 2), SLAB layout, "
                               f"{math.ceil(MALL_BYTES / (17408 * 2880)) + 1} rotating weight copies"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["traffic_bytes"] if traffic else None,
                     "algorithmic_bytes": head["bytes"], "kernel_us": round(kernel_us, 3),
                     "kernel_us_window": round(head["ms"] * 1e3, 3),
                     "kernel_us_eager_median": round(head["event_median_us"], 3),
                     "floor_us": round(floor["us"], 3), "floor_GB/s": round(floor["gbs"], 1),
                     "frac_of_floor": round(floor["us"] / kernel_us, 4),
                     "floor_note": "one read-only stream over the same 50 MB (halo_mi_stream_read, best of "
                                   f"a sweep: {floor['workgroups_per_cu']} workgroups per CU, "
                                   f"{floor['loads_in_flight']} 16 B loads in flight per thread)",
                     "traffic_source": traffic["source"] if traffic else None},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    if args.calibration_copy_mib > 0:
        a = torch.empty(args.calibration_copy_mib << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
