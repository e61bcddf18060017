"""Benchmark of the matrix-multiply hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline workload: BASELINE config 5, the largest single-GPU configuration --
the Whisper large-v3-turbo encoder linears at 1500 frames, fp32, as one
32-layer sweep with each layer's own weights (2.3 GB of weights per sweep,
nine times the 256 MB Infinity Cache).  One "step" is one sweep, on one
stream, operands resident in HBM:
    QKV      X[1500x1280] . W[1280x3840]   (the fused q, k, v projections)
    FFN-up   X[1500x1280] . W[1280x5120]
    FFN-down H[1500x5120] . W[5120x1280]
for each of 32 layers: 96 GEMMs, 1.730 TFLOP.
Inputs (host generator of tomoul_amd/synth.py, SplitMix64 -> Box-Muller):
X ~ N(0,1) seed 1001, H ~ N(0,1) seed 1002, layer l's three weights
~ N(0, 0.02) drawn in that order from one stream of seed 2002 + l.
`value` = TFLOP per sweep x K / wall time of the K timed sweeps.

The same JSON line also carries:
  batches       the K timed sweeps as 5 consecutive batches (HIP events on
                the stream the sweeps run on), each batch's TFLOP/s and
                their median;
  roofline      the GEMM kernel against the fp32 MFMA peak (157.3 TFLOP/s),
                from HIP events over the timed region on the launch stream;
  config5_q     the same sweep with Q8_0 and Q4_0 weights;
  config2       the XLM-R-large layer linears at seq 512;
  config1, qgemm, gemv, sentence_transformer   the other configs;
  host_pointer  the drop-in's host-pointer calls (PCIe transfers included);
  cpu_baseline  the reference's CPU path (the oracle's restatement of the
                ops.zig fallback and quantization.zig loops, test
                infrastructure) on a bounded sample of the same workloads.
Prints exactly one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
HBM_PEAK_GBS = 8000.0


def qgemm_peak(M: int) -> dict:
    """Roofline of a Q8_0 / Q4_0 GEMM of M rows: past the GEMV rows (M > 8)
    the bf16 matrix-core kernel (gemm_qbf.hip), which issues two bf16 MFMAs
    per product (activation hi + lo), so its MFMA work is twice the
    algorithmic flops against the dense bf16 peak; at M <= 8 the GEMV
    kernels, here priced against the fp32 peak."""
    if M > 8:
        return {"kernel": "bf16 MFMA, hi + lo activation terms", "peak": BF16_PEAK_TFLOPS, "mfma_per_flop": 2}
    return {"kernel": "fp32 MFMA", "peak": FP32_PEAK_TFLOPS, "mfma_per_flop": 1}


def qgemm_frac(M: int, tf: float) -> float:
    pk = qgemm_peak(M)
    return round(tf * pk["mfma_per_flop"] / pk["peak"], 4)

ENC_SHAPES = [  # config 5, per layer: (name, M, N, K)
    ("qkv", 1500, 3840, 1280),
    ("ffn_up", 1500, 5120, 1280),
    ("ffn_down", 1500, 1280, 5120),
]
ENC_LAYERS = 32
XLMR_SHAPES = [  # config 2: (name, M, N, K)
    ("qkv", 512, 3072, 1024),
    ("out", 512, 1024, 1024),
    ("ffn_up", 512, 4096, 1024),
    ("ffn_down", 512, 1024, 4096),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20, help="timed sweeps (one sweep = 32 layers x 3 GEMMs)")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--settle", type=float, default=1.0,
                   help="seconds of untimed replays of the captured sweep after the warm-up steps, so the "
                        "timed region runs at steady clocks")
    p.add_argument("--layers", type=int, default=ENC_LAYERS, help="layers per sweep (32 = the config)")
    p.add_argument("--gen-workers", type=int, default=min(16, os.cpu_count() or 1),
                   help="processes drawing the config-5 weights on the host (0: in this process, for "
                        "rocprofv3 runs)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true", help="only the headline workload")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the 1-thread CPU baseline sample")
    p.add_argument("--profile-step", action="store_true",
                   help="only warm up and run the timed headline sweeps (for rocprofv3 runs)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run a plain 256 MiB device copy 5 times (scale for FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--config2-only", action="store_true",
                   help="only the XLM-R layer step (config 2), for kernel traces")
    p.add_argument("--config1-only", action="store_true",
                   help="only config 1 (Whisper-tiny MLP + bias, 20 launches per replay), for kernel traces")
    p.add_argument("--qgemm-only", action="store_true",
                   help="only config 3 at M = 128 / 512 (Q8_0, bf16 matrix-core GEMM), for kernel traces")
    p.add_argument("--config5-quant-only", action="store_true",
                   help="only the config-5 sweep with Q8_0 / Q4_0 weights (bf16 matrix-core GEMM), for kernel traces")
    p.add_argument("--gemv-only", action="store_true",
                   help="only the decoder GEMVs (configs 3/4, vocabulary projections) with their read floors")
    p.add_argument("--profile-gemv", action="store_true",
                   help="only run the decoder GEMVs (configs 3/4, M = 1) 50 times per path, eagerly, for rocprofv3")
    return p.parse_args()


# ------------------------------------------------------------ host inputs
def _layer_weights(layer: int):
    """Layer `layer`'s three config-5 weights: one N(0, 0.02) stream of seed
    2002 + layer, drawn in the order QKV, FFN-up, FFN-down."""
    from tomoul_amd import synth
    out, off = [], 0
    for (_, M, N, K) in ENC_SHAPES:
        out.append(synth.normal(2002 + layer, K * N, 0.0, 0.02, offset=off).reshape(K, N))
        off += K * N
    return out


def encoder_weights(layers: int, workers: int):
    """All layers' weights, drawn before the GPU is used: by `workers` child
    processes (spawned: fresh interpreters that never touch the GPU), or in
    this process when workers == 0 -- for runs under rocprofv3, whose
    preloaded library would follow every child."""
    if workers <= 0:
        out = []
        for li in range(layers):
            out.append(_layer_weights(li))
            if li % 8 == 7:
                log(f"config-5 weights: {li + 1} of {layers} layers drawn")
        return out
    import multiprocessing as mp
    from multiprocessing import resource_tracker
    import gc
    pool = mp.get_context("spawn").Pool(max(1, min(workers, layers)))
    try:
        out = pool.map(_layer_weights, range(layers))
    finally:
        pool.close()
        pool.join()
    # The spawn context started a resource-tracker process for the pool's
    # locks.  Release the locks first (their finalizers unregister them with
    # the tracker), then stop the tracker, so that no process of this run
    # outlives it.
    del pool
    gc.collect()
    tracker = getattr(resource_tracker, "_resource_tracker", None)
    if tracker is not None and hasattr(tracker, "_stop"):
        tracker._stop()
    return out


class Timer:
    """Times a launch sequence replayed from a HIP graph, with HIP events
    recorded on the stream the graph runs on.  `launch(stream_ptr)` issues
    the kernels on the given stream; it is run once eagerly (so workspaces
    exist) and captured once."""

    def __init__(self, torch, settle_s: float = 0.2):
        self.torch = torch
        self.settle_s = settle_s

    def time_ms(self, launch, reps: int, per_replay: int = 1) -> float:
        t = self.torch
        side = t.cuda.Stream()
        with t.cuda.stream(side):
            launch(side.cuda_stream)
        t.cuda.synchronize()
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g, stream=side):
            launch(side.cuda_stream)
        t.cuda.synchronize()
        cur = t.cuda.current_stream()
        # untimed replays until the clocks have settled (they drop while the
        # host prepares the next workload)
        t_end = time.perf_counter() + self.settle_s
        g.replay()
        while time.perf_counter() < t_end:
            g.replay()
            t.cuda.synchronize()
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record(cur)
        for _ in range(reps):
            g.replay()
        e.record(cur)
        e.synchronize()
        return s.elapsed_time(e) / (reps * per_replay)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        log("bench.py: only --gpus 1 is supported (single-GPU hot-path build)")
        sys.exit(2)

    import numpy as np

    from tomoul_amd import synth

    headline = not (args.config1_only or args.config2_only or args.qgemm_only or args.profile_gemv or
                    args.calibrate_copy or args.gemv_only)
    if headline:
        t0 = time.perf_counter()
        host_w = encoder_weights(args.layers, args.gen_workers)
        host_x = synth.normal_matrix(1001, 1500, 1280)
        host_h = synth.normal_matrix(1002, 1500, 5120)
        log(f"config-5 inputs drawn on the host in {time.perf_counter() - t0:.1f} s")

    import torch

    from tomoul_amd import _abi

    _abi.init()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    timer = Timer(torch)
    log(f"device: {_abi.device_name()}")

    if args.profile_gemv:
        profile_gemv(torch, dev, sptr, _abi, synth)
        return
    if args.config1_only:
        print(json.dumps({"config1": bench_config1(torch, dev, sptr, Timer(torch), _abi, synth, np)}), flush=True)
        return
    if args.config2_only:
        print(json.dumps({"config2": bench_config2(torch, dev, sptr, timer, _abi, synth, args)}), flush=True)
        return
    if args.qgemm_only:
        print(json.dumps({"qgemm": bench_qgemm(torch, dev, sptr, timer, _abi, synth, np)}), flush=True)
        return
    if args.gemv_only:
        print(json.dumps({"gemv": bench_gemv(torch, dev, stream, sptr, timer, _abi, synth, np)}), flush=True)
        return
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 256 << 20, "copies": 5}), flush=True)
        return

    # ---------------------------------------------------------------- headline
    L = args.layers
    x = torch.from_numpy(host_x).to(dev)
    h = torch.from_numpy(host_h).to(dev)
    wdev = [[torch.from_numpy(w).to(dev) for w in layer] for layer in host_w]
    outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for (_, M, N, K) in ENC_SHAPES]
    sweep_flops = L * sum(2.0 * M * N * K for (_, M, N, K) in ENC_SHAPES)
    if args.config5_quant_only:
        print(json.dumps({"config5_q": bench_config5_quant(torch, dev, sptr, _abi, wdev, x, h, outs, L)}), flush=True)
        return

    def sweep(st=sptr, layers=None):
        for li in (range(L) if layers is None else layers):
            for i, (_, M, N, K) in enumerate(ENC_SHAPES):
                a = x if K == 1280 else h
                _abi.gemm_dev(_abi.FMT_F32, M, N, K, a.data_ptr(), wdev[li][i].data_ptr(), outs[i].data_ptr(),
                              stream=st)

    for _ in range(args.warmup):
        sweep()
    torch.cuda.synchronize()
    # correctness guard: the first and last layers against a float64 product
    # of the same device operands
    max_rel = 0.0
    for li in sorted({0, L - 1}):
        sweep(layers=[li])
        torch.cuda.synchronize()
        for i, (_, M, N, K) in enumerate(ENC_SHAPES):
            a = x if K == 1280 else h
            ref = a.double() @ wdev[li][i].double()
            max_rel = max(max_rel, float((outs[i].double() - ref).abs().max() / ref.abs().max()))
            del ref
    torch.cuda.empty_cache()
    log(f"headline max rel err vs f64: {max_rel:.3e}")

    # One sweep (96 launches, plus a split-K reduce where the plan splits K)
    # captured as one HIP graph; the timed region replays it K times in 5
    # consecutive batches with HIP events at the batch boundaries on the
    # stream the graph runs on.  MI355X lowers its clocks whenever the GPU
    # idles, so untimed replays run for --settle seconds first.
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        sweep(side.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        sweep(side.cuda_stream)
    torch.cuda.synchronize()
    extra_warmup = 0
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < args.settle or extra_warmup == 0:
        graph.replay()
        torch.cuda.synchronize()
        extra_warmup += 1
    K = max(1, args.steps)
    nb = min(5, K)
    bounds = [round(K * b / nb) for b in range(nb + 1)]
    cur = torch.cuda.current_stream(dev)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(nb + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record(cur)
    for b in range(nb):
        for _ in range(bounds[b + 1] - bounds[b]):
            graph.replay()
        evs[b + 1].record(cur)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_ms = evs[0].elapsed_time(evs[-1])
    batch = []
    for b in range(nb):
        ms_b = evs[b].elapsed_time(evs[b + 1])
        n_b = bounds[b + 1] - bounds[b]
        batch.append({"sweeps": n_b, "ms": round(ms_b, 4), "TFLOP/s": round(sweep_flops * n_b / ms_b / 1e9, 2)})
    med = sorted(bb["TFLOP/s"] for bb in batch)[nb // 2]
    ms_per_step = wall_ms / K
    value = sweep_flops / (ms_per_step * 1e-3) / 1e12
    log(f"headline: {ms_per_step:.3f} ms/sweep wall, {ev_ms / K:.3f} ms/sweep events, {value:.2f} TFLOP/s, "
        f"batches {[bb['TFLOP/s'] for bb in batch]}")
    if args.profile_step:
        print(json.dumps({"profile_step": True, "ms_per_step": ms_per_step, "tflops": value}), flush=True)
        return

    # Per-shape launch durations: the 32 layers' launches of one shape in one
    # graph (each layer its own weights, as in the sweep), 5 replays.
    per_shape = {}
    for i, (name, M, N, K_) in enumerate(ENC_SHAPES):
        a = x if K_ == 1280 else h

        def one_shape(st, i=i, a=a, M=M, N=N, K_=K_):
            for li in range(L):
                _abi.gemm_dev(_abi.FMT_F32, M, N, K_, a.data_ptr(), wdev[li][i].data_ptr(), outs[i].data_ptr(),
                              stream=st)

        ms = timer.time_ms(one_shape, 5, per_replay=L)
        per_shape[name] = {"M": M, "N": N, "K": K_, "us": round(ms * 1e3, 2),
                           "tflops": round(2.0 * M * N * K_ / ms / 1e9, 2)}
    achieved = sweep_flops / (ev_ms / K) / 1e9
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "traffic": traffic_per_sweep(),
                "algorithmic_bytes": int(L * sum(4 * (M * K_ + K_ * N + M * N) for (_, M, N, K_) in ENC_SHAPES)),
                "kernel": "gemm_dma_kernel<f32 B> (128x64 tiles, 8 waves, BK 32, three LDS stages; FFN-down K "
                          "split 2 + splitk_reduce_kernel), v_mfma_f32_16x16x4_f32",
                "per_unit": "2*M*N*K flop per GEMM launch; 96 launches per sweep",
                "per_shape": per_shape}
    log(f"roofline: {json.dumps(roofline)}")

    result = {
        "metric": "GEMM TFLOP/s + quant GEMV HBM GB/s (as % of MI355X peak), 1 GPU",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "extra_warmup_steps": extra_warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64/Box-Muller: X~N(0,1) seed 1001, H~N(0,1) seed 1002, "
                "W~N(0,0.02) seed 2002+layer)",
        "config": {"workload": f"config 5: Whisper large-v3-turbo encoder linears, fp32, {L}-layer sweep "
                               f"(1500x1280.1280x3840, 1500x1280.1280x5120, 1500x5120.5120x1280 per layer, "
                               f"own weights per layer)",
                   "parallelism": "single GPU"},
        "max_rel_err_vs_f64": max_rel,
        "batches": {"n": nb, "per_batch": batch, "median_TFLOP/s": med},
        "roofline": roofline,
    }

    if not args.no_extras:
        result["config5_q"] = bench_config5_quant(torch, dev, sptr, _abi, wdev, x, h, outs, L)
    del wdev
    torch.cuda.empty_cache()
    if not args.no_extras:
        result["config2"] = bench_config2(torch, dev, sptr, timer, _abi, synth, args)
        result["gemv"] = bench_gemv(torch, dev, stream, sptr, timer, _abi, synth, np)
        result["qgemm"] = bench_qgemm(torch, dev, sptr, timer, _abi, synth, np)
        result["config1"] = bench_config1(torch, dev, sptr, timer, _abi, synth, np)
        result["sentence_transformer"] = bench_sentence_transformer(torch, dev, sptr, timer, _abi, synth)
        result["host_pointer"] = bench_host_pointer(_abi, synth, np)

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, host_w, host_x, host_h,
                                              quantized=not args.no_extras)
        if not args.no_extras:
            attach_cpu_quantized(result)

    print(json.dumps(result), flush=True)


def traffic_per_sweep():
    """HBM bytes per headline sweep from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy kernel),
    or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemm_whisper_encoder_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_sweep")
    except (OSError, ValueError):
        return None


def bench_config5_quant(torch, dev, sptr, _abi, wdev, x, h, outs, layers):
    """Config 5 with Q8_0 and Q4_0 weights: the headline's fp32 weights
    quantized on the device by the reference quantizer (per tensor), then
    the same sweep (graph of 96 launches, replays timed with HIP events)."""
    res = {}
    flops = layers * sum(2.0 * M * N * K for (_, M, N, K) in ENC_SHAPES)
    for fmt, name in ((_abi.FMT_Q8_0, "q8_0"), (_abi.FMT_Q4_0, "q4_0")):
        rows, keep = [], []
        for li in range(layers):
            row = []
            for i, (_, M, N, K) in enumerate(ENC_SHAPES):
                nbytes = _abi.weight_bytes(fmt, K, N)
                q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
                sc = torch.empty(1, dtype=torch.float32, device=dev)
                _abi.quantize_dev(fmt, K * N, wdev[li][i].data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
                keep.append((q, sc))
                row.append((q.data_ptr(), sc))
            rows.append(row)
        torch.cuda.synchronize()
        rows = [[(p, float(s.item())) for (p, s) in row] for row in rows]

        def sweep(st, rows=rows, fmt=fmt):
            for row in rows:
                for i, (_, M, N, K) in enumerate(ENC_SHAPES):
                    a = x if K == 1280 else h
                    p, sc = row[i]
                    _abi.gemm_dev(fmt, M, N, K, a.data_ptr(), p, outs[i].data_ptr(), scale=sc, stream=st)

        ms = Timer(torch, settle_s=0.5).time_ms(sweep, 5)
        tf = flops / (ms * 1e-3) / 1e12
        wbytes = layers * sum(_abi.weight_bytes(fmt, K, N) for (_, M, N, K) in ENC_SHAPES)
        res[name] = {"ms_per_sweep": round(ms, 3), "TFLOP/s": round(tf, 2), "frac": qgemm_frac(1500, tf),
                     "frac_of_fp32_peak": round(tf / FP32_PEAK_TFLOPS, 4), "weight_bytes": wbytes,
                     **qgemm_peak(1500)}
        log(f"config5 {name}: {layers} layers, {ms:.2f} ms/sweep, {tf:.1f} TFLOP/s")
        del keep, rows
        torch.cuda.empty_cache()
    res["flops_per_sweep"] = flops
    res["layers"] = layers
    return res


def bench_config2(torch, dev, sptr, timer, _abi, synth, args):
    """Config 2: the four XLM-R-large layer linears at seq 512 in fp32 (QKV,
    out, FFN-up, FFN-down), one step = the four back to back, K steps
    captured as one graph and replayed; plus each shape as 20 back-to-back
    launches."""
    x = torch.from_numpy(synth.normal_matrix(1001, 512, 1024)).to(dev)
    hh = torch.from_numpy(synth.normal_matrix(1001, 512, 4096)).to(dev)
    ws = [torch.from_numpy(synth.normal_matrix(2002 + i, K, N, 0.02)).to(dev)
          for i, (_, M, N, K) in enumerate(XLMR_SHAPES)]
    outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for (_, M, N, K) in XLMR_SHAPES]
    ins = [x, x, x, hh]
    step_flops = sum(2.0 * M * N * K for (_, M, N, K) in XLMR_SHAPES)
    launches = []
    for i, (name, M, N, K) in enumerate(XLMR_SHAPES):
        a_p, b_p, c_p = ins[i].data_ptr(), ws[i].data_ptr(), outs[i].data_ptr()
        launches.append((name, M, N, K, lambda st, M=M, N=N, K=K, a_p=a_p, b_p=b_p, c_p=c_p:
                         _abi.gemm_dev(_abi.FMT_F32, M, N, K, a_p, b_p, c_p, stream=st)))
    steps = 200
    ms = timer.time_ms(lambda st: [fn(st) for _ in range(steps) for (_, _, _, _, fn) in launches], 3,
                       per_replay=steps)
    max_rel = 0.0
    for i, (name, M, N, K) in enumerate(XLMR_SHAPES):
        ref = ins[i].double() @ ws[i].double()
        max_rel = max(max_rel, float((outs[i].double() - ref).abs().max() / ref.abs().max()))
    per_shape = {}
    for (name, M, N, K, fn) in launches:
        ms_s = timer.time_ms(lambda st, fn=fn: [fn(st) for _ in range(20)], 5, per_replay=20)
        per_shape[name] = {"M": M, "N": N, "K": K, "us": round(ms_s * 1e3, 2),
                           "tflops": round(2.0 * M * N * K / ms_s / 1e9, 2)}
    tf = step_flops / ms / 1e9
    log(f"config2 (XLM-R layer, seq 512): {ms * 1e3:.1f} us/step, {tf:.2f} TFLOP/s, max rel err {max_rel:.2e}")
    return {"us_per_step": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": round(tf / FP32_PEAK_TFLOPS, 4),
            "max_rel_err_vs_f64": max_rel, "steps_per_graph": steps, "per_shape": per_shape,
            "per_shape_note": "each shape timed as 20 back-to-back launches (L2 warm)"}


def bench_host_pointer(_abi, synth, np):
    """The drop-in as the Zig shim calls it (src/core/ops.zig:266-275): host
    slices in and out, every call synchronous.  A registered weight stays
    resident (tml_hip_weight_register), so a call moves A up and C down over
    PCIe; an unregistered one uploads B too.  Per call, averaged over 10
    calls after 2 warm-up calls."""
    res = {}

    def timed(fn, n=10):
        for _ in range(2):
            fn()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return (time.perf_counter() - t0) / n * 1e3

    # config 2 step through tml_hip_sgemm (registered weights)
    xs = synth.normal_matrix(1001, 512, 1024)
    hs = synth.normal_matrix(1001, 512, 4096)
    wts = [synth.normal_matrix(2002 + i, K, N, 0.02) for i, (_, M, N, K) in enumerate(XLMR_SHAPES)]
    cs = [np.zeros((M, N), np.float32) for (_, M, N, K) in XLMR_SHAPES]
    ins = [xs, xs, xs, hs]
    step_flops = sum(2.0 * M * N * K for (_, M, N, K) in XLMR_SHAPES)

    def step():
        for i, (_, M, N, K) in enumerate(XLMR_SHAPES):
            _abi.sgemm(M, N, K, ins[i], wts[i], cs[i])

    ms_unreg = timed(step, 5)
    for w in wts:
        _abi.weight_register(w)
    try:
        ms_reg = timed(step)
    finally:
        for w in wts:
            _abi.weight_release(w)
    pcie = sum(4 * (M * K + M * N) for (_, M, N, K) in XLMR_SHAPES)
    res["config2_sgemm"] = {
        "registered": {"ms_per_step": round(ms_reg, 3), "TFLOP/s": round(step_flops / ms_reg / 1e9, 2),
                       "pcie_bytes_per_step": pcie},
        "unregistered": {"ms_per_step": round(ms_unreg, 3), "TFLOP/s": round(step_flops / ms_unreg / 1e9, 2),
                         "pcie_bytes_per_step": pcie + sum(4 * K * N for (_, M, N, K) in XLMR_SHAPES)}}
    log(f"host-pointer config2 step: {ms_reg:.2f} ms registered, {ms_unreg:.2f} ms unregistered")
    # config 1 through tml_hip_sgemm_bias (registered weight)
    a = synth.normal_matrix(1001, 1500, 384)
    w = synth.normal_matrix(2002, 384, 1536, 0.02)
    b = synth.normal(3003, 1536, 0.0, 0.02)
    c = np.zeros((1500, 1536), np.float32)
    _abi.weight_register(w)
    try:
        ms1 = timed(lambda: _abi.sgemm_bias(1500, 1536, 384, a, w, b, c))
    finally:
        _abi.weight_release(w)
    res["config1_sgemm_bias"] = {"registered": {"ms_per_call": round(ms1, 3),
                                                "TFLOP/s": round(2.0 * 1500 * 1536 * 384 / ms1 / 1e9, 2),
                                                "pcie_bytes_per_call": 4 * (1500 * 384 + 1500 * 1536 + 1536)}}
    log(f"host-pointer config1 sgemm_bias: {ms1:.3f} ms per call")
    return res


def bench_gemv(torch, dev, stream, sptr, timer, _abi, synth, np):
    """Configs 3 (Q8_0, M in {1, 8}) and 4 (Q4_0 pair, M in {1, 4, 8}), plus
    the decoder vocab projection (d=1280 x n_vocab=51866, M = 1).

    Two paths per shape: "prepared" -- the device-native K-contiguous copy
    made once per weight (tml_hip_prepare_dev), used where its kernel covers
    M -- and "kn" -- the weight in the reference's [K,N] layout, per call.
    Algorithmic bytes per launch = weight bytes + scale bytes (4, or 4*N for
    the per-column formats) + 4*M*K + 4*M*N.
    Each timed pass walks >= 1 GiB of distinct weight copies, so neither L2
    nor the 256 MB Infinity Cache serves them.  Beside each: the read floor
    for the same weight bytes over the same rotation of the same copies
    (tml_hip_stream_read_dev, 16-byte loads only, the fastest of 1, 2, 4
    and 8 loads a lane) and the GEMV's time as a fraction of it
    ("frac_of_floor" = floor / GEMV time); torch's device copy of the same
    bytes and its read-only row reduction are listed as context."""
    out = {}
    rot_bytes = 1 << 30

    def copies_for(nbytes):
        return max(2, -(-rot_bytes // nbytes))  # >= 1 GiB of distinct copies

    def run(fmt, K, N, Ms, seed, label):
        w = synth.normal_matrix(seed, K, N, 0.02)
        wt = torch.from_numpy(w).to(dev)
        cols = fmt in (_abi.FMT_Q8_0_PC, _abi.FMT_Q4_0_PC)
        wbytes = _abi.weight_bytes(fmt, K, N)
        sbytes = 4 * _abi.scale_count(fmt, K, N)
        q = torch.empty(wbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(sbytes // 4, dtype=torch.float32, device=dev)
        if cols:
            _abi.quantize_cols_dev(fmt, K, N, wt.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        else:
            _abi.quantize_dev(fmt, K * N, wt.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        scale = 1.0 if cols else float(sc.item())
        sc_ptr = sc.data_ptr() if cols else None
        ncopy = copies_for(wbytes)
        copies = q.repeat(ncopy).view(ncopy, wbytes)
        del wt
        ptrs = [copies[i].data_ptr() for i in range(ncopy)]
        handles = [_abi.prepare_ex_dev(fmt, K, N, p, scale=scale, scales_ptr=sc_ptr, stream=sptr) for p in ptrs]
        torch.cuda.synchronize()
        res = {"read_floor": stream_floor(ptrs, wbytes, label)}
        floor_us = res["read_floor"]["us"]
        for M in Ms:
            x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            alg = wbytes + sbytes + 4 * M * K + 4 * M * N
            entry = {"bytes": alg}

            def kn(st):
                for p in ptrs:
                    _abi.gemm_dev(fmt, M, N, K, x.data_ptr(), p, y.data_ptr(), scale=scale, scales_ptr=sc_ptr,
                                  stream=st)

            def prep(st):
                for h in handles:
                    _abi.gemm_prepared(h, M, x.data_ptr(), y.data_ptr(), stream=st)

            entry["floor_us"] = floor_us
            entry["torch_copy_us"] = read_floor(wbytes)
            for name, fn in (("prepared", prep), ("kn", kn)):
                ms = timer.time_ms(fn, 3, per_replay=ncopy)
                gbs = alg / (ms * 1e-3) / 1e9
                entry[name] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                               "frac_of_floor": round(floor_us / (ms * 1e3), 4)}
                log(f"gemv {label} M={M} {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s "
                    f"({floor_us / (ms * 1e3):.2f} of the read floor)")
            res[f"M{M}"] = entry
        # the decoder's growth with M: each row count's prepared time over M = 1's
        if "M1" in res:
            for key, entry in res.items():
                if key == "read_floor":
                    continue
                entry["prepared"]["x_of_M1"] = round(entry["prepared"]["us"] / res["M1"]["prepared"]["us"], 3)
        for h in handles:
            _abi.prepared_free(h)
        del copies
        torch.cuda.empty_cache()
        return res

    def run_rows_f32(N, K, Ms, seed, label, ncopy):
        # The tied vocabulary projection as the reference stores it: the f32
        # token embedding E [n_vocab, d], logits = x . E^T, with E used in
        # place as a rows-prepared weight (no per-step transpose, no copy).
        # "kn": the reference's own per-step call, ops.matmul of x by the
        # transposed embedding [K, N] (decoder.zig:936-940), through the
        # [K,N] GEMV (N = 51866 is not a whole number of lane chunks); the
        # transpose is the caller's and is not timed.
        e = torch.from_numpy(synth.normal_matrix(seed, N, K, 0.02)).to(dev)
        copies = e.reshape(1, N * K).repeat(ncopy, 1)
        copies_t = e.t().contiguous().reshape(1, K * N).repeat(ncopy, 1)
        del e
        handles = [_abi.prepare_rows_dev(_abi.FMT_F32, K, N, copies[i].data_ptr(), 4 * K, 1.0, sptr)
                   for i in range(ncopy)]
        torch.cuda.synchronize()
        res = {}
        for M in Ms:
            x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            alg = 4 * N * K + 4 * M * K + 4 * M * N

            def prep(st):
                for h in handles:
                    _abi.gemm_prepared(h, M, x.data_ptr(), y.data_ptr(), stream=st)

            def kn(st):
                for i in range(ncopy):
                    _abi.gemm_dev(_abi.FMT_F32, M, N, K, x.data_ptr(), copies_t[i].data_ptr(), y.data_ptr(),
                                  stream=st)

            res[f"M{M}"] = {"bytes": alg}
            for name, fn in (("prepared_rows", prep), ("kn", kn)):
                ms = timer.time_ms(fn, 3, per_replay=ncopy)
                gbs = alg / (ms * 1e-3) / 1e9
                res[f"M{M}"][name] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}
                log(f"gemv {label} M={M} {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
        for h in handles:
            _abi.prepared_free(h)
        del copies, copies_t
        torch.cuda.empty_cache()
        return res

    def stream_floor(ptrs, nbytes, label):
        # The read floor: one tml_hip_stream_read_dev launch per weight copy,
        # over the same rotation the GEMVs walk; the fastest of 1, 2, 4 and 8
        # 16-byte loads a lane.
        out_buf = torch.empty(nbytes // 4096 + 2, dtype=torch.float32, device=dev)
        by_u = {}
        for u in (1, 2, 4, 8):
            def fn(st, u=u):
                for p in ptrs:
                    _abi.stream_read_dev(p, nbytes, u, out_buf.data_ptr(), st)
            by_u[u] = timer.time_ms(fn, 3, per_replay=len(ptrs)) * 1e3
        best = min(by_u, key=by_u.get)
        us = by_u[best]
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"read floor {label} ({nbytes} B): {us:.2f} us ({best} loads a lane), {gbs:.0f} GB/s; "
            + ", ".join(f"{u}: {t:.2f}" for u, t in by_u.items()))
        del out_buf
        return {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                "chunks_per_lane": best, "us_by_chunks_per_lane": {str(u): round(t, 3) for u, t in by_u.items()},
                "kernel": "stream_read_kernel (tml_hip_stream_read_dev)"}

    floors = {}

    def read_floor(nbytes):
        # Floors for a launch that streams `nbytes` of weights, over the same
        # >= 1 GiB rotation of distinct buffers the GEMVs use: torch's own
        # fastest memory operation at that size, a device copy of the same
        # bytes (nbytes read and nbytes written: no slower a floor than a
        # pure read would be), and torch's read-only row reduction
        # (nbytes read, 1/256 of it written).  Returns the copy time.
        if nbytes in floors:
            return floors[nbytes]["copy_us"]
        nb4 = -(-nbytes // 1024) * 256  # floats, a multiple of 256
        ncopy = copies_for(4 * nb4)
        src = torch.ones((ncopy, nb4), dtype=torch.float32, device=dev)
        dst = torch.empty((ncopy, nb4), dtype=torch.float32, device=dev)

        def cp(st):
            for i in range(ncopy):
                dst[i].copy_(src[i])

        def rd(st):
            for i in range(ncopy):
                torch.sum(src[i].view(-1, 256), dim=1, out=dst[i, : nb4 // 256])

        ms_c = timer.time_ms(cp, 3, per_replay=ncopy)
        ms_r = timer.time_ms(rd, 3, per_replay=ncopy)
        del src, dst
        torch.cuda.empty_cache()
        floors[nbytes] = {"copy_us": round(ms_c * 1e3, 3), "row_sum_us": round(ms_r * 1e3, 3)}
        log(f"floors for {nbytes} B: torch copy {ms_c * 1e3:.2f} us, torch row sum {ms_r * 1e3:.2f} us")
        return floors[nbytes]["copy_us"]

    def copy_floor(nbytes):
        # Context for the decoder shapes: torch's own device copy moving
        # 2 * nbytes per launch (nbytes read, nbytes written), rotating over
        # >= 1 GB like the GEMVs.  A launch that moves a few MB costs this
        # much on MI355X whatever it computes.
        ncopy = copies_for(nbytes)
        src = torch.empty((ncopy, nbytes), dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)

        def fn(st):
            for i in range(ncopy):
                dst[i].copy_(src[i])

        ms = timer.time_ms(fn, 3, per_replay=ncopy)
        gbs = 2 * nbytes / (ms * 1e-3) / 1e9
        log(f"copy floor {nbytes >> 20} MiB -> {nbytes >> 20} MiB: {ms * 1e3:.2f} us, {gbs:.0f} GB/s moved")
        del src, dst
        torch.cuda.empty_cache()
        return {"bytes_moved": 2 * nbytes, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4)}

    out["torch_copy_floor"] = {"2MiB": copy_floor(2 << 20), "4MiB": copy_floor(4 << 20),
                               "32MiB": copy_floor(32 << 20)}
    out["q8_1024x4096"] = run(_abi.FMT_Q8_0, 1024, 4096, [1, 4, 8], 2002, "q8 1024x4096")
    out["q4_1280x5120"] = run(_abi.FMT_Q4_0, 1280, 5120, [1, 4, 8], 2002, "q4 1280x5120")
    out["q4_5120x1280"] = run(_abi.FMT_Q4_0, 5120, 1280, [1, 4, 8], 2003, "q4 5120x1280")
    # config 3 read as "one scale per output column" (Q8_0_PC, an extension)
    # and the same for the int4 pair's first shape (Q4_0_PC)
    out["q8pc_1024x4096"] = run(_abi.FMT_Q8_0_PC, 1024, 4096, [1, 8], 2002, "q8pc 1024x4096")
    out["q4pc_1280x5120"] = run(_abi.FMT_Q4_0_PC, 1280, 5120, [1, 4], 2002, "q4pc 1280x5120")
    out["f32_vocab_rows_51866x1280"] = run_rows_f32(51866, 1280, [1, 4], 2004, "f32 vocab rows 51866x1280",
                                                    copies_for(4 * 51866 * 1280))
    out["q8_vocab_1280x51866"] = run(_abi.FMT_Q8_0, 1280, 51866, [1], 2004, "q8 vocab 1280x51866")
    out["q4_vocab_1280x51866"] = run(_abi.FMT_Q4_0, 1280, 51866, [1], 2004, "q4 vocab 1280x51866")
    out["floors_by_weight_bytes"] = {str(k): v for k, v in floors.items()}
    return out


def bench_qgemm(torch, dev, sptr, timer, _abi, synth, np):
    """Config 3 at M in {128, 512}: Q8_0 W[1024x4096] (bf16 matrix-core GEMM).
    Each launch reads a different copy of the weight, rotating through >= 1 GiB
    of copies, so neither L2 nor the Infinity Cache holds it between launches."""
    res = {}
    K, N = 1024, 4096
    w = torch.from_numpy(synth.normal_matrix(2002, K, N, 0.02)).to(dev)
    q = torch.empty(_abi.weight_bytes(_abi.FMT_Q8_0, K, N), dtype=torch.uint8, device=dev)
    sc = torch.empty(1, dtype=torch.float32, device=dev)
    _abi.quantize_dev(_abi.FMT_Q8_0, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
    torch.cuda.synchronize()
    scale = float(sc.item())
    ncopy = -(-(1 << 30) // (K * N))
    copies = q.repeat(ncopy).view(ncopy, K * N)
    ptrs = [copies[i].data_ptr() for i in range(ncopy)]
    for M in (128, 512):
        x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)

        def fn(st, M=M, x=x, y=y):
            for p in ptrs:
                _abi.gemm_dev(_abi.FMT_Q8_0, M, N, K, x.data_ptr(), p, y.data_ptr(), scale=scale, stream=st)
        ms = timer.time_ms(fn, 3, per_replay=ncopy)
        tf = 2.0 * M * N * K / ms / 1e9
        res[f"q8_M{M}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": qgemm_frac(M, tf), **qgemm_peak(M)}
        log(f"qgemm q8 M={M}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
    del copies
    torch.cuda.empty_cache()
    return res


def bench_config1(torch, dev, sptr, timer, _abi, synth, np):
    """Config 1: Whisper-tiny MLP X[1500x384] . W[384x1536] + bias (fused)."""
    x = torch.from_numpy(synth.normal_matrix(1001, 1500, 384)).to(dev)
    w = torch.from_numpy(synth.normal_matrix(2002, 384, 1536, 0.02)).to(dev)
    b = torch.from_numpy(synth.normal(3003, 1536, 0.0, 0.02)).to(dev)
    y = torch.empty((1500, 1536), dtype=torch.float32, device=dev)
    fn = lambda st: _abi.gemm_dev(_abi.FMT_F32, 1500, 1536, 384, x.data_ptr(), w.data_ptr(),  # noqa: E731
                                  y.data_ptr(), bias_ptr=b.data_ptr(), stream=st)
    ms = timer.time_ms(lambda st: [fn(st) for _ in range(20)], 5, per_replay=20)
    tf = 2.0 * 1500 * 1536 * 384 / ms / 1e9
    log(f"config1: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
    return {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": round(tf / FP32_PEAK_TFLOPS, 4)}


def bench_sentence_transformer(torch, dev, sptr, timer, _abi, synth, tokens: int = 512, layers: int = 6):
    """The sentence-transformer encoder's linears (src/models/sentence_transformer/model.zig:40-46:
    hidden 384, intermediate 1536, 6 layers) over `tokens` tokens: per layer
    Q, K, V, O [384x384], FFN up [384x1536] and down [1536x384], each layer
    with its own weights, in fp32, F16 and Q8_K (the formats its .tl files
    carry; quantized / converted on the device by the reference's
    quantizers).  One sweep = 6 layers x 6 GEMMs, 20 sweeps per graph replay.
    "<fmt>_fused_qkv": the same sweep with each layer's Q, K and V weights
    concatenated along N at load into one [384 x 1152] weight (one GEMM
    instead of three: exact, each N-slice is its own projection; for Q8_K the
    32-element scale blocks of a 384-wide row stay whole), so 4 GEMMs a layer."""
    d, ff, M = 384, 1536, tokens
    shapes = [(d, d)] * 4 + [(d, ff), (ff, d)]
    fused_shapes = [(d, 3 * d), (d, d), (d, ff), (ff, d)]
    flops = layers * sum(2.0 * M * K * N for (K, N) in shapes)
    assert flops == layers * sum(2.0 * M * K * N for (K, N) in fused_shapes)
    x = torch.from_numpy(synth.normal_matrix(1001, M, d)).to(dev)
    h = torch.from_numpy(synth.normal_matrix(1002, M, ff)).to(dev)
    y = torch.empty((M, ff), dtype=torch.float32, device=dev)
    res = {}
    for fmt, name, lshapes in ((_abi.FMT_F32, "fp32", shapes), (_abi.FMT_F16, "f16", shapes),
                               (_abi.FMT_Q8_K, "q8_k", shapes), (_abi.FMT_F32, "fp32_fused_qkv", fused_shapes),
                               (_abi.FMT_F16, "f16_fused_qkv", fused_shapes),
                               (_abi.FMT_Q8_K, "q8_k_fused_qkv", fused_shapes)):
        keep, row = [], []
        for layer in range(layers):
            for i, (K, N) in enumerate(lshapes):
                w = torch.from_numpy(synth.normal_matrix(2002 + 8 * layer + i, K, N, 0.02)).to(dev)
                if fmt == _abi.FMT_F32:
                    keep.append(w)
                    row.append((K, N, w.data_ptr(), None))
                    continue
                b = torch.empty(_abi.weight_bytes(fmt, K, N), dtype=torch.uint8, device=dev)
                sc = torch.empty(max(_abi.scale_count(fmt, K, N), 1), dtype=torch.float32, device=dev)
                _abi.quantize_dev(fmt, K * N, w.data_ptr(), b.data_ptr(), sc.data_ptr(), sptr)
                keep += [b, sc]
                row.append((K, N, b.data_ptr(), sc.data_ptr() if fmt == _abi.FMT_Q8_K else None))
        torch.cuda.synchronize()

        def sweep(st, row=row, fmt=fmt):
            for (K, N, bp, sp_) in row:
                a = x if K == d else h
                _abi.gemm_dev(fmt, M, N, K, a.data_ptr(), bp, y.data_ptr(), scales_ptr=sp_, stream=st)

        ms = timer.time_ms(lambda st: [sweep(st) for _ in range(20)], 3, per_replay=20)
        tf = flops / ms / 1e9
        res[name] = {"us_per_sweep": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2),
                     "frac": round(tf / FP32_PEAK_TFLOPS, 4)}
        log(f"sentence-transformer {name}: {tokens} tokens x {layers} layers, {ms * 1e3:.1f} us/sweep, "
            f"{tf:.1f} TFLOP/s")
        del keep
    res["tokens"] = tokens
    res["layers"] = layers
    res["flops_per_sweep"] = flops
    return res


def profile_gemv(torch, dev, sptr, _abi, synth, launches: int = 50):
    """Decoder GEMVs for kernel traces / counters: Q8_0 1024x4096 and Q4_0
    1280x5120 and 5120x1280 at M = 1, 4 and 8, each on its prepared copy and
    in the [K,N] layout, `launches` times over 16 distinct weight copies;
    then the Q8_0 and Q4_0 vocabulary projections (1280 x 51866, M = 1) on
    3 / 4 prepared copies and on the same copies in the [K,N] layout, and the
    f32 one on the token embedding used in place (rows-prepared) and on its
    transpose in the [K,N] layout (the reference's own per-step call), 3
    copies each.  At M = 1 each layer shape also runs the read floor
    (tml_hip_stream_read_dev, two 16-byte loads a lane) over the same 16
    copies, and Q4_0 the per-lane VALU kernel (TML_GEMVX=0) that the
    staged-activation kernel replaced, for comparison.  Each batch is one
    eager launch (workspaces), then its `launches` launches captured in a HIP
    graph and replayed once, back to back as the benchmark's timings run
    them: a trace shows each batch as a run of launches + 1 dispatches whose
    first is the eager one."""
    def batch(launch):
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            launch(side.cuda_stream, 1)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            launch(side.cuda_stream, launches)
        g.replay()
        torch.cuda.synchronize()
        del g

    for fmt, K, N, M in ((_abi.FMT_Q8_0, 1024, 4096, 1), (_abi.FMT_Q8_0, 1024, 4096, 4),
                         (_abi.FMT_Q8_0, 1024, 4096, 8),
                         (_abi.FMT_Q4_0, 1280, 5120, 1), (_abi.FMT_Q4_0, 1280, 5120, 4),
                         (_abi.FMT_Q4_0, 1280, 5120, 8),
                         (_abi.FMT_Q4_0, 5120, 1280, 1), (_abi.FMT_Q4_0, 5120, 1280, 4),
                         (_abi.FMT_Q4_0, 5120, 1280, 8)):
        w = torch.from_numpy(synth.normal_matrix(2002, K, N, 0.02)).to(dev)
        nbytes = _abi.weight_bytes(fmt, K, N)
        q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(1, dtype=torch.float32, device=dev)
        _abi.quantize_dev(fmt, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        scale = float(sc.item())
        copies = q.repeat(16).view(16, nbytes)
        hs = [_abi.prepare_dev(fmt, K, N, copies[i].data_ptr(), scale, sptr) for i in range(16)]
        x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        batch(lambda st, n: [_abi.gemm_prepared(hs[i % 16], M, x.data_ptr(), y.data_ptr(), stream=st)
                             for i in range(n)])
        batch(lambda st, n: [_abi.gemm_dev(fmt, M, N, K, x.data_ptr(), copies[i % 16].data_ptr(), y.data_ptr(),
                                           scale=scale, stream=st) for i in range(n)])
        if M == 1:
            floor_out = torch.empty(nbytes // 4096 + 2, dtype=torch.float32, device=dev)
            batch(lambda st, n: [_abi.stream_read_dev(copies[i % 16].data_ptr(), nbytes, 2, floor_out.data_ptr(), st)
                                 for i in range(n)])
            if fmt == _abi.FMT_Q4_0:
                os.environ["TML_GEMVX"] = "0"
                try:
                    batch(lambda st, n: [_abi.gemm_prepared(hs[i % 16], M, x.data_ptr(), y.data_ptr(), stream=st)
                                         for i in range(n)])
                finally:
                    os.environ.pop("TML_GEMVX", None)
        torch.cuda.synchronize()
        for h_ in hs:
            _abi.prepared_free(h_)
        log(f"profile-gemv: fmt {fmt} {K}x{N} M={M}: {launches} prepared + {launches} [K,N] launches")
    # the vocabulary projection (1280 x 51866) at M = 1 on prepared copies
    for fmt, ncopy in ((_abi.FMT_Q8_0, 3), (_abi.FMT_Q4_0, 4)):
        K, N = 1280, 51866
        w = torch.from_numpy(synth.normal_matrix(2004, K, N, 0.02)).to(dev)
        nbytes = _abi.weight_bytes(fmt, K, N)
        q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(1, dtype=torch.float32, device=dev)
        _abi.quantize_dev(fmt, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        copies = q.repeat(ncopy).view(ncopy, nbytes)
        del w
        scale = float(sc.item())
        hs = [_abi.prepare_dev(fmt, K, N, copies[i].data_ptr(), scale, sptr) for i in range(ncopy)]
        x = torch.from_numpy(synth.normal_matrix(1001, 1, K)).to(dev)
        y = torch.empty((1, N), dtype=torch.float32, device=dev)
        batch(lambda st, n: [_abi.gemm_prepared(hs[i % ncopy], 1, x.data_ptr(), y.data_ptr(), stream=st)
                             for i in range(n)])
        batch(lambda st, n: [_abi.gemm_dev(fmt, 1, N, K, x.data_ptr(), copies[i % ncopy].data_ptr(), y.data_ptr(),
                                           scale=scale, stream=st) for i in range(n)])
        torch.cuda.synchronize()
        for h_ in hs:
            _abi.prepared_free(h_)
        del copies
        torch.cuda.empty_cache()
        log(f"profile-gemv: fmt {fmt} vocab {K}x{N}: {launches} prepared + {launches} [K,N] launches")
    # the f32 token embedding [51866 x 1280] used in place (rows-prepared), M = 1
    K, N, ncopy = 1280, 51866, 3
    e = torch.from_numpy(synth.normal_matrix(2004, N, K, 0.02)).to(dev)
    copies = e.reshape(1, N * K).repeat(ncopy, 1)
    copies_t = e.t().contiguous().reshape(1, K * N).repeat(ncopy, 1)
    del e
    hs = [_abi.prepare_rows_dev(_abi.FMT_F32, K, N, copies[i].data_ptr(), 4 * K, 1.0, sptr) for i in range(ncopy)]
    x = torch.from_numpy(synth.normal_matrix(1001, 1, K)).to(dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    batch(lambda st, n: [_abi.gemm_prepared(hs[i % ncopy], 1, x.data_ptr(), y.data_ptr(), stream=st)
                         for i in range(n)])
    batch(lambda st, n: [_abi.gemm_dev(_abi.FMT_F32, 1, N, K, x.data_ptr(), copies_t[i % ncopy].data_ptr(),
                                       y.data_ptr(), stream=st) for i in range(n)])
    torch.cuda.synchronize()
    for h_ in hs:
        _abi.prepared_free(h_)
    del copies, copies_t
    torch.cuda.empty_cache()
    log(f"profile-gemv: f32 embedding {N}x{K}: {launches} launches in place + {launches} on its transpose")
    print(json.dumps({"profile_gemv": True}), flush=True)


def host_nproc() -> int:
    """CPUs this process may run on (what `nproc` prints)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def host_cpu_model() -> str:
    """The host CPU's model string (`model name` of /proc/cpuinfo, as lscpu shows it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(budget_s: float, host_w, host_x, host_h, quantized: bool = True):
    """The reference's CPU path on a bounded sample of the headline workload:
    the oracle's restatement of the register-blocked ops.zig:277-414 fallback
    (the reference's fp32 path without zblas), single-threaded as in the
    reference, over whole config-5 layers (three GEMMs, 54 GFLOP each) until
    about `budget_s` seconds are spent; then the same loops row-parallel with
    the reference's matmulParallel cap of 4 threads (src/core/context.zig:285)
    and with every host thread.  With `quantized`, also the reference's
    weight-only loops (quantization.zig:240-311 Q8_0, :829-957 Q4_0) at the
    config-3 and config-4 shapes."""
    from oracle import oracle as orc

    orc.lib()
    layer_flops = sum(2.0 * M * N * K for (_, M, N, K) in ENC_SHAPES)

    def run_layer(li, nt):
        for i, (_, M, N, K) in enumerate(ENC_SHAPES):
            a = host_x if K == 1280 else host_h
            if nt == 1:
                orc.matmul(a, host_w[li][i])
            else:
                orc.matmul_mt(a, host_w[li][i], nt)

    def sample(nt, budget):
        n, t = 0, 0.0
        while (t < budget or n == 0) and n < len(host_w):
            t0 = time.perf_counter()
            run_layer(n, nt)
            t += time.perf_counter() - t0
            n += 1
        return n, t

    n1, t1 = sample(1, budget_s)
    tf = layer_flops * n1 / t1 / 1e12
    log(f"cpu baseline: {n1} config-5 layers in {t1:.1f} s, {tf * 1e3:.2f} GFLOP/s (1 thread)")
    threaded = {}
    for nt in sorted({4, max(1, orc.max_threads())}):
        n, t = sample(nt, budget_s / 4)
        threaded[f"{nt}_threads"] = {"value": round(layer_flops * n / t / 1e12, 6), "layers": n,
                                     "seconds": round(t, 2)}
        log(f"cpu baseline, {nt} threads: {n} layers in {t:.1f} s, {layer_flops * n / t / 1e9:.2f} GFLOP/s")
    out = {"value": round(tf, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "sample": f"{n1} of the {len(host_w)} config-5 layers (3 GEMMs, {layer_flops / 1e9:.1f} GFLOP each, the "
                     f"headline's own inputs) with the oracle's restatement of the ops.zig:277-414 fallback, "
                     f"1 thread, -O3 AVX2, {t1:.1f} s; zblas (the reference default) is not vendored and "
                     f"cannot be timed, OpenBLAS is not installed",
           "host_cpus": os.cpu_count(), "nproc": host_nproc(), "cpu_model": host_cpu_model(),
           "threaded": threaded}
    if quantized:
        out["quantized"] = cpu_quantized(orc)
    return out


def cpu_quantized(orc):
    """The reference's weight-only loops at configs 3 and 4, on the oracle's
    restatement (i, k, j order, f32(q) * scale per element): Q8_0 W[1024x4096]
    at M in {1, 8, 128, 512}; Q4_0 W[1280x5120] and W[5120x1280] at M in
    {1, 4, 8}.  1 thread (the reference's Q4_0 loop is always
    single-threaded) and 4 threads (rows split; the reference's cap).  Each
    timed for at least 0.2 s."""
    from tomoul_amd import synth

    def tm(fn):
        n, t = 0, 0.0
        while t < 0.2:
            t0 = time.perf_counter()
            fn()
            t += time.perf_counter() - t0
            n += 1
        return round(t / n * 1e6, 1)

    res = {}
    w = synth.normal_matrix(2002, 1024, 4096, 0.02)
    q, s = orc.quantize_q8(w)
    q = q.reshape(1024, 4096)
    for M in (1, 8, 128, 512):
        a = synth.normal_matrix(1001, M, 1024)
        res[f"q8_1024x4096_M{M}"] = {"1_thread_us": tm(lambda: orc.matmul_q8(a, q, s)),
                                     "4_threads_us": tm(lambda: orc.matmul_q8_mt(a, q, s, 4))}
    for (K, N, seed) in ((1280, 5120, 2002), (5120, 1280, 2003)):
        w = synth.normal_matrix(seed, K, N, 0.02)
        p, s4 = orc.quantize_q4(w)
        for M in (1, 4, 8):
            a = synth.normal_matrix(1001, M, K)
            res[f"q4_{K}x{N}_M{M}"] = {"1_thread_us": tm(lambda: orc.matmul_q4(a, p, K, N, s4)),
                                       "4_threads_us": tm(lambda: orc.matmul_q4_mt(a, p, K, N, s4, 4))}
    for k, v in res.items():
        log(f"cpu baseline {k}: {v['1_thread_us']:.0f} us (1 thread), {v['4_threads_us']:.0f} us (4 threads)")
    return res


def attach_cpu_quantized(result):
    """Puts each quantized CPU figure beside the GPU entry of the same shape."""
    cq = result.get("cpu_baseline", {}).get("quantized", {})
    for key, v in cq.items():
        name, m = key.rsplit("_M", 1)
        M = int(m)
        if name.startswith("q8_") and M > 8:
            e = result.get("qgemm", {}).get(f"q8_M{M}")
            gpu_us = e and e.get("us")
        else:
            e = result.get("gemv", {}).get(name, {}).get(f"M{M}")
            gpu_us = e and e.get("prepared", {}).get("us")
        if e is not None:
            e["cpu"] = dict(v)
            if gpu_us:
                e["cpu"]["gpu_speedup_vs_1_thread"] = round(v["1_thread_us"] / gpu_us, 1)


if __name__ == "__main__":
    main()
