"""Benchmark of the matrix-multiply hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (XLM-RoBERTa-large layer at seq=512, fp32):
one "step" is the four linear layers of one encoder layer, back to back on
one stream, operands resident in HBM:
    QKV      X[512x1024] . W[1024x3072]
    out      X[512x1024] . W[1024x1024]
    FFN-up   X[512x1024] . W[1024x4096]
    FFN-down H[512x4096] . W[4096x1024]
Inputs: SplitMix64/Box-Muller, X,H ~ N(0,1) (seed 1001), W ~ N(0, 0.02)
(seed 2002 + index).  `value` = 2*M*N*K summed over the step / step time.

The same JSON line also carries:
  roofline      the GEMM kernel against the fp32 MFMA peak (157.3 TFLOP/s),
                from HIP events around each launch on the launch stream;
  gemv          quantized decoder GEMVs (configs 3 and 4 at M <= 8) in GB/s
                against 8 TB/s, rotating over >= 1 GB of distinct weight
                copies so neither L2 nor the 256 MB Infinity Cache serves them;
  qgemm, config1  the other configs' large-M products;
  cpu_baseline  the reference's CPU path (the oracle's restatement of the
                ops.zig fallback, test infrastructure) on the same workload.
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
HBM_PEAK_GBS = 8000.0

XLMR_SHAPES = [  # (name, M, N, K)
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
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--settle", type=float, default=1.0,
                   help="seconds of untimed replays of the captured steps after the warm-up steps, so the "
                        "timed region runs at steady clocks")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true", help="only the headline workload")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    p.add_argument("--profile-step", action="store_true",
                   help="only warm up and run the timed headline steps (for rocprofv3 runs)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run a plain 256 MiB device copy 5 times (scale for FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--config5-only", action="store_true",
                   help="only the config-5 sweep (Whisper encoder linears), for kernel traces and counters")
    p.add_argument("--config5-layers", type=int, default=32, help="layers of the config-5 sweep")
    p.add_argument("--config1-only", action="store_true",
                   help="only config 1 (Whisper-tiny MLP + bias, 20 launches per replay), for kernel traces")
    p.add_argument("--profile-gemv", action="store_true",
                   help="only run the decoder GEMVs (configs 3/4, M = 1) 50 times per path, eagerly, for rocprofv3")
    return p.parse_args()


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
    import torch

    from tomoul_amd import _abi, synth

    _abi.init()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    timer = Timer(torch)
    log(f"device: {_abi.device_name()}")

    def to_dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    # ---------------------------------------------------------------- headline
    x = to_dev(synth.normal_matrix(1001, 512, 1024))
    h = to_dev(synth.normal_matrix(1001, 512, 4096))
    ws = [to_dev(synth.normal_matrix(2002 + i, K, N, 0.02)) for i, (_, M, N, K) in enumerate(XLMR_SHAPES)]
    outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for (_, M, N, K) in XLMR_SHAPES]
    ins = [x, x, x, h]
    launches = []
    for i, (name, M, N, K) in enumerate(XLMR_SHAPES):
        a_p, b_p, c_p = ins[i].data_ptr(), ws[i].data_ptr(), outs[i].data_ptr()
        launches.append((name, M, N, K,
                         lambda st, M=M, N=N, K=K, a_p=a_p, b_p=b_p, c_p=c_p:
                         _abi.gemm_dev(_abi.FMT_F32, M, N, K, a_p, b_p, c_p, stream=st)))
    step_flops = sum(2.0 * M * N * K for (_, M, N, K) in XLMR_SHAPES)

    def step(st=sptr):
        for (_, _, _, _, fn) in launches:
            fn(st)

    if args.profile_gemv:
        profile_gemv(torch, dev, sptr, _abi, synth)
        return

    if args.config1_only:
        print(json.dumps({"config1": bench_config1(torch, dev, sptr, Timer(torch), _abi, synth, np)}), flush=True)
        return

    if args.config5_only:
        print(json.dumps({"config5": bench_config5(torch, dev, sptr, _abi, layers=args.config5_layers)}), flush=True)
        return

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 256 << 20, "copies": 5}), flush=True)
        return

    # The K timed steps are captured as one HIP graph (4 GEMM launches per
    # step, plus a split-K reduce where the plan splits K) and replayed once,
    # so the steps run back to back as a model's layers would; replaying a
    # one-step graph K times would add a graph launch (several us) per step.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        step(side.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(args.steps):
            step(side.cuda_stream)
    torch.cuda.synchronize()
    graph.replay()  # warm replay (first replay uploads the graph)
    torch.cuda.synchronize()
    # correctness guard against a float64 torch product on the GPU
    max_rel = 0.0
    for i, (name, M, N, K) in enumerate(XLMR_SHAPES):
        ref = (ins[i].double() @ ws[i].double())
        max_rel = max(max_rel, float((outs[i].double() - ref).abs().max() / ref.abs().max()))
    log(f"headline max rel err vs f64: {max_rel:.3e}")

    # Settle: MI355X raises its clocks over the first stretch of sustained
    # load and lowers them again when the GPU idles (the correctness guard
    # above idles it for a few hundred ms); a timed region that starts cold
    # measures that ramp (140-145 us per step against 131 us at steady
    # clocks), not the kernels.  Untimed replays of the same K-step graph run
    # until --settle seconds have passed, immediately before the timed
    # replay; their count is reported as extra_warmup_steps.
    extra_warmup = args.steps
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < args.settle:
        graph.replay()
        torch.cuda.synchronize()
        extra_warmup += args.steps
    cur = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(cur)
    graph.replay()
    ev1.record(cur)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall_ms / args.steps
    value = step_flops / (ms_per_step * 1e-3) / 1e12
    log(f"headline: {ms_per_step * 1e3:.1f} us/step wall, {ev_ms / args.steps * 1e3:.1f} us/step events, "
        f"{value:.2f} TFLOP/s")
    if args.profile_step:
        print(json.dumps({"profile_step": True, "ms_per_step": ms_per_step, "tflops": value}), flush=True)
        return

    # Per-launch durations of the GEMM kernels: 20 back-to-back launches of
    # each shape in one graph, HIP events around 5 replays on the stream the
    # graph runs on.
    per_shape = {}
    tot_fl, tot_ms = 0.0, 0.0
    for (name, M, N, K, fn) in launches:
        ms = timer.time_ms(lambda st, fn=fn: [fn(st) for _ in range(20)], 5, per_replay=20)
        fl = 2.0 * M * N * K
        per_shape[name] = {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2), "tflops": round(fl / ms / 1e9, 2)}
        tot_fl += fl
        tot_ms += ms
    # achieved: the step's algorithmic flops over its HIP-event duration in
    # the timed region (every GEMM launch of the step, split-K reduces
    # included; the GEMMs start with a cold L2, unlike the per-shape repeats).
    achieved = step_flops / (ev_ms / args.steps) / 1e9
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "traffic": traffic_per_step(),
                "algorithmic_bytes": int(sum(4 * (M * K + K * N + M * N) for (_, M, N, K) in XLMR_SHAPES)),
                "kernel": "gemm_dma_kernel<f32 B> (32x64 tiles; BK 32 for QKV and FFN-up, BK 64 with two wave "
                          "groups along K for out and FFN-down), v_mfma_f32_16x16x4_f32",
                "per_shape": per_shape, "per_shape_sum_tflops": round(tot_fl / tot_ms / 1e9, 2),
                "per_shape_note": "each shape timed as 20 back-to-back launches (L2 warm)"}
    log(f"roofline: {json.dumps(roofline)}")

    result = {
        "metric": "GEMM TFLOP/s + quant GEMV HBM GB/s (as % of MI355X peak), 1 GPU",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "extra_warmup_steps": extra_warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64/Box-Muller, X~N(0,1), W~N(0,0.02))",
        "config": {"workload": "XLM-R-large layer linears, seq=512, fp32: 512x1024.1024x3072, "
                               "512x1024.1024x1024, 512x1024.1024x4096, 512x4096.4096x1024",
                   "parallelism": "single GPU"},
        "max_rel_err_vs_f64": max_rel,
        "roofline": roofline,
    }

    if not args.no_extras:
        result["gemv"] = bench_gemv(torch, dev, stream, sptr, timer, _abi, synth, np)
        result["qgemm"] = bench_qgemm(torch, dev, sptr, timer, _abi, synth, np)
        result["config1"] = bench_config1(torch, dev, sptr, timer, _abi, synth, np)
        result["config5"] = bench_config5(torch, dev, sptr, _abi, layers=args.config5_layers)
        result["sentence_transformer"] = bench_sentence_transformer(torch, dev, sptr, timer, _abi, synth)

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)

    print(json.dumps(result), flush=True)


def traffic_per_step():
    """HBM bytes per headline step from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy kernel),
    or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemm_xlmr_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_step")
    except (OSError, ValueError):
        return None


def bench_gemv(torch, dev, stream, sptr, timer, _abi, synth, np):
    """Configs 3 (Q8_0, M in {1, 8}) and 4 (Q4_0 pair, M in {1, 4, 8}), plus
    the decoder vocab projection (d=1280 x n_vocab=51866, M = 1).

    Two paths per shape: "prepared" -- the device-native K-contiguous copy
    made once per weight (tml_hip_prepare_dev), used where its kernel covers
    M -- and "kn" -- the weight in the reference's [K,N] layout, per call.
    Algorithmic bytes per launch = weight bytes + scale bytes (4, or 4*N for
    the per-column formats) + 4*M*K + 4*M*N.
    Each timed pass walks >= 1 GB of distinct weight copies, so neither L2
    nor the 256 MB Infinity Cache serves them."""
    out = {}
    rot_bytes = 1 << 30

    def run(fmt, K, N, Ms, seed, label, max_copies=256):
        w = synth.normal_matrix(seed, K, N, 0.02)
        wt = torch.from_numpy(w).to(dev)
        cols = fmt in (_abi.FMT_Q8_0_PC, _abi.FMT_Q4_0_PC)
        wbytes = K * N if fmt in (_abi.FMT_Q8_0, _abi.FMT_Q8_0_PC) else (K * N + 1) // 2
        sbytes = 4 * N if cols else 4
        q = torch.empty(wbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(sbytes // 4, dtype=torch.float32, device=dev)
        if cols:
            _abi.quantize_cols_dev(fmt, K, N, wt.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        else:
            _abi.quantize_dev(fmt, K * N, wt.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        scale = 1.0 if cols else float(sc.item())
        sc_ptr = sc.data_ptr() if cols else None
        ncopy = min(max_copies, max(2, rot_bytes // wbytes))
        copies = q.repeat(ncopy).view(ncopy, wbytes)
        del wt
        ptrs = [copies[i].data_ptr() for i in range(ncopy)]
        handles = [_abi.prepare_ex_dev(fmt, K, N, p, scale=scale, scales_ptr=sc_ptr, stream=sptr) for p in ptrs]
        torch.cuda.synchronize()
        res = {}
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

            for name, fn in (("prepared", prep), ("kn", kn)):
                ms = timer.time_ms(fn, 3, per_replay=ncopy)
                gbs = alg / (ms * 1e-3) / 1e9
                entry[name] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
                log(f"gemv {label} M={M} {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
            res[f"M{M}"] = entry
        for h in handles:
            _abi.prepared_free(h)
        del copies
        torch.cuda.empty_cache()
        return res

    def run_rows_f32(N, K, Ms, seed, label, ncopy):
        # The tied vocabulary projection as the reference stores it: the f32
        # token embedding E [n_vocab, d], logits = x . E^T, with E used in
        # place as a rows-prepared weight (no per-step transpose, no copy).
        e = torch.from_numpy(synth.normal_matrix(seed, N, K, 0.02)).to(dev)
        copies = e.reshape(1, N * K).repeat(ncopy, 1)
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

            ms = timer.time_ms(prep, 3, per_replay=ncopy)
            gbs = alg / (ms * 1e-3) / 1e9
            res[f"M{M}"] = {"bytes": alg, "prepared_rows": {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                                             "frac": round(gbs / HBM_PEAK_GBS, 4)}}
            log(f"gemv {label} M={M} rows in place: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
        for h in handles:
            _abi.prepared_free(h)
        del copies
        torch.cuda.empty_cache()
        return res

    def copy_floor(nbytes):
        # Context for the decoder shapes: torch's own device copy moving
        # 2 * nbytes per launch (nbytes read, nbytes written), rotating over
        # >= 1 GB like the GEMVs.  A launch that moves a few MB costs this
        # much on MI355X whatever it computes.
        ncopy = min(256, max(2, rot_bytes // nbytes))
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
    out["q8_1024x4096"] = run(_abi.FMT_Q8_0, 1024, 4096, [1, 8], 2002, "q8 1024x4096")
    out["q4_1280x5120"] = run(_abi.FMT_Q4_0, 1280, 5120, [1, 4, 8], 2002, "q4 1280x5120")
    out["q4_5120x1280"] = run(_abi.FMT_Q4_0, 5120, 1280, [1, 4, 8], 2003, "q4 5120x1280")
    # config 3 read as "one scale per output column" (Q8_0_PC, an extension)
    # and the same for the int4 pair's first shape (Q4_0_PC)
    out["q8pc_1024x4096"] = run(_abi.FMT_Q8_0_PC, 1024, 4096, [1, 8], 2002, "q8pc 1024x4096")
    out["q4pc_1280x5120"] = run(_abi.FMT_Q4_0_PC, 1280, 5120, [1, 4], 2002, "q4pc 1280x5120")
    out["f32_vocab_rows_51866x1280"] = run_rows_f32(51866, 1280, [1, 4], 2004, "f32 vocab rows 51866x1280", 4)
    out["q8_vocab_1280x51866"] = run(_abi.FMT_Q8_0, 1280, 51866, [1], 2004, "q8 vocab 1280x51866", 12)
    out["q4_vocab_1280x51866"] = run(_abi.FMT_Q4_0, 1280, 51866, [1], 2004, "q4 vocab 1280x51866", 24)
    return out


def bench_qgemm(torch, dev, sptr, timer, _abi, synth, np):
    """Config 3 at M in {128, 512}: Q8_0 W[1024x4096] (MFMA path)."""
    res = {}
    K, N = 1024, 4096
    w = torch.from_numpy(synth.normal_matrix(2002, K, N, 0.02)).to(dev)
    q = torch.empty(K * N, dtype=torch.uint8, device=dev)
    sc = torch.empty(1, dtype=torch.float32, device=dev)
    _abi.quantize_dev(_abi.FMT_Q8_0, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
    torch.cuda.synchronize()
    scale = float(sc.item())
    for M in (128, 512):
        x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        fn = lambda st: _abi.gemm_dev(_abi.FMT_Q8_0, M, N, K, x.data_ptr(), q.data_ptr(),  # noqa: E731
                                      y.data_ptr(), scale=scale, stream=st)
        # 20 launches per graph replay, as for the per-shape fp32 figures (a
        # graph of one launch adds a graph launch to every kernel)
        ms = timer.time_ms(lambda st, fn=fn: [fn(st) for _ in range(20)], 5, per_replay=20)
        tf = 2.0 * M * N * K / ms / 1e9
        res[f"q8_M{M}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": round(tf / FP32_PEAK_TFLOPS, 4)}
        log(f"qgemm q8 M={M}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
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
    quantizers).  One sweep = 6 layers x 6 GEMMs, 20 sweeps per graph replay."""
    d, ff, M = 384, 1536, tokens
    shapes = [(d, d)] * 4 + [(d, ff), (ff, d)]
    flops = layers * sum(2.0 * M * K * N for (K, N) in shapes)
    x = torch.from_numpy(synth.normal_matrix(1001, M, d)).to(dev)
    h = torch.from_numpy(synth.normal_matrix(1002, M, ff)).to(dev)
    y = torch.empty((M, ff), dtype=torch.float32, device=dev)
    res = {}
    for fmt, name in ((_abi.FMT_F32, "fp32"), (_abi.FMT_F16, "f16"), (_abi.FMT_Q8_K, "q8_k")):
        keep, row = [], []
        for layer in range(layers):
            for i, (K, N) in enumerate(shapes):
                w = torch.from_numpy(synth.normal_matrix(2002 + 8 * layer + i, K, N, 0.02)).to(dev)
                if fmt == _abi.FMT_F32:
                    keep.append(w)
                    row.append((K, N, w.data_ptr(), None))
                    continue
                b = torch.empty(K * N * (2 if fmt == _abi.FMT_F16 else 1), dtype=torch.uint8, device=dev)
                sc = torch.empty(max(K * N // 32, 1), dtype=torch.float32, device=dev)
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
    """Decoder GEMVs for kernel traces / counters: Q8_0 1024x4096 at M = 1
    and 8, Q4_0 1280x5120 and 5120x1280 at M = 1 and 4, each on its prepared
    copy and in the [K,N] layout, `launches` times over 16 distinct weight
    copies (eager launches, one kernel per call); then the Q8_0 and Q4_0
    vocabulary projections (1280 x 51866, M = 1) on 3 / 4 prepared copies."""
    for fmt, K, N, M in ((_abi.FMT_Q8_0, 1024, 4096, 1), (_abi.FMT_Q8_0, 1024, 4096, 8),
                         (_abi.FMT_Q4_0, 1280, 5120, 1), (_abi.FMT_Q4_0, 1280, 5120, 4),
                         (_abi.FMT_Q4_0, 5120, 1280, 1), (_abi.FMT_Q4_0, 5120, 1280, 4)):
        w = torch.from_numpy(synth.normal_matrix(2002, K, N, 0.02)).to(dev)
        nbytes = K * N if fmt == _abi.FMT_Q8_0 else (K * N + 1) // 2
        q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(1, dtype=torch.float32, device=dev)
        _abi.quantize_dev(fmt, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        scale = float(sc.item())
        copies = q.repeat(16).view(16, nbytes)
        hs = [_abi.prepare_dev(fmt, K, N, copies[i].data_ptr(), scale, sptr) for i in range(16)]
        x = torch.from_numpy(synth.normal_matrix(1001, M, K)).to(dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        for i in range(launches):
            _abi.gemm_prepared(hs[i % 16], M, x.data_ptr(), y.data_ptr(), stream=sptr)
        for i in range(launches):
            _abi.gemm_dev(fmt, M, N, K, x.data_ptr(), copies[i % 16].data_ptr(), y.data_ptr(), scale=scale,
                          stream=sptr)
        torch.cuda.synchronize()
        for h_ in hs:
            _abi.prepared_free(h_)
        log(f"profile-gemv: fmt {fmt} {K}x{N}: {launches} prepared + {launches} [K,N] launches")
    # the vocabulary projection (1280 x 51866) at M = 1 on prepared copies
    for fmt, ncopy in ((_abi.FMT_Q8_0, 3), (_abi.FMT_Q4_0, 4)):
        K, N = 1280, 51866
        w = torch.from_numpy(synth.normal_matrix(2004, K, N, 0.02)).to(dev)
        nbytes = K * N if fmt == _abi.FMT_Q8_0 else (K * N + 1) // 2
        q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        sc = torch.empty(1, dtype=torch.float32, device=dev)
        _abi.quantize_dev(fmt, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
        torch.cuda.synchronize()
        copies = q.repeat(ncopy).view(ncopy, nbytes)
        del w
        hs = [_abi.prepare_dev(fmt, K, N, copies[i].data_ptr(), float(sc.item()), sptr) for i in range(ncopy)]
        x = torch.from_numpy(synth.normal_matrix(1001, 1, K)).to(dev)
        y = torch.empty((1, N), dtype=torch.float32, device=dev)
        for i in range(launches):
            _abi.gemm_prepared(hs[i % ncopy], 1, x.data_ptr(), y.data_ptr(), stream=sptr)
        torch.cuda.synchronize()
        for h_ in hs:
            _abi.prepared_free(h_)
        del copies
        torch.cuda.empty_cache()
        log(f"profile-gemv: fmt {fmt} vocab {K}x{N}: {launches} prepared launches")
    # the f32 token embedding [51866 x 1280] used in place (rows-prepared), M = 1
    K, N, ncopy = 1280, 51866, 3
    e = torch.from_numpy(synth.normal_matrix(2004, N, K, 0.02)).to(dev)
    copies = e.reshape(1, N * K).repeat(ncopy, 1)
    del e
    hs = [_abi.prepare_rows_dev(_abi.FMT_F32, K, N, copies[i].data_ptr(), 4 * K, 1.0, sptr) for i in range(ncopy)]
    x = torch.from_numpy(synth.normal_matrix(1001, 1, K)).to(dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    for i in range(launches):
        _abi.gemm_prepared(hs[i % ncopy], 1, x.data_ptr(), y.data_ptr(), stream=sptr)
    torch.cuda.synchronize()
    for h_ in hs:
        _abi.prepared_free(h_)
    del copies
    torch.cuda.empty_cache()
    log(f"profile-gemv: f32 embedding rows {N}x{K} in place: {launches} launches")
    print(json.dumps({"profile_gemv": True}), flush=True)


def bench_config5(torch, dev, sptr, _abi, layers: int = 32):
    """Config 5: the Whisper large-v3-turbo encoder linears at 1500 frames --
    X[1500x1280] . W[1280x3840] (fused QKV), X . W[1280x5120] (FFN up),
    H[1500x5120] . W[5120x1280] (FFN down) -- for each of `layers` layers with
    their own weights, back to back, in fp32 and as Q8_0 / Q4_0 weights
    (quantized on the device by the reference quantizer).  Weights are drawn
    on the GPU (seeded N(0, 0.02)); X, H ~ N(0, 1).  The fp32 sweep streams
    2.3 GB of weights, more than the 256 MB Infinity Cache."""
    shapes = [(1500, 3840, 1280), (1500, 5120, 1280), (1500, 1280, 5120)]
    flops = layers * sum(2.0 * M * N * K for (M, N, K) in shapes)
    g = torch.Generator(device=dev)
    g.manual_seed(1001)
    x = torch.randn(1500, 1280, generator=g, device=dev)
    h = torch.randn(1500, 5120, generator=g, device=dev)
    outs = [torch.empty(M, N, device=dev) for (M, N, K) in shapes]
    res = {}
    for fmt, name in ((_abi.FMT_F32, "fp32"), (_abi.FMT_Q8_0, "q8_0"), (_abi.FMT_Q4_0, "q4_0")):
        weights = []  # per layer: [(ptr, scale)] and the tensors that own them
        keep = []
        for layer in range(layers):
            g.manual_seed(2002 + layer)
            row = []
            for (M, N, K) in shapes:
                w = torch.randn(K, N, generator=g, device=dev) * 0.02
                if fmt == _abi.FMT_F32:
                    keep.append(w)
                    row.append((w.data_ptr(), 1.0))
                    continue
                nbytes = K * N if fmt == _abi.FMT_Q8_0 else (K * N + 1) // 2
                q = torch.empty(nbytes, dtype=torch.uint8, device=dev)
                sc = torch.empty(1, dtype=torch.float32, device=dev)
                _abi.quantize_dev(fmt, K * N, w.data_ptr(), q.data_ptr(), sc.data_ptr(), sptr)
                keep.append((q, sc))
                row.append((q.data_ptr(), sc))
                del w
            weights.append(row)
        torch.cuda.synchronize()
        weights = [[(p, s if isinstance(s, float) else float(s.item())) for (p, s) in row] for row in weights]

        def sweep():
            for row in weights:
                for i, (M, N, K) in enumerate(shapes):
                    a = x if K == 1280 else h
                    p, sc = row[i]
                    _abi.gemm_dev(fmt, M, N, K, a.data_ptr(), p, outs[i].data_ptr(), scale=sc, stream=sptr)

        # warm-up: workspaces, then sweeps until the clocks have settled
        t_end = time.perf_counter() + 0.3
        sweep()
        torch.cuda.synchronize()
        while time.perf_counter() < t_end:
            sweep()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 3
        e0.record()
        for _ in range(reps):
            sweep()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / reps
        tf = flops / (ms * 1e-3) / 1e12
        wbytes = sum((K * N * 4 if fmt == _abi.FMT_F32 else (K * N if fmt == _abi.FMT_Q8_0 else K * N // 2))
                     for (M, N, K) in shapes) * layers
        res[name] = {"ms_per_sweep": round(ms, 3), "TFLOP/s": round(tf, 2), "frac": round(tf / FP32_PEAK_TFLOPS, 4),
                     "weight_bytes": wbytes}
        log(f"config5 {name}: {layers} layers, {ms:.2f} ms/sweep, {tf:.1f} TFLOP/s")
        del keep, weights
        torch.cuda.empty_cache()
    res["flops_per_sweep"] = flops
    res["layers"] = layers
    return res


def cpu_baseline(budget_s: float):
    """The reference's fp32 CPU path (oracle restatement of the register-
    blocked ops.zig fallback, single-threaded as in the reference) on the
    headline step; repeated until about `budget_s` seconds are spent."""
    from oracle import oracle as orc
    from tomoul_amd import synth

    xs = synth.normal_matrix(1001, 512, 1024)
    hs = synth.normal_matrix(1001, 512, 4096)
    wts = [synth.normal_matrix(2002 + i, K, N, 0.02) for i, (_, M, N, K) in enumerate(XLMR_SHAPES)]
    ins = [xs, xs, xs, hs]
    step_flops = sum(2.0 * M * N * K for (_, M, N, K) in XLMR_SHAPES)
    orc.lib()
    steps, t_tot = 0, 0.0
    while t_tot < budget_s and steps < 50:
        t0 = time.perf_counter()
        for i in range(4):
            orc.matmul(ins[i], wts[i])
        t_tot += time.perf_counter() - t0
        steps += 1
    tf = step_flops * steps / t_tot / 1e12
    log(f"cpu baseline: {steps} steps in {t_tot:.1f} s, {tf * 1e3:.2f} GFLOP/s (1 thread)")
    # The same loops row-parallel (rows are independent, results bitwise
    # unchanged) with the reference's matmulParallel cap of 4 threads
    # (src/core/context.zig:285) and with every host thread the oracle's
    # OpenMP runtime offers; a few steps each, reported beside the baseline.
    threaded = {}
    for nt in sorted({4, max(1, orc.max_threads())}):
        n_mt, t_mt = 0, 0.0
        while t_mt < budget_s / 4 and n_mt < 50:
            t0 = time.perf_counter()
            for i in range(4):
                orc.matmul_mt(ins[i], wts[i], nt)
            t_mt += time.perf_counter() - t0
            n_mt += 1
        threaded[f"{nt}_threads"] = {"value": round(step_flops * n_mt / t_mt / 1e12, 6), "steps": n_mt,
                                     "seconds": round(t_mt, 2)}
        log(f"cpu baseline, {nt} threads: {n_mt} steps in {t_mt:.1f} s, "
            f"{step_flops * n_mt / t_mt / 1e9:.2f} GFLOP/s")
    return {"value": round(tf, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{steps} full headline steps (4 GEMMs, {step_flops / 1e9:.2f} GFLOP each) with the "
                      f"oracle's restatement of the ops.zig:277-414 fallback, 1 thread, -O3 AVX2, "
                      f"{t_tot:.1f} s; zblas (the reference default) is not vendored and cannot be timed",
            "host_cpus": os.cpu_count(), "threaded": threaded}


if __name__ == "__main__":
    main()
