#!/usr/bin/env python3
"""Benchmark of the FP4 dequant-GEMM hot path on one MI355X.

Headline (BASELINE.json metric "FP4 dequant-GEMM: achieved HBM TB/s at M=1;
TFLOP/s at M=2048"):
  * value  = achieved HBM TB/s at M=1 over one Llama-3-8B layer (config 2: qkv
    4096->6144, o 4096->4096, gate_up 4096->28672, down 14336->4096, summed),
    algorithmic bytes (packed weights + scales + A + C) / GPU time;
  * prefill = TFLOP/s at M=2048 on 4096->14336 and 14336->4096 (config 4).
A "step" is one pass of the four layer GEMMs.  Weights are synthetic
(N(0, 0.02) fp16 quantized on the GPU by the library's FP4 quantizer, g=128),
with enough rotated copies that every step reads HBM, not the 256 MB
Infinity Cache.  Kernel time comes from HIP events recorded on the launch
stream; the launches are queued behind a GPU sleep so host launch overhead is
not part of the measurement (this is the time a captured decode loop sees).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--all]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "metal-marlin_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA, TFLOP/s
G = 128
LLAMA_LAYER = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672),
               ("down", 14336, 4096)]
PREFILL = [("up", 4096, 14336), ("down", 14336, 4096)]
ROTATE_BYTES = 640 << 20       # rotated weight footprint > 2.5x the 256 MB MALL


def alg_bytes(M: int, K: int, N: int, int4: bool = False) -> int:
    """Algorithmic HBM bytes of one GEMM: packed B + scales (+ zeros) + A + C."""
    b = K * N // 2 + 2 * N * (K // G) * (2 if int4 else 1)
    return b + 2 * M * K + 2 * M * N


def make_weights(torch, mmfp4, K: int, N: int, seed: int, int4: bool = False):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    if int4:
        return mmfp4.pack_u4_weights(w, group_size=G)
    return mmfp4.quantize_fp4(w, group_size=G)


def gpu_sleep_ahead(torch, ms: float = 60.0) -> None:
    """Queue a GPU-side wait so the host can enqueue the timed launches ahead."""
    torch.cuda._sleep(int(ms * 1e-3 * 1.9e9))   # ~1.9e6 sleep cycles per ms


def timed_launches(torch, launches, steps: int, warmup: int) -> float:
    """Run `launches` (list of per-step lists of callables, rotated) for
    `warmup` untimed then `steps` timed steps; returns ms over the timed steps
    (HIP events on the launch stream; only two events, so nothing is inserted
    between the kernels).  The launches are queued behind a GPU sleep sized
    from the measured host enqueue rate; if the sleep ran out before the host
    finished enqueueing (the GPU could have idled), the run is repeated with a
    longer sleep."""
    t_host = time.perf_counter()
    for s in range(warmup):
        for fn in launches[s % len(launches)]:
            fn()
    per_launch_s = (time.perf_counter() - t_host) / max(1, warmup * len(launches[0]))
    torch.cuda.synchronize()
    sleep_ms = 2.0 + 3e3 * per_launch_s * steps * len(launches[0])
    for _ in range(6):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gpu_sleep_ahead(torch, sleep_ms)
        t0.record()
        for s in range(steps):
            for fn in launches[s % len(launches)]:
                fn()
        starved = t0.query()          # sleep already over while still enqueueing
        t1.record()
        torch.cuda.synchronize()
        if not starved:
            return t0.elapsed_time(t1)
        sleep_ms *= 3
    raise RuntimeError("could not queue the timed launches ahead of the GPU")


def per_shape_us(torch, launches, reps: int = 40) -> list[float]:
    """Average µs per launch of each step position, timed in its own batch."""
    out = []
    for i in range(len(launches[0])):
        seq = [[step[i]] for step in launches]
        out.append(1e3 * timed_launches(torch, seq, reps, 2) / reps)
    return out


def run_layer_bench(torch, mmfp4, M: int, steps: int, warmup: int, int4: bool = False):
    layer_w = sum(alg_bytes(0, K, N, int4) for _, K, N in LLAMA_LAYER)
    copies = max(2, -(-ROTATE_BYTES // layer_w))
    sets = []
    for c in range(copies):
        ws = [make_weights(torch, mmfp4, K, N, 100 * c + i, int4)
              for i, (_, K, N) in enumerate(LLAMA_LAYER)]
        sets.append(ws)
    gen = torch.Generator(device="cuda").manual_seed(1)
    acts = {K: torch.randn((M, K), generator=gen, device="cuda").half() for _, K, _ in LLAMA_LAYER}
    launches = []
    for ws in sets:
        step = []
        for (_, K, N), wt in zip(LLAMA_LAYER, ws):
            a = acts[K]
            if int4:
                step.append(lambda a=a, w=wt: mmfp4.marlin_gemm_int4(a, w[0], w[1], w[2], G))
            else:
                step.append(lambda a=a, w=wt: mmfp4.marlin_gemm_fp4(a, w[0], w[1], G))
        launches.append(step)
    total_ms = timed_launches(torch, launches, steps, warmup)
    step_bytes = sum(alg_bytes(M, K, N, int4) for _, K, N in LLAMA_LAYER)
    per_shape = {}
    for (name, K, N), us in zip(LLAMA_LAYER, per_shape_us(torch, launches)):
        per_shape[name] = {"K": K, "N": N, "us": round(us, 3),
                           "GBps": round(alg_bytes(M, K, N, int4) / (us * 1e3), 1)}
    return {"ms_per_step": total_ms / steps, "step_bytes": step_bytes,
            "launch_us_avg": 1e3 * total_ms / (steps * len(LLAMA_LAYER)),
            "per_shape": per_shape, "copies": copies}


# Read-kernel configurations (blocks, threads, 16-byte loads in flight per
# lane, mode: bit 0 non-temporal, bit 1 grid-stride order) that came out on
# top of a 336-point sweep of mm_stream_read on MI355X for 8.7-60.6 MB
# (profiles/hbm_read_ceiling_sweep.md); the first is the aid's default plan.
READ_CONFIGS = [(0, 0, 4, 1), (4096, 512, 2, 3), (1024, 512, 4, 1), (2048, 1024, 2, 1),
                (1024, 512, 2, 3), (2048, 512, 2, 3), (8192, 256, 2, 3), (4096, 512, 2, 1)]


def best_read(torch, nbytes: int, steps: int, warmup: int):
    """The fastest of READ_CONFIGS for one read of `nbytes` (rotated buffers
    past the Infinity Cache, back-to-back launches, HIP events): (µs, config,
    launch builder for that config)."""
    import bench_aids
    copies = max(2, -(-ROTATE_BYTES // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    sink = torch.empty(16384 * 1024, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream

    def mk(cfg):
        return [[lambda b=b: bench_aids.call("mm_stream_read", b.data_ptr(), nbytes,
                                             sink.data_ptr(), sink.numel() * 4, *cfg, st)]
                for b in bufs]
    best = None
    for cfg in READ_CONFIGS:
        us = 1e3 * timed_launches(torch, mk(cfg), steps, warmup) / steps
        if best is None or us < best[0]:
            best = (us, cfg)
    return best[0], best[1], mk


def run_read_sweep(torch):
    """Sweep mm_stream_read over grid, loads in flight, cache hint and order
    for the layer's read sizes (8.7, 13.0, 30.3 and 60.6 MB): µs per launch,
    back to back over rotated buffers, best of three timed batches of 60."""
    import itertools
    import bench_aids
    st = torch.cuda.current_stream().cuda_stream
    sink = torch.empty(16384 * 1024, dtype=torch.int32, device="cuda")
    rows = []
    for nbytes in (8_650_752, 12_999_984, 30_277_632, 60_555_264):
        copies = max(2, -(-800_000_000 // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        for blocks, threads, unroll, mode in itertools.product(
                (256, 512, 1024, 2048, 4096, 8192, 16384), (256, 512, 1024), (2, 4, 8, 16),
                (0, 1, 2, 3)):
            if blocks * threads > 16384 * 1024:
                continue
            cfg = (blocks, threads, unroll, mode)
            launches = [[lambda b=b, cfg=cfg: bench_aids.call(
                "mm_stream_read", b.data_ptr(), nbytes, sink.data_ptr(), sink.numel() * 4, *cfg,
                st)] for b in bufs]
            us = min(1e3 * timed_launches(torch, launches, 60, 4) / 60 for _ in range(3))
            rows.append({"bytes": nbytes, "blocks": blocks, "threads": threads,
                         "unroll": unroll, "mode": mode, "us": round(us, 3),
                         "TBps": round(nbytes / us / 1e6, 3)})
        del bufs
        torch.cuda.empty_cache()
    best = {}
    for r in rows:
        if r["bytes"] not in best or r["us"] < best[r["bytes"]]["us"]:
            best[r["bytes"]] = r
    return {"best": list(best.values()), "points": len(rows), "all": rows}


def run_read_ceiling(torch, steps: int, warmup: int):
    """The HBM read rate this GPU reaches for the same bytes in the same
    back-to-back launch pattern: `mm_stream_read` (a read-only stream, no
    decode, no math, nothing written; bench_aids) over each layer GEMM's
    packed weights + scales, rotated copies, timed exactly like the GEMMs, in
    the best of READ_CONFIGS for each size.  The practical ceiling of a
    weight-streaming kernel of that size (launch, ramp-up and drain
    included)."""
    per, cfgs, launches = {}, {}, []
    for name, K, N in LLAMA_LAYER:
        nbytes = -(-alg_bytes(0, K, N) // 16) * 16
        us, cfg, mk = best_read(torch, nbytes, steps, warmup)
        per[name], cfgs[name] = round(us, 3), list(cfg)
        launches.append(mk(cfg))
    n = min(len(x) for x in launches)
    step = [[launches[j][i][0] for j in range(len(LLAMA_LAYER))] for i in range(n)]
    total_ms = timed_launches(torch, step, steps, warmup)
    byts = sum(-(-alg_bytes(0, K, N) // 16) * 16 for _, K, N in LLAMA_LAYER)
    return {"kernel": "mm_stream_read (bench_aids: 16-byte loads, no writes), best of "
                      f"{len(READ_CONFIGS)} configurations per size",
            "per_shape_us": per, "per_shape_config": cfgs,
            "layer_us": round(1e3 * total_ms / steps, 3),
            "layer_TBps": round(byts / (total_ms / steps * 1e-3) / 1e12, 3)}


def run_prefill_bench(torch, mmfp4, M: int, steps: int, warmup: int):
    ws = [make_weights(torch, mmfp4, K, N, 7 + i) for i, (_, K, N) in enumerate(PREFILL)]
    gen = torch.Generator(device="cuda").manual_seed(2)
    acts = {K: torch.randn((M, K), generator=gen, device="cuda").half() for _, K, _ in PREFILL}
    step = [lambda a=acts[K], w=w: mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
            for (_, K, _), w in zip(PREFILL, ws)]
    total_ms = timed_launches(torch, [step], steps, warmup)
    flops = sum(2 * M * K * N for _, K, N in PREFILL)
    per_shape = {}
    for (name, K, N), us in zip(PREFILL, per_shape_us(torch, [step], reps=max(3, steps))):
        per_shape[name] = {"K": K, "N": N, "us": round(us, 2),
                           "TFLOPs": round(2 * M * K * N / (us * 1e-6) / 1e12, 1)}
    return {"ms_per_step": total_ms / steps, "flops": flops, "per_shape": per_shape,
            "launch_us_avg": 1e3 * total_ms / (steps * len(PREFILL))}


def prefill_steps(args) -> tuple[int, int]:
    """(timed, warm-up) steps of the M=2048 prefill pair.  Each step is about
    0.5 ms of full-chip MFMA load; the clock needs ~10 ms of it to settle (a
    measured ramp on MI355X: 851 -> 930 -> 969 -> 996 TF/s over the first
    runs), so the untimed warm-up covers that before the timed steps."""
    return max(20, args.steps // 5), max(20, args.warmup)


def run_mfma_ceiling(torch, mmfp4, prefill_tflops: float):
    """The sustained MFMA 32x32x16 f16 rate on this GPU with nothing else in
    the loop (`mm_mfma_ceiling`), fed (a) the prefill GEMM's own operand
    values -- N(0,1) fp16 activations and the decoded FP4 weights of the
    config-4 matrices -- and (b) all-ones operands.  The board's power limit
    lowers the clock as more operand bits toggle, so (a) is the practical
    matrix-core ceiling of this GEMM and (b) shows the dense peak."""
    import bench_aids
    n = 1 << 20
    gen = torch.Generator(device="cuda").manual_seed(11)
    acts = torch.randn(n, generator=gen, device="cuda").half()
    wp, ws = make_weights(torch, mmfp4, 4096, 256, 13)
    wdq = mmfp4.dequant_fp4(wp, ws, 4096, 256, G).reshape(-1).contiguous()
    ones = torch.ones(n, device="cuda").half()
    sink = torch.empty(256 * 512, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    iters = 400
    flops = 256 * 8 * iters * 32 * 32768.0
    res = {"kernel": "mm_mfma_ceiling (MFMA 32x32x16 f16 only, 256 blocks x 8 waves)"}
    for name, a, b in (("gemm_operands", acts, wdq), ("ones", ones, ones)):
        nh = min(a.numel(), b.numel()) // 8 * 8
        fn = lambda a=a, b=b, nh=nh: bench_aids.call("mm_mfma_ceiling", a.data_ptr(), b.data_ptr(),
                                                     nh, iters, sink.data_ptr(), sink.numel() * 4,
                                                     st)
        ms = timed_launches(torch, [[fn]], 40, 40)
        res[name + "_tflops"] = round(flops * 40 / (ms * 1e-3) / 1e12, 1)
    res["prefill_fraction_of_gemm_operand_ceiling"] = round(
        prefill_tflops / res["gemm_operands_tflops"], 4)
    return res


def run_single_bench(torch, mmfp4, M: int, K: int, N: int, steps: int):
    """One FP4 linear (config 1: M=1, 4096 -> 4096), rotated weight copies."""
    copies = max(2, -(-ROTATE_BYTES // alg_bytes(0, K, N)))
    ws = [make_weights(torch, mmfp4, K, N, 500 + c) for c in range(copies)]
    a = torch.randn((M, K), device="cuda").half()
    launches = [[lambda w=w: mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)] for w in ws]
    ms = timed_launches(torch, launches, steps, 10)
    us = 1e3 * ms / steps
    return {"M": M, "K": K, "N": N, "us": round(us, 3),
            "TBps": round(alg_bytes(M, K, N) / (us * 1e-6) / 1e12, 3)}


def rand_weights(torch, K: int, N: int, gen):
    """Random packed words and scales of the right shape (timing only: the
    kernels' cost does not depend on the values)."""
    p = torch.randint(-2**31, 2**31 - 1, (K // 8, N), generator=gen, dtype=torch.int32,
                      device="cuda")
    s = (torch.rand((K // G, N), generator=gen, device="cuda") * 0.01).half()
    return p, s


def run_north_star_decode(torch, mmfp4, steps: int):
    """The north star's decode shapes at M=1 (4096 -> 14336 and 14336 -> 4096),
    each on its own with rotated weight copies: µs per launch, algorithmic
    TB/s, fraction of HBM peak and of the 0.70 target, and beside it the best
    single-launch read of the same weight bytes (best_read) and the GEMM's
    fraction of that read time."""
    out = {}
    for name, K, N in (("4096x14336", 4096, 14336), ("14336x4096", 14336, 4096)):
        copies = max(2, -(-ROTATE_BYTES // alg_bytes(0, K, N)))
        ws = [make_weights(torch, mmfp4, K, N, 700 + c) for c in range(copies)]
        a = torch.randn((1, K), device="cuda").half()
        launches = [[lambda w=w: mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)] for w in ws]
        us = 1e3 * timed_launches(torch, launches, steps, 10) / steps
        tbs = alg_bytes(1, K, N) / (us * 1e-6) / 1e12
        del ws
        ceil_us, cfg, _ = best_read(torch, -(-alg_bytes(0, K, N) // 16) * 16, steps, 10)
        out[name] = {"us": round(us, 3), "TBps": round(tbs, 3),
                     "frac_hbm_peak": round(tbs * 1e3 / HBM_PEAK_GBS, 4),
                     "frac_of_0.70_target": round(tbs * 1e3 / HBM_PEAK_GBS / 0.70, 4),
                     "read_ceiling_us": round(ceil_us, 3), "read_ceiling_config": list(cfg),
                     "read_ceiling_frac_hbm_peak": round(
                         alg_bytes(0, K, N) / (ceil_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "frac_of_read_ceiling": round(ceil_us / us, 4)}
    return out


def run_host_paced(torch, mmfp4, n: int = 400):
    """Per-call latency as a caller without a captured graph sees it: the
    Python-level enqueue time per marlin_gemm_fp4 call, and the wall time per
    call of back-to-back calls synchronised once at the end (no GPU-side
    queue-ahead)."""
    out = {}
    for name, M, K, N in (("config1_4096x4096_M1", 1, 4096, 4096),
                          ("4096x14336_M1", 1, 4096, 14336)):
        w = make_weights(torch, mmfp4, K, N, 800)
        a = torch.randn((M, K), device="cuda").half()
        for _ in range(20):
            mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        out[name] = {"host_enqueue_us_per_call": round(1e6 * (t1 - t0) / n, 2),
                     "wall_us_per_call": round(1e6 * (t2 - t0) / n, 2)}
    out["llama_layer_M1"] = run_layer_graph(torch, mmfp4, max(50, n // 4))
    return out


def run_layer_graph(torch, mmfp4, n: int):
    """The four Llama-layer GEMMs at M=1 host-paced, eager (four library calls
    per step), as one captured HIP graph of one step replayed per step, and as
    one graph of ten steps: wall µs per step over back-to-back steps (same
    weights every step), plus the GPU-side time per step with the launches
    queued behind a GPU sleep (no host pacing).  A replay costs a fixed gap on
    the GPU between consecutive graph launches; kernels inside a graph run at
    their eager durations, so longer graphs amortise it."""
    ws = [make_weights(torch, mmfp4, K, N, 820 + i) for i, (_, K, N) in enumerate(LLAMA_LAYER)]
    xs = {K: torch.randn((1, K), device="cuda").half() for _, K, _ in LLAMA_LAYER}

    def step():
        return [mmfp4.marlin_gemm_fp4(xs[K], w[0], w[1], G)
                for (_, K, _), w in zip(LLAMA_LAYER, ws)]

    def wall(fn, reps, per):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        w = 1e6 * (time.perf_counter() - t0) / (reps * per)
        gpu = 1e3 * timed_launches(torch, [[fn]], reps, 2) / (reps * per)
        return round(w, 2), round(gpu, 2)

    eager = wall(step, n, 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g1, g10 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=s):
        step()
    with torch.cuda.graph(g10, stream=s):
        for _ in range(10):
            step()
    graph = wall(g1.replay, n, 1)
    graph10 = wall(g10.replay, max(5, n // 10), 10)
    return {"eager_wall_us_per_step": eager[0], "eager_gpu_us_per_step": eager[1],
            "graph_wall_us_per_step": graph[0], "graph_gpu_us_per_step": graph[1],
            "graph_of_10_steps_wall_us_per_step": graph10[0],
            "graph_of_10_steps_gpu_us_per_step": graph10[1],
            "launches_per_step": len(LLAMA_LAYER)}


def cpu_model_name() -> str:
    """The host CPU's model name as lscpu prints it (from /proc/cpuinfo), with
    the CPU family and model numbers, which identify the generation where a
    virtual machine reports only a generic name (family 26 = Zen 5)."""
    info = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key = key.strip().lower()
            if key in ("model name", "cpu family", "model") and key not in info:
                info[key] = val.strip()
            if not line.strip() and info:
                break
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or "unknown"
    if "cpu family" in info:
        name += f" (family {info['cpu family']} model {info.get('model', '?')})"
    return name


def run_fused_bench(torch, mmfp4, steps: int):
    """The operators either side of the GEMM at the Llama-3-8B and Qwen3 MoE
    shapes, fused vs unfused, rotated weight copies: gate_up+SiLU (4096 ->
    2 x 14336) at M=1 and M=2048, the Q/K/V projections (4096 -> 4096 + 1024
    + 1024) at M=1, and the router at T=32 and T=1024."""
    gen = torch.Generator(device="cuda").manual_seed(900)
    res = {}
    K, N = 4096, 14336
    copies = max(2, -(-ROTATE_BYTES // (2 * alg_bytes(0, K, N))))
    gu = [(rand_weights(torch, K, N, gen), rand_weights(torch, K, N, gen)) for _ in range(copies)]
    cat = [(torch.cat([g[0], u[0]], 1), torch.cat([g[1], u[1]], 1)) for g, u in gu]
    for M, st in ((1, steps), (2048, max(3, steps // 40))):
        a = torch.randn((M, K), generator=gen, device="cuda").half()
        fused = [[lambda w=w: mmfp4.mmfp4_fused_gate_up_marlin(a, w[0][0], w[0][1], w[1][0],
                                                               w[1][1], G)] for w in gu]
        def unfused_step(w):
            h = mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
            return torch.nn.functional.silu(h[:, :N]) * h[:, N:]
        unfused = [[lambda w=w: unfused_step(w)] for w in cat]
        uf = 1e3 * timed_launches(torch, fused, st, 3) / st
        uu = 1e3 * timed_launches(torch, unfused, st, 3) / st
        byts = 2 * alg_bytes(M, K, N) - 2 * M * K
        res[f"gate_up_silu_M{M}"] = {
            "K": K, "N_each": N, "fused_us": round(uf, 2), "unfused_us": round(uu, 2),
            "fused_TBps": round(byts / (uf * 1e-6) / 1e12, 3),
            "fused_TFLOPs": round(4 * M * K * N / (uf * 1e-6) / 1e12, 1),
            "unfused": "marlin_gemm_fp4 on the concatenated [K/8, 2N] weights + torch silu*mul"}
    # The reference's mmfp4_fused_gate_up and MMFP4 GEMM take row-packed [N, K/8] weights:
    # read in place against transposing them per call, as the reference does.
    rows = [((g[0].t().contiguous(), g[1]), (u[0].t().contiguous(), u[1])) for g, u in gu]
    del cat
    for M, st in ((1, steps), (2048, max(3, steps // 40))):
        a = torch.randn((M, K), generator=gen, device="cuda").half()
        inplace = [[lambda w=w: mmfp4.mmfp4_fused_gate_up(a, w[0][0], w[0][1], w[1][0], w[1][1],
                                                          G)] for w in rows]
        transp = [[lambda w=w: mmfp4.mmfp4_fused_gate_up_marlin(
            a, w[0][0].t().contiguous(), w[0][1], w[1][0].t().contiguous(), w[1][1], G)]
            for w in rows]
        one = [[lambda w=w: mmfp4.mmfp4_gemm_rowpacked(a, w[0][0], w[0][1], G)] for w in rows]
        ui = 1e3 * timed_launches(torch, inplace, st, 3) / st
        ut = 1e3 * timed_launches(torch, transp, max(3, st // 4), 2) / max(3, st // 4)
        uo = 1e3 * timed_launches(torch, one, st, 3) / st
        res[f"rowpacked_M{M}"] = {
            "K": K, "N": N, "gate_up_silu_in_place_us": round(ui, 2),
            "gate_up_silu_transpose_per_call_us": round(ut, 2),
            "gemm_in_place_us": round(uo, 2),
            "gate_up_silu_in_place_TFLOPs": round(4 * M * K * N / (ui * 1e-6) / 1e12, 1)}
    del gu, rows
    Ns = (4096, 1024, 1024)
    copies = max(2, -(-ROTATE_BYTES // sum(alg_bytes(0, K, n) for n in Ns)))
    qkv = [[rand_weights(torch, K, n, gen) for n in Ns] for _ in range(copies)]
    a = torch.randn((1, K), generator=gen, device="cuda").half()
    fused = [[lambda w=w: mmfp4.mmfp4_fused_qkv(a, w[0][0], w[0][1], w[1][0], w[1][1], w[2][0],
                                                w[2][1], G)] for w in qkv]
    sep = [[lambda w=w, i=i: mmfp4.marlin_gemm_fp4(a, w[i][0], w[i][1], G) for i in range(3)]
           for w in qkv]
    uf = 1e3 * timed_launches(torch, fused, steps, 5) / steps
    us = 1e3 * timed_launches(torch, sep, steps, 5) / steps
    byts = sum(alg_bytes(1, K, n) for n in Ns) - 2 * 2 * K
    res["qkv_M1"] = {"K": K, "N": list(Ns), "fused_us": round(uf, 2), "three_launches_us":
                     round(us, 2), "fused_TBps": round(byts / (uf * 1e-6) / 1e12, 3)}
    # Router (config 5 shape): gate GEMM + softmax + top-8 + renormalise.
    E, H, k = MOE["E"], MOE["H"], MOE["k"]
    gate = torch.nn.Linear(H, E, bias=False).to("cuda").half()
    for T in (32, 1024):
        x = torch.randn((T, H), generator=gen, device="cuda").half()

        def torch_router():
            p = torch.softmax(gate(x).float(), -1)
            w, i = torch.topk(p, k, -1)
            return (w / w.sum(-1, keepdim=True)).half(), i
        uf = 1e3 * timed_launches(torch, [[lambda: mmfp4.fused_router_topk(x, gate, k)]],
                                  steps, 5) / steps
        ut = 1e3 * timed_launches(torch, [[torch_router]], steps, 5) / steps
        res[f"router_T{T}"] = {"E": E, "H": H, "k": k, "fused_us": round(uf, 2),
                               "torch_ops_us": round(ut, 2)}
    return res


def hipblaslt_fp16_reference(torch, M: int):
    """Plain fp16 GEMM (torch.matmul -> hipBLASLt) on the prefill shapes with
    already-dequantised weights: the vendor library's rate for the same
    arithmetic without the FP4 decode, as context for the prefill figure."""
    out = {}
    for name, K, N in PREFILL:
        a = torch.randn((M, K), device="cuda").half()
        w = torch.randn((K, N), device="cuda").half()
        for _ in range(3):
            a @ w
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(10):
            a @ w
        t1.record()
        torch.cuda.synchronize()
        us = 1e3 * t0.elapsed_time(t1) / 10
        out[name] = {"us": round(us, 2), "TFLOPs": round(2 * M * K * N / (us * 1e-6) / 1e12, 1)}
    return out


MOE = {"E": 128, "H": 2048, "I": 768, "k": 8}


def run_moe_bench(torch, mmfp4, T: int, steps: int, warmup: int = 60):
    """Qwen3-30B-A3B routed experts (config 5): sort -> gate_up (+SwiGLU) ->
    down -> combine, four launches, all 128 experts resident; router logits
    N(0,1) seed 2, fp32 softmax -> top-8 -> renormalise.  Two copies of the
    expert weights (622 MB) are rotated so each step reads HBM.  The untimed
    warm-up (60 steps, ~10 ms at T=1024) lets the clock settle first."""
    E, H, I, k = MOE["E"], MOE["H"], MOE["I"], MOE["k"]
    sets = []
    for c in range(2):
        gen = torch.Generator(device="cuda").manual_seed(600 + c)
        gu_p = torch.empty((E, H // 8, 2 * I), dtype=torch.int32, device="cuda")
        gu_s = torch.empty((E, H // G, 2 * I), dtype=torch.float16, device="cuda")
        dn_p = torch.empty((E, I // 8, H), dtype=torch.int32, device="cuda")
        dn_s = torch.empty((E, I // G, H), dtype=torch.float16, device="cuda")
        for e in range(E):
            w = (torch.randn((2 * I, H), generator=gen, device="cuda") * 0.02).half()
            gu_p[e], gu_s[e] = mmfp4.quantize_fp4(w, group_size=G)
            w = (torch.randn((H, I), generator=gen, device="cuda") * 0.02).half()
            dn_p[e], dn_s[e] = mmfp4.quantize_fp4(w, group_size=G)
        sets.append((gu_p, gu_s, dn_p, dn_s))
    gen = torch.Generator(device="cuda").manual_seed(2)
    logits = torch.randn((T, E), generator=gen, device="cuda")
    probs = torch.softmax(logits.float(), dim=-1)
    topw, ids = torch.topk(probs, k, dim=-1)
    topw = topw / topw.sum(dim=-1, keepdim=True)
    x = torch.randn((T, H), generator=gen, device="cuda").half()
    used = int(torch.unique(ids).numel())
    launches = [[lambda s=s: mmfp4.moe_mlp_fp4(x, s[0], s[1], s[2], s[3], ids, topw, G)]
                for s in sets]
    ms = timed_launches(torch, launches, steps, warmup)
    us = 1e3 * ms / steps
    per_expert = (H * 2 * I // 2 + 2 * 2 * I * (H // G)) + (I * H // 2 + 2 * H * (I // G))
    byts = used * per_expert + 2 * T * H * 2 + 2 * (T * k) * I * 2
    flops = 9437184 * T * k
    return {"T": T, "experts_hit": used, "us": round(us, 2),
            "TBps": round(byts / (us * 1e-6) / 1e12, 3),
            "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1), "algorithmic_bytes": byts}


def measured_traffic(name: str) -> float | None:
    """HBM bytes per launch from the committed rocprofv3 --pmc summary (FETCH_SIZE
    and WRITE_SIZE runs of `bench.py --pmc-probe`, calibrated on a known copy)."""
    path = ROOT / "profiles" / name
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def cpu_baseline(budget_s: float = 15.0):
    """The reference's CPU path (torch fp32 LUT dequant + matmul, redone per
    call) over the same Llama layer at M=1, on this host's cores."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.cpu_path import marlin_gemm_fp4_cpu
    from oracle.fp4 import quantize_fp4
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    mats = []
    for _, K, N in LLAMA_LAYER:
        # random codes/scales of the right shape (quantizing 112 M weights on
        # the host would dominate the budget); the CPU path's cost does not
        # depend on the values.
        packed = torch.from_numpy(rng.integers(0, 2**32, (K // 8, N), dtype=np.uint64)
                                  .astype(np.uint32).view(np.int32))
        scales = torch.from_numpy(rng.normal(0, 0.005, (K // G, N)).astype(np.float16))
        mats.append((torch.randn(1, K).half(), packed, scales))
    del quantize_fp4
    marlin_gemm_fp4_cpu(*mats[1], G)          # warm-up on the smallest shape
    t0 = time.perf_counter()
    steps = 0
    while True:
        for a, p, s in mats:
            marlin_gemm_fp4_cpu(a, p, s, G)
        steps += 1
        elapsed = time.perf_counter() - t0
        # a bounded sample of at least ~10 s of CPU work (and at least 3 steps)
        if (elapsed >= 10.0 and steps >= 3) or elapsed > budget_s:
            break
    dt = (time.perf_counter() - t0) / steps
    step_bytes = sum(alg_bytes(1, K, N) for _, K, N in LLAMA_LAYER)
    return {"value": round(step_bytes / dt / 1e12, 6), "unit": "TB/s", "cores": cores,
            "kind": "port", "ms_per_step": round(dt * 1e3, 1),
            "cpu_model": cpu_model_name(),
            "sample": f"{steps} step(s) of the 4-GEMM Llama-3-8B layer at M=1 "
                      f"(torch-CPU fp32 dequant+matmul)"}


def pmc_probe(torch, mmfp4) -> int:
    """Dispatches whose hardware counters calibrate and measure HBM traffic:
    one copy of 512 MiB (known: 512 MiB read + 512 MiB written), then every
    Llama-layer GEMM at M=1 on 4 rotated weight copies x 5, then the two
    M=2048 prefill GEMMs x 2, then the MoE MLP at T=32 and T=1024 x 2."""
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for _, K, N in LLAMA_LAYER:
        ws = [make_weights(torch, mmfp4, K, N, 300 + c) for c in range(4)]
        a = torch.randn((1, K), device="cuda").half()
        for _ in range(5):
            for w in ws:
                mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
        torch.cuda.synchronize()
        del ws
    for _, K, N in PREFILL:
        w = make_weights(torch, mmfp4, K, N, 400)
        a = torch.randn((2048, K), device="cuda").half()
        for _ in range(2):
            mmfp4.marlin_gemm_fp4(a, w[0], w[1], G)
        torch.cuda.synchronize()
    # MoE (config 5) at T=32 and T=1024, two calls each on one weight set.
    E, H, I, k = MOE["E"], MOE["H"], MOE["I"], MOE["k"]
    gen = torch.Generator(device="cuda").manual_seed(600)
    gu_p = torch.randint(-2**31, 2**31 - 1, (E, H // 8, 2 * I), generator=gen, dtype=torch.int32,
                         device="cuda")
    gu_s = (torch.rand((E, H // G, 2 * I), generator=gen, device="cuda") * 0.01).half()
    dn_p = torch.randint(-2**31, 2**31 - 1, (E, I // 8, H), generator=gen, dtype=torch.int32,
                         device="cuda")
    dn_s = (torch.rand((E, I // G, H), generator=gen, device="cuda") * 0.01).half()
    for T in (32, 1024):
        p, ids = torch.topk(torch.softmax(torch.randn((T, E), generator=gen, device="cuda"), -1),
                            k, -1)
        x = torch.randn((T, H), generator=gen, device="cuda").half()
        for _ in range(2):
            mmfp4.moe_mlp_fp4(x, gu_p, gu_s, dn_p, dn_s, ids, p / p.sum(-1, keepdim=True), G)
        torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": "done"}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--all", action="store_true", help="accepted for compatibility; every "
                    "BASELINE config is reported by default")
    ap.add_argument("--section", choices=("all", "layer", "prefill", "moe", "fused", "graph",
                                          "read_sweep"),
                    default="all",
                    help="run one workload alone (for profiling); the default runs all and "
                         "prints the contract line")
    ap.add_argument("--layer-m", type=int, default=1,
                    help="rows of the layer GEMMs for --section layer (1: the metric's "
                         "workload; 8, 16, 32: the other decode sizes of config 2 and 3)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="no timing: run a 512 MiB copy (counter calibration) then the M=1 layer "
                         "GEMMs and the M=2048 prefill GEMMs, for rocprofv3 --pmc runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the FP4 dequant-GEMM "
                          "path runs on a single GPU (column- or expert-sharded multi-GPU "
                          "runs are not part of it); run with --gpus 1"}))
        return 2

    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device visible"}))
        return 1
    import mmfp4

    if args.pmc_probe:
        return pmc_probe(torch, mmfp4)
    torch.cuda.synchronize()
    if args.section != "all":
        # One workload alone, for a clean rocprofv3 kernel trace of it.
        if args.section == "layer":
            r = run_layer_bench(torch, mmfp4, args.layer_m, args.steps, args.warmup)
            res = {"us_per_step": round(1e3 * r["ms_per_step"], 3), "per_shape": r["per_shape"],
                   "TBps": round(r["step_bytes"] / (r["ms_per_step"] * 1e-3) / 1e12, 4)}
        elif args.section == "prefill":
            r = run_prefill_bench(torch, mmfp4, 2048, *prefill_steps(args))
            tf = r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12
            res = {"ms_per_step": round(r["ms_per_step"], 4), "per_shape": r["per_shape"],
                   "TFLOPs": round(tf, 1), "mfma_ceiling": run_mfma_ceiling(torch, mmfp4, tf)}
        elif args.section == "read_sweep":
            res = run_read_sweep(torch)
        elif args.section == "graph":
            res = run_layer_graph(torch, mmfp4, 200)
        elif args.section == "moe":
            res = [run_moe_bench(torch, mmfp4, T, 20) for T in (32, 1024)]
        else:
            res = run_fused_bench(torch, mmfp4, 100)
        print(json.dumps({"section": args.section, "result": res}))
        return 0
    layer = run_layer_bench(torch, mmfp4, 1, args.steps, args.warmup)
    pre = run_prefill_bench(torch, mmfp4, 2048, *prefill_steps(args))
    value_tbs = layer["step_bytes"] / (layer["ms_per_step"] * 1e-3) / 1e12
    achieved = layer["step_bytes"] / 4 / (layer["launch_us_avg"] * 1e-6) / 1e9
    tflops = pre["flops"] / (pre["ms_per_step"] * 1e-3) / 1e12
    out = {
        "metric": "FP4 dequant-GEMM: achieved HBM TB/s at M=1; TFLOP/s at M=2048",
        "value": round(value_tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(layer["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4(e2m1,g128) x fp16 -> fp32 acc",
        "data": "synthetic: weights N(0,0.02) fp16 quantized by the library's FP4 quantizer "
                "(g=128), activations N(0,1) fp16, seeded",
        "config": {"workload": "llama3-8b-layer-fp4-decode-M1", "M": 1, "group_size": G,
                   "layers": {n: [K, N] for n, K, N in LLAMA_LAYER},
                   "weight_copies_rotated": layer["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("k_skinny_llama3_layer_m1.md"),
                     "traffic_source": "profiles/k_skinny_llama3_layer_m1.md",
                     "kernel": "k_skinny + k_skinny_dual (M<=16 decode path, 4 launches per layer)",
                     "launch_us_avg": round(layer["launch_us_avg"], 3)},
        "per_shape_m1": layer["per_shape"],
        "prefill_m2048": {"tflops": round(tflops, 1), "frac_fp16_peak": round(tflops /
                          FP16_PEAK_TFLOPS, 4), "ms_per_step": round(pre["ms_per_step"], 4),
                          "per_shape": pre["per_shape"], "kernel": "k_prefill2 (MFMA 32x32x16, global->LDS pipeline)"},
    }
    ceil = run_read_ceiling(torch, args.steps, args.warmup)
    ceil["layer_time_fraction"] = round(ceil["layer_us"] / (1e3 * layer["ms_per_step"]), 4)
    out["hbm_read_ceiling_m1"] = ceil
    out["config1_single_linear_m1"] = run_single_bench(torch, mmfp4, 1, 4096, 4096, 100)
    out["north_star_decode_m1"] = run_north_star_decode(torch, mmfp4, 100)
    out["host_paced_per_call"] = run_host_paced(torch, mmfp4)
    out["config5_moe_qwen3_30b_a3b"] = [run_moe_bench(torch, mmfp4, T, 20) for T in (32, 1024)]
    out["prefill_m2048"]["hipblaslt_fp16_same_shapes"] = hipblaslt_fp16_reference(torch, 2048)
    out["prefill_m2048"]["mfma_ceiling"] = run_mfma_ceiling(torch, mmfp4, tflops)
    out["fused_next_rows"] = run_fused_bench(torch, mmfp4, 100)
    if True:   # the other BASELINE configs (2 at M=8/32, 3, 4 at M=512/8192), reported beside
        extra = {}
        for M in (8, 32):
            r = run_layer_bench(torch, mmfp4, M, max(20, args.steps // 4), 5)
            extra[f"fp4_layer_M{M}"] = {"TBps": round(r["step_bytes"] / (r["ms_per_step"] * 1e-3)
                                                      / 1e12, 3), "per_shape": r["per_shape"]}
        for M in (1, 16):
            r = run_layer_bench(torch, mmfp4, M, max(20, args.steps // 4), 5, int4=True)
            extra[f"int4_layer_M{M}"] = {"TBps": round(r["step_bytes"] / (r["ms_per_step"] * 1e-3)
                                                       / 1e12, 3), "per_shape": r["per_shape"]}
        for M in (512, 8192):
            r = run_prefill_bench(torch, mmfp4, M, 5, 2)
            extra[f"prefill_M{M}"] = {"TFLOPs": round(r["flops"] / (r["ms_per_step"] * 1e-3)
                                                      / 1e12, 1), "per_shape": r["per_shape"]}
        out["other_baseline_configs"] = extra
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
