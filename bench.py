"""Benchmark of the TriAttention KV-compression step on one MI355X.

A step is one batched pass of the hot path over the whole synthetic batch:
phase table -> paged-K scoring of the sampled layers -> head statistics ->
aggregate -> keep-set selection -> K/V compaction of every layer -> block-table
rewrite.  Inputs are resident in HBM before timing starts.

Default workload: Qwen2.5-14B-shaped cache (48 layers, 40 query / 8 KV heads,
head_dim 128, bf16), 16 sequences x 16384 tokens in randomly permuted
128-token pages, budget 4096, recent window 128, score-layer stride 8.

Prints one JSON line: tokens/s (value), the compaction kernel's achieved HBM
bandwidth against MI355X peak (roofline), per-stage times, and the CPU
baseline (the oracle's torch restatement of the reference path, timed on a
bounded one-sequence sample on this host).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "vllm-ascend-kvcompress-hust_amd"))

HBM_PEAK_GBS = 8000.0
# KV pool of the default workload as a serving deployment sizes it: most of
# the 288 GB left after a 14B model's weights, 2 GiB per layer and K/V buffer
# (192 GiB over 48 layers), with the batch's pages scattered through it.  The
# bench measures the workload's own pool first and this one second.
SERVING_POOL_PAGES = {2: 8192}


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", type=int, default=2, help="workload configuration 1-5")
    p.add_argument("--layers", type=int, default=None, help="override the materialised layer count")
    p.add_argument(
        "--pool-pages",
        type=int,
        default=0,
        help="pages per layer and K/V buffer of the KV pool; 0 (default) = exactly the pages the workload names "
        "(the Qwen2.5-14B 16x16384 workload: 2048 source + 512 destination pages), larger = a bigger pool with "
        "the workload's pages scattered through it at random",
    )
    p.add_argument(
        "--serving-pool-pages",
        type=int,
        default=None,
        help="after the main measurement, measure the same workload again in a pool of this many pages per "
        "buffer and report it beside the main figure (default: 8192 = 2 GiB per buffer for the Qwen2.5-14B "
        "16x16384 workload, the size a serving deployment of a 14B model gives its KV pool; 0 = skip)",
    )
    p.add_argument(
        "--arena",
        action="store_true",
        help="carve every layer's K and V pool out of one allocation instead of one allocation each",
    )
    p.add_argument(
        "--graph",
        action="store_true",
        help="capture the step once as a HIP graph and time its replays (small batches are launch-bound)",
    )
    p.add_argument(
        "--restore-front",
        action="store_true",
        help="in-place workloads: before every step, restore the original contents of the pages that "
        "compaction overwrites (outside the timed region; each step is timed with HIP events), so every "
        "step is a first compaction of the same cache instead of a re-compaction of its own output",
    )
    p.add_argument(
        "--score-aggregation",
        choices=("mean", "max"),
        default="mean",
        help="aggregation of the rotary score over the future offsets (the reference's score_aggregation option)",
    )
    p.add_argument(
        "--compaction-order",
        choices=("auto", "layer_major", "interleaved"),
        default="auto",
        help="compaction layer order: auto (time both on the cache, keep the faster) or a fixed one",
    )
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument(
        "--cpu-repeats",
        type=int,
        default=12,
        help="timed repetitions of the CPU baseline's one-sequence sample after one warm-up (about 10 s of host "
        "work on the default workload)",
    )
    p.add_argument(
        "--calibration",
        action="store_true",
        help="only measure calibration statistics (kvc_qstats_accumulate) over a Qwen2.5-14B-shaped calibration "
        "pass: 48 layers of 4096-token bf16 query projections (40 heads x 128), one buffer per layer",
    )
    p.add_argument(
        "--kernel-micro",
        action="store_true",
        help="only measure the reference's NPU kernel micro-benchmark shapes (tests/run_npu_kernel_benchmark.py): "
        "2176 bf16 tokens, budget 2048, 8 KV heads x 5 query heads, head_dim 128, 12 offsets at round start "
        "8192, 6 sampled layers; copy, score, phase, aggregate and position-shift calls one by one",
    )
    p.add_argument(
        "--no-other-configs",
        action="store_true",
        help="default workload only: skip the Qwen3.5 hybrid and 4 x 131072 in-place entries of other_configs",
    )
    p.add_argument(
        "--tp-rank-scorer",
        action="store_true",
        help="only measure the one-layer scorer on one tensor-parallel rank's share of a Qwen3.5-35B-A3B cache: "
        "1 KV head, 8 query heads, head_dim 256 with 64 rotary dims, 32768 bf16 tokens in contiguous 128-token "
        "pages, 16 offsets at round start 65536 (the shape of the reference's partial-RoPE scorer benchmark, "
        "tests/run_npu_partial_rope_benchmark.py)",
    )
    return p.parse_args()


# Calls recorded back to back in one HIP graph when a small call's device
# time is measured: a graph launch costs about 7 us on this platform
# whatever the graph holds (one call per graph: 20.6 us for a call whose two
# kernels run 13.8 us), so the per-call figure divides one replay of many
# calls by their count.
CALLS_PER_GRAPH = 16


def graph_ms_per_call(fn, replays: int, calls: int = CALLS_PER_GRAPH) -> float:
    """Device time of one ``fn()`` call: ``calls`` calls captured back to back
    as one HIP graph on a side stream, ``replays`` replays timed with HIP
    events on the replay stream, divided by replays x calls."""
    import torch

    device = torch.cuda.current_device()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=side):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * calls)


def tp_rank_scorer_bench(steps: int, warmup: int, cpu_repeats: int, no_cpu: bool) -> int:
    """kvc_score_paged (through the reference-named wrapper
    score_paged_keys_mean_precomputed) on one rank's share of a Qwen3.5 cache:
    inputs drawn as the reference's benchmark draws them
    (tests/run_npu_partial_rope_benchmark.py:35-96).  Algorithmic bytes = the
    keys read once, 32768 x 256 x 2 B = 16.8 MB per call."""
    import torch

    from kvcompress_mi355x.methods.triattention import kernels

    device = torch.device("cuda:0")
    tokens, block, rotary, head_dim, kv_heads, qpk = 32768, 128, 64, 256, 1, 8
    freq = rotary // 2
    round_start = 65536
    g = torch.Generator(device=device).manual_seed(20260927)
    cache = torch.randn(tokens // block, block, kv_heads, head_dim, generator=g, device=device).to(torch.bfloat16)
    blocks = torch.arange(tokens // block, dtype=torch.int64, device=device)
    shape = (kv_heads, qpk, freq)
    q_real = torch.randn(shape, generator=g, device=device)
    q_imag = torch.randn(shape, generator=g, device=device)
    q_abs = torch.sqrt(q_real.square() + q_imag.square()) + 0.1
    q_pass = torch.randn(kv_heads, qpk, head_dim - rotary, generator=g, device=device)
    scale = torch.ones(shape, device=device)
    omega = torch.logspace(0, -4, freq, device=device)
    offsets = torch.arange(1, 17, dtype=torch.float32, device=device)
    phase = (offsets[:, None] + round_start) * omega[None, :]
    phase_cos = torch.cos(phase).mean(dim=0)
    phase_sin = torch.sin(phase).mean(dim=0)
    extra = q_abs - torch.sqrt(q_real.square() + q_imag.square() + 1e-8)
    out = torch.empty(kv_heads, qpk, tokens, dtype=torch.float32, device=device)

    def call() -> None:
        kernels.score_paged_keys_mean_precomputed(
            cache, blocks, q_real, q_imag, scale, extra, phase_cos, phase_sin, tokens, out, block, "half",
            q_pass_mean=q_pass, rotary_dim=rotary,
        )

    for _ in range(max(1, warmup)):
        call()
    torch.cuda.synchronize()
    # Wall time per eager call, as the reference's benchmark times its fused
    # kernel (host-bound at this size: the GPU work is shorter than the call).
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    torch.cuda.synchronize()
    wall_ms = 1000.0 * (time.perf_counter() - t0) / steps
    # Device time per call without the host: calls back to back in one HIP
    # graph (each call two launches, weight fold and scorer); and one call
    # per graph, which adds the graph launch to every call.
    device_ms = graph_ms_per_call(call, max(1, steps // CALLS_PER_GRAPH))
    single_graph_ms = graph_ms_per_call(call, steps, calls=1)
    nbytes = tokens * kv_heads * head_dim * 2
    result = {
        "metric": "one-layer scorer, tokens scored/s on one tensor-parallel rank's Qwen3.5 cache share; HBM GB/s",
        "value": round(tokens / (device_ms / 1000.0), 1),
        "unit": "tokens/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(device_ms, 5),
        "timing": f"ms_per_step and value: device time per call, {CALLS_PER_GRAPH} calls back to back in one HIP "
        "graph; one_call_per_graph_ms: one call per graph replay (adds the graph launch); wall_ms_per_call: "
        "eager calls",
        "one_call_per_graph_ms": round(single_graph_ms, 5),
        "wall_ms_per_call": round(wall_ms, 5),
        "higher_is_better": True,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "qwen3.5-35b-a3b-tp-rank-scorer-32768",
            "tokens": tokens, "kv_heads": kv_heads, "query_heads": kv_heads * qpk, "head_dim": head_dim,
            "rotary_dim": rotary, "offsets": 16, "round_start": round_start, "layers": 1,
        },
        "roofline": {
            "kernel": "kvc_score_paged (weight fold + scorer launches)",
            "bound": "hbm",
            "achieved": round(nbytes / (device_ms / 1000.0) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(nbytes / (device_ms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes,
            "timing": f"HIP events around replays of a graph of {CALLS_PER_GRAPH} calls on the replay stream",
        },
    }
    if not no_cpu:
        from oracle import triattention_ref as ref

        threads, thread_info = cpu_threads()
        torch.set_num_threads(threads)
        stats = ref.LayerStats(
            q_mean_real=q_real.cpu(), q_mean_imag=q_imag.cpu(), q_abs_mean=q_abs.cpu(),
            freq_scale_sq=scale.square().cpu(), omega=omega.cpu(), rope_style="half", rotary_dim=rotary,
            q_pass_mean=q_pass.cpu(),
        )
        host_cache, host_blocks, host_offsets = cache.cpu(), blocks.cpu(), offsets.cpu()
        reference = torch.empty(kv_heads, qpk, tokens, dtype=torch.float32)

        def generic() -> float:
            t = time.perf_counter()
            for s0 in range(0, tokens, 8192):
                count = min(8192, tokens - s0)
                keys = ref.gather_paged_range(host_cache, host_blocks, start=s0, count=count, block_size=block)
                reference[..., s0 : s0 + count] = ref.score_post_rope_keys(
                    keys, stats, round_start=round_start, offsets=host_offsets, aggregation="mean"
                )
            return time.perf_counter() - t

        generic()
        med = statistics.median(generic() for _ in range(cpu_repeats))
        hip = out.cpu()
        err = ((hip - reference).abs() / (reference.abs() + reference.square().mean(dim=-1, keepdim=True).sqrt())).max()
        result["cpu_baseline"] = {
            "value": round(tokens / med, 1),
            "unit": "tokens/s",
            "cores": threads,
            **thread_info,
            "kind": "port",
            "sample": f"the whole call: the torch restatement of score_post_rope_keys over 8192-token gathered chunks "
            f"(the reference benchmark's fallback path); median of {cpu_repeats} after 1 warm-up; "
            f"max |err| / (|ref| + rms) of the HIP scores against it {float(err):.2e}; host CPU {cpu_model()}",
        }
        result["speedup_vs_cpu_baseline"] = {
            "device": round(med * 1000.0 / device_ms, 1),
            "wall_per_eager_call": round(med * 1000.0 / wall_ms, 1),
        }
    print(json.dumps(result), flush=True)
    return 0


def calibration_bench(steps: int, warmup: int, cpu_repeats: int, no_cpu: bool) -> int:
    """Calibration statistics of one Qwen2.5-14B-shaped calibration pass per
    step: every layer's projection [4096, 40*128] bf16 read once by
    kvc_qstats_accumulate (distinct buffers, 2.0 GB in all, so no layer is
    served from a cache); algorithmic bytes = the projections' bytes."""
    import torch

    from kvcompress_mi355x.calibration import LayerAccumulator

    layers, tokens, heads, head_dim = 48, 4096, 40, 128
    device = torch.device("cuda:0")
    g = torch.Generator(device=device).manual_seed(0)
    projections = [torch.randn(tokens, heads * head_dim, generator=g, device=device).to(torch.bfloat16) for _ in range(layers)]
    accs = [LayerAccumulator(device=device) for _ in range(layers)]

    def step() -> None:
        for acc, q in zip(accs, projections):
            acc.add(q, heads, head_dim, head_dim)

    for _ in range(max(1, warmup)):
        step()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    # Kernel time without the host's per-call work: the pass captured as one
    # HIP graph (96 launches) and replayed.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=side):
        step()
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    device_ms = start.elapsed_time(end) / steps
    nbytes = layers * tokens * heads * head_dim * 2
    result = {
        "metric": "calibration query statistics: projection tokens x layers / s; HBM GB/s",
        "value": round(layers * tokens / wall, 1),
        "unit": "token-layers/s",
        "steps": steps,
        "ms_per_step": round(1000 * wall, 4),
        "graph_replay_ms_per_step": round(device_ms, 4),
        "launch": "eager per-layer calls (value); roofline from one HIP graph of the pass",
        "dtype": "bf16",
        "config": {"workload": "qwen2.5-14b-calibration-pass", "layers": layers, "tokens": tokens, "heads": heads, "head_dim": head_dim},
        "roofline": {
            "kernel": "kvc_qstats_accumulate",
            "bound": "hbm",
            "achieved": round(nbytes / (device_ms / 1000) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(nbytes / (device_ms / 1000) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes,
        },
    }
    if not no_cpu:
        from oracle import calibration_ref as cref

        threads, thread_info = cpu_threads()
        torch.set_num_threads(threads)
        sample = [q.cpu() for q in projections[:4]]

        def cpu_step() -> float:
            t = time.perf_counter()
            for q in sample:
                cref.QueryStatsAccumulator().add(q, heads, head_dim, head_dim)
            return time.perf_counter() - t

        cpu_step()
        med = statistics.median(cpu_step() for _ in range(cpu_repeats))
        result["cpu_baseline"] = {
            "value": round(len(sample) * tokens / med, 1),
            "unit": "token-layers/s",
            "cores": threads,
            **thread_info,
            "kind": "port",
            "sample": f"4 of 48 layers ({tokens} tokens each), torch float32 restatement; median of {cpu_repeats}",
        }
    print(json.dumps(result), flush=True)
    return 0


def kernel_micro_bench(steps: int, warmup: int, cpu_repeats: int, no_cpu: bool) -> int:
    """The reference's NPU kernel micro-benchmark (tests/run_npu_kernel_benchmark.py:44-282)
    on the same shapes and through the same wrapper names: one 2176-token
    bf16 sequence (8 KV heads x 5 query heads, head_dim 128) in 17
    contiguous pages, budget 2048, 12 offsets at round start 8192, 6 sampled
    layers for the phase preparation.  Each call is timed as the reference
    times it (wall clock over eager calls after warm-up) and as device time
    (the call captured once as a HIP graph, replays timed with HIP events);
    beside it the oracle's torch path for the same call on the host CPU."""
    import torch

    from kvcompress_mi355x.methods.triattention import cache as kcache
    from kvcompress_mi355x.methods.triattention import kernels

    device = torch.device("cuda:0")
    block, tokens, budget, kv_heads, qpk, head_dim, n_blocks = 128, 2176, 2048, 8, 5, 128, 32
    g = torch.Generator(device=device).manual_seed(20260401)
    k_cache = torch.randn(n_blocks, block, kv_heads, head_dim, generator=g, device=device).to(torch.bfloat16)
    v_cache = torch.randn(n_blocks, block, kv_heads, head_dim, generator=g, device=device).to(torch.bfloat16)
    source = torch.arange(-(-tokens // block), device=device, dtype=torch.int64)
    destination = source[: budget // block]
    keep = torch.arange(budget, device=device, dtype=torch.int64) + (tokens - budget)
    k_ws = torch.empty(budget, kv_heads, head_dim, device=device, dtype=torch.bfloat16)
    v_ws = torch.empty_like(k_ws)
    src_slots = kcache.token_slots(source, keep, block)
    dst_slots = kcache.token_slots(destination, torch.arange(budget, device=device, dtype=torch.int64), block)
    freq = head_dim // 2
    shape = (kv_heads, qpk, freq)
    q_real = torch.randn(shape, generator=g, device=device)
    q_imag = torch.randn(shape, generator=g, device=device)
    q_abs = torch.sqrt(q_real.square() + q_imag.square()) + 0.2
    scale = torch.ones(shape, device=device)
    omega = torch.logspace(0, -4, freq, device=device)
    offsets = torch.tensor([1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048], device=device, dtype=torch.float32)
    extra = q_abs - torch.sqrt(q_real.square() + q_imag.square() + 1e-8)
    out = torch.empty(kv_heads, qpk, tokens, device=device, dtype=torch.float32)
    off_cos = torch.cos(offsets.unsqueeze(1) * omega).mean(dim=0)
    off_sin = torch.sin(offsets.unsqueeze(1) * omega).mean(dim=0)
    layers = 6
    layer_omega = omega.unsqueeze(0).expand(layers, -1).contiguous()
    layer_cos = off_cos.unsqueeze(0).expand(layers, -1).contiguous()
    layer_sin = off_sin.unsqueeze(0).expand(layers, -1).contiguous()
    phase_cos, phase_sin = torch.empty_like(layer_omega), torch.empty_like(layer_omega)
    kernels.prepare_mean_phase_coefficients(layer_omega, layer_cos, layer_sin, 8192, phase_cos, phase_sin)
    kernels.score_paged_keys_mean_precomputed(k_cache, source, q_real, q_imag, scale, extra, phase_cos[0], phase_sin[0],
                                              tokens, out, block, "half")
    head_mean = out.mean(dim=-1)
    head_var = out.var(dim=-1, correction=0)
    agg = torch.empty(tokens, device=device, dtype=torch.float32)
    positions = torch.arange(4096, device=device, dtype=torch.int64)
    req_idx = torch.arange(4096, device=device, dtype=torch.int64) % 16
    req_off = torch.arange(16, device=device, dtype=torch.int64) * 128
    physical = torch.empty_like(positions)

    calls = {
        "copy": lambda: kcache.materialize_selected_tokens(k_cache, v_cache, source, destination, keep, block),
        "copy_slots": lambda: kcache.materialize_token_slots(k_cache, v_cache, src_slots, dst_slots, k_ws, v_ws),
        "score": lambda: kernels.score_paged_keys_mean(k_cache, source, q_real, q_imag, scale, extra, omega, off_cos,
                                                       off_sin, 8192, tokens, out, block, "half"),
        "score_precomputed": lambda: kernels.score_paged_keys_mean_precomputed(
            k_cache, source, q_real, q_imag, scale, extra, phase_cos[0], phase_sin[0], tokens, out, block, "half"),
        "phase6": lambda: kernels.prepare_mean_phase_coefficients(layer_omega, layer_cos, layer_sin, 8192, phase_cos, phase_sin),
        "aggregate": lambda: kernels.aggregate_normalized_scores(out, head_mean, head_var, agg, tokens,
                                                                 layer_aggregation="mean", first_layer=True),
        "shift": lambda: kernels.shift_positions(positions, req_idx, req_off, physical),
    }
    row_bytes = kv_heads * head_dim * 2
    algo_bytes = {
        "copy": budget * row_bytes * 2 * 2, "copy_slots": budget * row_bytes * 2 * 2,
        "score": tokens * row_bytes, "score_precomputed": tokens * row_bytes,
        "aggregate": kv_heads * qpk * tokens * 4 + tokens * 4, "shift": 4096 * 8 * 3,
    }
    # materialize_selected_tokens checks its keep indices against the table on
    # the host (a device read), as the reference's does, so it cannot be
    # captured: its device time is taken around eager calls instead.
    eager_only = {"copy"}
    results = {}
    for name, fn in calls.items():
        for _ in range(max(1, warmup)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        wall_ms = 1000.0 * (time.perf_counter() - t0) / steps
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if name in eager_only:
            start.record()
            for _ in range(steps):
                fn()
            end.record()
        torch.cuda.synchronize()
        if name in eager_only:
            device_ms = start.elapsed_time(end) / steps
        else:
            device_ms = graph_ms_per_call(fn, max(1, steps // CALLS_PER_GRAPH))
        entry = {"wall_ms_per_call": round(wall_ms, 5), "device_ms_per_call": round(device_ms, 5)}
        if name in eager_only:
            entry["device_timing"] = "HIP events around eager calls (includes the host's per-call work)"
        if name in algo_bytes:
            entry["hbm_frac"] = round(algo_bytes[name] / (device_ms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4)
        results[name] = entry
    score_ms = results["score_precomputed"]["device_ms_per_call"]
    result = {
        "metric": "reference NPU kernel micro-benchmark shapes: tokens scored/s of one layer (precomputed phases); "
        "per-call times of every call",
        "value": round(tokens / (score_ms / 1000.0), 1),
        "unit": "tokens/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": score_ms,
        "higher_is_better": True,
        "dtype": "bf16",
        "data": "synthetic",
        "timing": "wall_ms_per_call: eager calls as tests/run_npu_kernel_benchmark.py times them; device_ms_per_call: "
        f"{CALLS_PER_GRAPH} calls back to back in one HIP graph, HIP events on the replay stream",
        "config": {"workload": "reference-kernel-micro-2176", "tokens": tokens, "budget": budget, "kv_heads": kv_heads,
                   "query_heads": kv_heads * qpk, "head_dim": head_dim, "offsets": 12, "round_start": 8192,
                   "sampled_layers": layers},
        "calls": results,
        "amortized_score_ms": round(score_ms + results["phase6"]["device_ms_per_call"] / layers, 5),
    }
    if not no_cpu:
        from oracle import triattention_ref as ref

        threads, thread_info = cpu_threads()
        torch.set_num_threads(threads)
        hk, hv = k_cache.cpu(), v_cache.cpu()
        hsrc, hdst, hkeep = source.cpu(), destination.cpu(), keep.cpu()
        stats = ref.LayerStats(q_mean_real=q_real.cpu(), q_mean_imag=q_imag.cpu(), q_abs_mean=q_abs.cpu(),
                               freq_scale_sq=scale.square().cpu(), omega=omega.cpu(), rope_style="half", rotary_dim=head_dim)
        hout, hmean, hvar = out.cpu(), head_mean.cpu(), head_var.cpu()
        hoffsets = offsets.cpu()
        hpos, hidx, hoff = positions.cpu(), req_idx.cpu(), req_off.cpu()
        generic = {
            "copy": lambda: ref.materialize_selected_tokens(hk, hv, hsrc, hdst, hkeep, block),
            "score": lambda: ref.score_post_rope_keys(
                ref.gather_paged_range(hk, hsrc, start=0, count=tokens, block_size=block), stats,
                round_start=8192, offsets=hoffsets, aggregation="mean"),
            "aggregate": lambda: torch.amax((hout - hmean.unsqueeze(-1)) * torch.rsqrt(hvar.unsqueeze(-1) + 1e-6), dim=(0, 1)),
            "shift": lambda: torch.sub(hpos, hoff.index_select(0, hidx)),
        }
        cpu = {}
        for name, fn in generic.items():
            fn()
            times = []
            for _ in range(cpu_repeats):
                t = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t)
            cpu[name] = round(1000.0 * statistics.median(times), 5)
        result["cpu_baseline"] = {
            "value": round(tokens / (cpu["score"] / 1000.0), 1),
            "unit": "tokens/s",
            "cores": threads,
            **thread_info,
            "kind": "port",
            "sample": f"the oracle's torch path for each call on the host CPU (generic functions of the reference "
            f"benchmark), median of {cpu_repeats} after 1 warm-up, ms per call: {cpu}; host CPU {cpu_model()}",
        }
    print(json.dumps(result), flush=True)
    return 0


def cpu_threads() -> tuple[int, dict]:
    """Host threads for a CPU baseline and how they were chosen: every core
    os.cpu_count() reports, capped by OMP_NUM_THREADS where that is set (a
    job scheduler that shares the host between GPUs exports each job's CPU
    share there, whatever the host's core count)."""
    count = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    threads = min(count, int(env)) if env and env.isdigit() and int(env) > 0 else count
    return threads, {
        "os_cpu_count": count,
        "threads_rule": "os.cpu_count()" if threads == count else f"capped by OMP_NUM_THREADS={env} (the job's CPU share)",
    }


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class FrontRestore:
    """Saved contents of the pages an in-place compaction overwrites (the
    first ceil(budget/128) pages of every source table, every layer, K and V);
    calling the object copies them back."""

    def __init__(self, cache, budget: int) -> None:
        import torch

        n_front = -(-budget // 128)
        self.pages = torch.cat([t[:n_front] for t in cache.source_tables])
        self.caches = [*cache.k_caches, *cache.v_caches]
        self.saved = [c.index_select(0, self.pages) for c in self.caches]

    def __call__(self) -> None:
        for c, s in zip(self.caches, self.saved):
            c.index_copy_(0, self.pages, s)


def time_steps(pipeline, batch, steps: int, warmup: int, graph: bool = False, restore=None) -> tuple[float, float | None]:
    """Wall time of exactly `steps` compression steps (synchronised on both
    sides), after `warmup` untimed ones, and the mean kvc_compact time inside
    those steps from HIP events recorded around each compaction launch on the
    stream it runs on (events made before the loop).  A step is
    pipeline.step's own sequence: select_step, compact, rewrite.  With `graph`,
    the step is captured once and each timed step is one replay (no events
    inside it: the compaction time is None).  With `restore`, it runs before
    every step outside the timing, and the time is the sum of the steps'
    HIP-event durations."""
    import torch

    def step(marks=None) -> None:
        pipeline.select_step(batch)
        if marks is not None:
            marks[0].record()
        pipeline.compact(batch)
        if marks is not None:
            marks[1].record()
        pipeline.rewrite(batch)

    if graph:
        replay = pipeline.capture(batch).replay
        for _ in range(warmup):
            replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, None
    compact_marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    compact_ms = lambda: sum(a.elapsed_time(b) for a, b in compact_marks) / steps  # noqa: E731
    if restore is not None:
        for _ in range(warmup):
            restore()
            step()
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        torch.cuda.synchronize()
        for (start, end), cm in zip(marks, compact_marks):
            restore()
            start.record()
            step(cm)
            end.record()
        torch.cuda.synchronize()
        return sum(start.elapsed_time(end) for start, end in marks) / 1000.0, compact_ms()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for cm in compact_marks:
        step(cm)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, compact_ms()


def stage_times(pipeline, batch, reps: int, restore=None) -> dict[str, float]:
    """Mean device time of each stage over `reps` steps, from HIP events
    created before the loop (outside the timed steps: creating events per step
    costs more host time than a small step's kernels)."""
    import torch

    names = ("score", "aggregate", "select", "compact", "rewrite")
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(reps)]
    torch.cuda.synchronize()
    for m in marks:
        pipeline.validate(batch)
        if restore is not None:
            restore()
        m[0].record()
        pipeline.score(batch)
        m[1].record()
        pipeline.aggregate(batch)
        m[2].record()
        pipeline.select(batch)
        m[3].record()
        pipeline.compact(batch)
        m[4].record()
        pipeline.rewrite(batch)
        m[5].record()
    torch.cuda.synchronize()
    return {n: statistics.mean(m[i].elapsed_time(m[i + 1]) for m in marks) for i, n in enumerate(names)}


def cpu_baseline(cache, spec, repeats: int, score_aggregation: str = "mean") -> dict:
    """Time the oracle (torch CPU restatement of the reference path) on one
    sequence: score the sampled layers, select, materialise every layer."""
    import torch

    from oracle import stats_ref
    from oracle import triattention_ref as ref

    threads, thread_info = cpu_threads()
    torch.set_num_threads(threads)
    b = 0
    n = spec.seq_lens[b]
    src = cache.source_tables[b]
    dst = cache.destination_tables[b] if cache.destination_tables is not None else src[: -(-spec.budget // 128)]
    pages = torch.cat([src, dst]).unique()
    remap = {int(p): i for i, p in enumerate(pages.tolist())}
    h_src = torch.tensor([remap[int(p)] for p in src.tolist()])
    h_dst = torch.tensor([remap[int(p)] for p in dst.tolist()])
    k_host = [k[pages].cpu() for k in cache.k_caches]
    v_host = [v[pages].cpu() for v in cache.v_caches]
    model = spec.model_shape()
    laid_out = stats_ref.layer_stats_for_device(
        cache.calibration.layers,
        cache.calibration.metadata,
        num_attention_heads=model.num_attention_heads,
        num_kv_heads=model.num_kv_heads,
        head_dim=model.head_dim,
        rotary_dim=model.effective_rotary_dim,
        rope_theta=model.rope_theta,
    )
    layer_stats = [laid_out[layer] for layer in spec.scoring_layers]
    cfg = ref.MethodConfig(
        budget=spec.budget, recent=spec.recent, prefix=spec.prefix, segments=spec.segments, policy=spec.policy,
        score_aggregation=score_aggregation, score_chunk_size=8192, score_layer_stride=spec.score_layer_stride,
    )
    offsets = ref.build_geometric_offsets(spec.max_model_len)

    def one() -> float:
        t = time.perf_counter()
        out = ref.method_select([k_host[l] for l in spec.scoring_layers], layer_stats, h_src, n, cache.round_starts[b], offsets, cfg)
        ref.method_compress(k_host, v_host, h_src, h_dst, out["keep"], spec.budget)
        return time.perf_counter() - t

    one()  # warm-up
    times = [one() for _ in range(repeats)]
    med = statistics.median(times)
    return {
        "value": round(n / med, 1),
        "unit": "tokens/s",
        "cores": threads,
        **thread_info,
        "kind": "port",
        "sample": (
            f"1 of {len(spec.seq_lens)} sequences ({n} tokens): score {len(spec.scoring_layers)} layers "
            f"(chunk 8192), select, materialise {spec.n_layers} layers; median of {repeats} after 1 warm-up; "
            f"{med:.2f} s per sequence; host CPU {cpu_model()}"
        ),
    }


def step_hbm(spec, ms_per_step: float) -> dict:
    algo = spec.algorithmic_bytes()
    gbs = algo["total"] / (ms_per_step / 1000.0) / 1e9
    return {"algorithmic_bytes": algo["total"], "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def measure(spec, args) -> dict:
    """Build the workload's cache and pipeline, time exactly args.steps steps
    (after args.warmup), then the per-stage pass; returns the figures and the
    cache (kept alive for the CPU baseline)."""
    import torch

    from kvcompress_mi355x import workloads

    device = torch.device("cuda:0")
    cache = workloads.build_synthetic_cache(spec, device, seed=0, arena=args.arena)
    pipeline, batch = workloads.build_pipeline(cache, score_aggregation=args.score_aggregation,
                                               compaction_order=getattr(args, "compaction_order", "auto"))
    restore = FrontRestore(cache, spec.budget) if args.restore_front else None
    # Pipeline set-up, untimed: the compaction form for this cache's
    # placement in HBM is chosen from timed trials of both forms.
    pipeline.select_step(batch)
    pipeline.settle_compaction(batch, repeat_in_place=True)  # in place: the front pages are restored below
    if restore is not None:
        restore()
    torch.cuda.synchronize()
    wall, timed_compact_ms = time_steps(pipeline, batch, args.steps, args.warmup, graph=args.graph, restore=restore)
    stage_ms = stage_times(pipeline, batch, max(1, min(args.steps, 20)), restore=restore)
    # The roofline's kernel time: events around kvc_compact inside the timed
    # steps (graph replays have none inside: the per-stage pass then).
    pool = cache.k_caches[0]
    return {
        "cache": cache,
        "ms_per_step": 1000.0 * wall / args.steps,
        "compact_ms": timed_compact_ms if timed_compact_ms is not None else stage_ms["compact"],
        "compact_timing": "HIP events around kvc_compact in the timed steps"
        if timed_compact_ms is not None
        else "HIP events around kvc_compact in the per-stage pass",
        "stages_ms": stage_ms,
        "compaction_form": pipeline.compaction_form.chosen,
        "kv_pool": ("one arena, per-layer K/V views" if args.arena else "one allocation per layer and K/V")
        + f", {pool.shape[0]} pages each ({pool.numel() * pool.element_size() / 2**30:.2f} GiB)"
        + (", workload pages scattered through it" if spec.permute_pages else ""),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU: the compression step has no cross-GPU work "
            f"(sequences shard across GPUs with no exchange); --gpus {args.gpus} is not supported",
            file=sys.stderr,
        )
        return 2
    import torch

    from kvcompress_mi355x import workloads

    if args.calibration:
        return calibration_bench(args.steps, args.warmup, args.cpu_repeats, args.no_cpu_baseline)
    if args.tp_rank_scorer:
        return tp_rank_scorer_bench(args.steps, args.warmup, args.cpu_repeats, args.no_cpu_baseline)
    if args.kernel_micro:
        return kernel_micro_bench(args.steps, args.warmup, args.cpu_repeats, args.no_cpu_baseline)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    overrides = {} if args.layers is None else {"n_layers": args.layers}
    if args.pool_pages:
        overrides["pool_pages"] = args.pool_pages
    spec = workloads.config_spec(args.config, **overrides)
    if args.restore_front and not spec.inplace:
        print("--restore-front applies to in-place workloads only", file=sys.stderr)
        return 2
    m = measure(spec, args)
    cache = m.pop("cache")
    tokens = spec.total_tokens
    algo = spec.algorithmic_bytes()
    compact_gbs = algo["compact"] / (m["compact_ms"] / 1000.0) / 1e9
    # HBM bytes per kvc_compact launch from rocprofv3 FETCH_SIZE / WRITE_SIZE
    # counter runs of this workload (a profiler run of its own, recorded in
    # profiles/), not measured in this process.
    traffic, traffic_source = None, None
    traffic_file = REPO / "profiles" / f"compact_traffic_config{args.config}.json"
    if traffic_file.is_file() and args.layers is None and not args.pool_pages:
        recorded = json.loads(traffic_file.read_text())
        traffic = recorded.get("bytes_per_launch")
        traffic_source = (
            f"profiles/{traffic_file.name}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this workload "
            f"(commit {recorded.get('commit', 'unrecorded')}), scaled by a 1 GiB copy; not measured in this process"
        )

    result = {
        "metric": "KV tokens scored+compacted/sec at 1 GPU; achieved HBM GB/s as % of peak",
        "value": round(tokens / (m["ms_per_step"] / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if spec.dtype == torch.bfloat16 else "fp16",
        "data": "synthetic",
        "config": {
            "workload": spec.name,
            "layers": spec.n_layers,
            "scoring_layers": len(spec.scoring_layers),
            "n_seq": len(spec.seq_lens),
            "tokens": tokens,
            "budget": spec.budget,
            "recent": spec.recent,
            "policy": spec.policy,
            "heads": f"{spec.num_attention_heads}q/{spec.num_kv_heads}kv",
            "head_dim": spec.head_dim,
            "compaction": "in-place" if spec.inplace else "private destinations",
            "kv_pool": m["kv_pool"],
            "compaction_form": m["compaction_form"],
            **({"compaction_order": args.compaction_order} if args.compaction_order != "auto" else {}),
            "launch": "one HIP graph per step" if args.graph else "kernel launches per step",
            **({"score_aggregation": "max"} if args.score_aggregation == "max" else {}),
            **(
                {"timing": "sum of per-step HIP-event times; overwritten front pages restored before each step, untimed"}
                if args.restore_front
                else {}
            ),
        },
        "roofline": {
            "kernel": "kvc_compact",
            "bound": "hbm",
            "achieved": round(compact_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(compact_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes": algo["compact"],
            "kernel_ms": round(m["compact_ms"], 4),
            "timing": m["compact_timing"],
        },
        "step_hbm": step_hbm(spec, m["ms_per_step"]),
        "stages_ms": {k: round(v, 4) for k, v in m["stages_ms"].items()},
        "score_gbs": round(algo["score"] / (m["stages_ms"]["score"] / 1000.0) / 1e9, 1),
    }
    serving = args.serving_pool_pages
    if serving is None:
        serving = SERVING_POOL_PAGES.get(args.config, 0) if args.layers is None and not args.pool_pages else 0
    if serving:
        # The same workload in a serving-sized pool, measured after the main
        # figure in a fresh allocation (the main cache is released first).
        del cache
        torch.cuda.empty_cache()
        sspec = workloads.config_spec(args.config, **{**overrides, "pool_pages": serving})
        sm = measure(sspec, args)
        cache = sm.pop("cache")
        result["serving_pool"] = {
            "kv_pool": sm["kv_pool"],
            "compaction_form": sm["compaction_form"],
            "value": round(tokens / (sm["ms_per_step"] / 1000.0), 1),
            "ms_per_step": round(sm["ms_per_step"], 4),
            "step_hbm_frac": step_hbm(sspec, sm["ms_per_step"])["frac"],
            "compact_ms": round(sm["compact_ms"], 4),
            "compact_frac": round(algo["compact"] / (sm["compact_ms"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
        }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cache, cache.spec, args.cpu_repeats, args.score_aggregation)
    if args.config == 2 and not args.no_other_configs and args.layers is None and not args.pool_pages:
        del cache
        torch.cuda.empty_cache()
        result["other_configs"] = other_configs(args)
    print(json.dumps(result), flush=True)
    return 0


# The reference's other headline shapes, measured after the default workload:
# the Qwen3.5-35B-A3B hybrid batch (partial RoPE, v3 quotas, 2048-token
# scheduler pages; tests/run_npu_partial_rope_benchmark.py:35-41,
# tests/run_npu_qwen35_transaction_benchmark.py:92) and 4 x 131072 tokens
# compacted in place in a full pool, each step a first compaction of the
# same cache (front pages restored between steps, untimed).
OTHER_CONFIGS = ((3, False), (4, True))
OTHER_STEPS, OTHER_WARMUP = 10, 2


def other_configs(args) -> list[dict]:
    import torch

    from kvcompress_mi355x import workloads

    entries = []
    for config, restore_front in OTHER_CONFIGS:
        spec = workloads.config_spec(config)
        sub = argparse.Namespace(**{**vars(args), "steps": OTHER_STEPS, "warmup": OTHER_WARMUP,
                                    "restore_front": restore_front, "graph": False, "arena": False})
        m = measure(spec, sub)
        del m["cache"]
        torch.cuda.empty_cache()
        algo = spec.algorithmic_bytes()
        entries.append({
            "workload": spec.name,
            "config": config,
            "tokens": spec.total_tokens,
            "n_seq": len(spec.seq_lens),
            "layers": spec.n_layers,
            "compaction": "in-place" if spec.inplace else "private destinations",
            "steps": OTHER_STEPS,
            "warmup": OTHER_WARMUP,
            "value": round(spec.total_tokens / (m["ms_per_step"] / 1000.0), 1),
            "unit": "tokens/s",
            "ms_per_step": round(m["ms_per_step"], 4),
            "step_hbm": step_hbm(spec, m["ms_per_step"]),
            "compaction_form": m["compaction_form"],
            "compact_roofline": {
                "kernel_ms": round(m["compact_ms"], 4),
                "achieved": round(algo["compact"] / (m["compact_ms"] / 1000.0) / 1e9, 1),
                "frac": round(algo["compact"] / (m["compact_ms"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
                "algorithmic_bytes": algo["compact"],
            },
            "stages_ms": {k: round(v, 4) for k, v in m["stages_ms"].items()},
            **({"timing": "sum of per-step HIP-event times; overwritten front pages restored before each step, untimed"}
               if restore_front else {}),
        })
    return entries


if __name__ == "__main__":
    sys.exit(main())
