"""Tensor-parallel halves of the step on one GPU (GPU).

The reference's TP path (tri/method.py:316-322,447-461) shards KV heads: each
rank scores and normalises its own query heads, all ranks all-reduce the
per-layer head maxima with MAX, and every rank then selects on the same
aggregate and compacts its own heads.  Here two "ranks" are two pipelines over
disjoint KV-head shards of one workload on one GPU; the collective is replaced
in the test by an elementwise torch.maximum of the two ranks' layer scores
(exactly what all_reduce(MAX) computes).  Both ranks must produce the keep set
of the unsharded pipeline, an aggregate equal to its aggregate (bit for bit
when both shardings give every KV head the same tile schedule), and each
rank's compacted heads must equal the unsharded compaction's slice of heads.
"""

from __future__ import annotations

import pytest
import torch

from helpers import assert_agg_close, assert_keep_matches

pytestmark = pytest.mark.gpu


def _shard_pipeline(cache, spec, tables, heads: slice):
    from kvcompress_mi355x.methods.triattention.pipeline import CompressionPipeline, ScoringTables

    ks = [k[:, :, heads, :].contiguous() for k in cache.k_caches]
    vs = [v[:, :, heads, :].contiguous() for v in cache.v_caches]
    part = lambda x: None if x is None else x[:, heads].contiguous()  # noqa: E731
    shard_tables = ScoringTables(
        part(tables.q_real), part(tables.q_imag), part(tables.freq_scale), part(tables.extra), part(tables.q_pass),
        tables.omega, tables.offsets, tables.rotary_dim, tables.rope_style,
    )
    pipeline = CompressionPipeline(
        scoring_k_caches=[ks[layer] for layer in spec.scoring_layers],
        k_caches=ks,
        v_caches=vs,
        tables=shard_tables,
        budget=spec.budget,
        protected_prefix=spec.prefix,
        protected_recent=spec.recent,
        segments=spec.segments,
        policy=spec.policy,
        layer_aggregation="mean",
        max_seqs=len(spec.seq_lens),
        max_seq_len=max(spec.seq_lens),
        max_tokens=spec.total_tokens,
    )
    return pipeline, ks, vs


@pytest.mark.parametrize(
    "config, overrides, exact",
    [
        # 8 KV heads in two shards of 4: every head keeps its tile schedule.
        (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(8192, 5000), budget=2048), True),
        # Qwen3.5 shape, one KV head per rank as the reference benchmarks it.
        (3, dict(n_layers=4, seq_lens=(20000, 9000)), False),
    ],
    ids=["qwen2.5-14b-tp2", "qwen3.5-tp2"],
)
def test_kv_head_shards_reproduce_the_unsharded_step(hip_device, config, overrides, exact) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(config, **overrides)
    cache = workloads.build_synthetic_cache(spec, hip_device, seed=0)
    full, batch = workloads.build_pipeline(cache)
    half = spec.num_kv_heads // 2
    shards = [_shard_pipeline(cache, spec, full.tables, slice(r * half, (r + 1) * half)) for r in range(2)]

    # Unsharded reference step (the shards hold their own copies of the caches).
    keep_full = full.step(batch)[0].clone()
    agg_full = full.agg[: batch.total_tokens].clone()

    # Each rank's local layer scores; the group MAX stands in for all_reduce.
    local = []
    for pipeline, _, _ in shards:
        pipeline.validate(batch)
        pipeline.score(batch)
        local.append(pipeline.local_layer_scores(batch).clone())
    reduced = torch.maximum(local[0], local[1])
    near = 0
    for r, (pipeline, ks, vs) in enumerate(shards):
        calls = []

        def all_reduce_max(t: torch.Tensor) -> None:
            calls.append(tuple(t.shape))
            t.copy_(reduced)

        keep, tables, freed = pipeline.step_sharded(batch, all_reduce_max)
        # One collective per step, of [scoring layers, tokens] (tests/test_selection.py:199-280).
        assert calls == [(len(spec.scoring_layers), spec.total_tokens)]
        torch.cuda.synchronize()
        agg = pipeline.agg[: batch.total_tokens]
        if exact:
            assert torch.equal(agg, agg_full), f"rank {r}: aggregate differs from the unsharded step"
            assert torch.equal(keep, keep_full), f"rank {r}: keep set differs"
        else:
            assert_agg_close(agg, agg_full, rel=1e-5)
            offset = 0
            for b, n in enumerate(spec.seq_lens):
                protected = torch.zeros(n, dtype=torch.bool)
                protected[: spec.prefix] = True
                protected[n - spec.recent :] = True
                near += assert_keep_matches(keep[b], keep_full[b], agg_full[offset : offset + n].cpu(), spec.budget, protected)
                offset += n
        # This rank's compacted heads are the unsharded compaction's head slice.
        heads = slice(r * half, (r + 1) * half)
        for layer in range(spec.n_layers):
            same = torch.equal(keep, keep_full)
            if same:
                assert torch.equal(ks[layer], cache.k_caches[layer][:, :, heads, :]), f"rank {r} K layer {layer}"
                assert torch.equal(vs[layer], cache.v_caches[layer][:, :, heads, :]), f"rank {r} V layer {layer}"
    assert near <= 4


def _free_port() -> int:
    import socket

    with socket.socket(socket.AF_INET, socket.SOCK_STREAM) as s:
        s.bind(("127.0.0.1", 0))
        return int(s.getsockname()[1])


def test_method_with_tensor_parallel_ranks(hip_device, tmp_path) -> None:
    """TriAttentionMethod at tensor_parallel_size 2: two rank processes on this
    GPU, each bound to half of the KV heads, meet in one MAX all-reduce over a
    gloo group (tri/method.py:106-122,315-322,447-461).  Both must select the
    keep set of the unsharded method and compact their heads exactly as the
    unsharded compaction does."""
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path
    from types import SimpleNamespace

    from kvcompress_mi355x import workloads
    from kvcompress_mi355x.methods import create_method
    from kvcompress_mi355x.methods.base import CompressionRequest, LayerCache
    from kvcompress_mi355x.methods.triattention.cache import token_slots

    overrides = dict(n_layers=4, score_layer_stride=2, seq_lens=(8192,), budget=2048, recent=128, max_model_len=16384)
    spec = workloads.config_spec(2, **overrides)
    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    stats_path = tmp_path / "stats.pt"
    torch.save(
        {
            "metadata": dict(host.calibration.metadata),
            "layer_stats": {
                i: {
                    "q_mean_real": s.q_mean_real,
                    "q_mean_imag": s.q_mean_imag,
                    "q_abs_mean": s.q_abs_mean,
                    "freq_scale_sq": s.freq_scale_sq,
                }
                for i, s in host.calibration.layers.items()
            },
        },
        stats_path,
    )
    options = {"stats_path": str(stats_path), "kv_budget": 2048, "score_layer_stride": 2, "protected_recent_window": 128}
    job = tmp_path / "job.json"
    job.write_text(json.dumps({"config": 2, "overrides": overrides, "options": options}))

    # The two ranks, as separate processes sharing this GPU.
    world, port = 2, _free_port()
    worker = Path(__file__).resolve().parent / "tp_rank_worker.py"
    env = dict(os.environ, MASTER_ADDR="127.0.0.1")
    procs, logs = [], []
    for r in range(world):
        log = open(tmp_path / f"rank{r}.log", "w")
        logs.append(log)
        procs.append(subprocess.Popen(
            [sys.executable, "-u", str(worker), "--rank", str(r), "--world", str(world), "--port", str(port),
             "--job", str(job), "--out", str(tmp_path / f"rank{r}.pt")],
            stdout=log, stderr=subprocess.STDOUT, env=env,
        ))

    # Meanwhile the unsharded method on the full cache in this process.
    cache = workloads.move_cache(host, hip_device)
    vllm_config = SimpleNamespace(
        parallel_config=SimpleNamespace(tensor_parallel_size=1),
        model_config=SimpleNamespace(max_model_len=spec.max_model_len),
        speculative_config=None,
    )
    method = create_method("triattention", options, vllm_config, spec.model_shape())
    layers = tuple(LayerCache(f"model.layers.{i}.self_attn.attn", i, cache.k_caches[i], cache.v_caches[i]) for i in range(spec.n_layers))
    method.bind_model_runner(SimpleNamespace(device=hip_device), layers)
    src, dst = cache.source_tables[0], cache.destination_tables[0]
    n, rs = spec.seq_lens[0], host.round_starts[0]
    keep_full = method.select_keep_indices(src, n, rs).cpu()
    method.compress(CompressionRequest(
        request_id="r0", semantic_num_tokens=rs, physical_num_tokens=n,
        source_block_ids=(tuple(src.cpu().tolist()),), destination_block_ids=(tuple(dst.cpu().tolist()),),
        source_block_ids_device=src, destination_block_ids_device=dst,
    ))
    torch.cuda.synchronize()
    slots = token_slots(dst, torch.arange(spec.budget, device=hip_device), 128)
    k_full = torch.stack([k.view(-1, spec.num_kv_heads, spec.head_dim)[slots] for k in cache.k_caches]).cpu()
    v_full = torch.stack([v.view(-1, spec.num_kv_heads, spec.head_dim)[slots] for v in cache.v_caches]).cpu()

    for r, proc in enumerate(procs):
        try:
            rc = proc.wait(timeout=300)
        except subprocess.TimeoutExpired:
            for p in procs:
                p.kill()
            pytest.fail(f"rank {r} did not finish")
        logs[r].close()
        assert rc == 0, f"rank {r} failed:\n" + (tmp_path / f"rank{r}.log").read_text()[-3000:]
    local = spec.num_kv_heads // world
    for r in range(world):
        got = torch.load(tmp_path / f"rank{r}.pt", weights_only=True)
        assert got["budget"] == spec.budget
        assert torch.equal(got["keep"], keep_full), f"rank {r}: keep set differs from the unsharded method"
        heads = slice(r * local, (r + 1) * local)
        assert torch.equal(got["k"], k_full[:, :, heads]), f"rank {r}: compacted K differs"
        assert torch.equal(got["v"], v_full[:, :, heads]), f"rank {r}: compacted V differs"
