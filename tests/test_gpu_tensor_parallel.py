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
