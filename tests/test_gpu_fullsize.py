"""Parity at the benchmark workloads' full sizes (GPU).

Each test builds a workload at its benchmark shape on the device and runs the
batched step, then checks
  * one full-length sequence against the oracle (raw scores of every scoring
    layer, head statistics, aggregate, keep set up to near-ties), the other
    sequences' oracle runs being too slow for a test on the host;
  * for every sequence, properties that hold at any size, on the GPU's own
    aggregate: the keep row is budget strictly increasing indices inside the
    sequence, holds the protected prefix and recent window, keeps exactly each
    segment's quota (the v3 closed form of tri/selection.py:165-196, or
    budget - protected for the global policy), every kept score of a segment
    is >= every evicted one, and ties at the threshold go to the lowest
    indices;
  * compaction bit-exact in every layer, K and V: each destination row equals
    the source row its keep index names (in place: the source as it was
    before the step, from a snapshot of the pages the step overwrites);
  * the new block table and freed pages as the scheduler commit defines them.
"""

from __future__ import annotations

import gc

import pytest
import torch

from helpers import assert_agg_close, assert_keep_matches, assert_scores_close, oracle_layer_stats
from oracle import triattention_ref as ref

pytestmark = pytest.mark.gpu


def _segments(n: int, spec) -> list[tuple[int, int, int]]:
    """(start, stop, quota) of the selectable middle of a sequence."""
    p = min(spec.prefix, n)
    r = min(spec.recent, n - p)
    ms, mc = p, n - p - r
    if spec.policy != "v3":
        return [(ms, ms + mc, spec.budget - p - r)]
    evict = n - spec.budget
    out = []
    for k in range(spec.segments):
        start, stop = ms + mc * k // spec.segments, ms + mc * (k + 1) // spec.segments
        if stop <= start:
            out.append((start, stop, 0))
            continue
        removed = evict * (stop - ms) // mc - evict * (start - ms) // mc
        out.append((start, stop, max(0, stop - start - removed)))
    return out


def _check_selection(spec, batch, agg: torch.Tensor, keep: torch.Tensor) -> None:
    offset = 0
    for b, n in enumerate(batch.seq_lens_host):
        k = keep[b]
        a = agg[offset : offset + n]
        offset += n
        assert k.numel() == spec.budget
        assert bool((k[1:] > k[:-1]).all()) and int(k[0]) >= 0 and int(k[-1]) < n, f"seq {b}: keep not a sorted index set"
        p = min(spec.prefix, n)
        r = min(spec.recent, n - p)
        dev = k.device
        assert torch.equal(k[:p], torch.arange(p, device=dev)), f"seq {b}: protected prefix"
        if r:
            assert torch.equal(k[-r:], torch.arange(n - r, n, device=dev)), f"seq {b}: protected recent window"
        kept = torch.zeros(n, dtype=torch.bool, device=dev)
        kept[k] = True
        for start, stop, quota in _segments(n, spec):
            seg_kept = kept[start:stop]
            assert int(seg_kept.sum()) == quota, f"seq {b}: segment [{start}, {stop}) keeps {int(seg_kept.sum())}, quota {quota}"
            if quota == 0 or quota == stop - start:
                continue
            vals = a[start:stop]
            threshold = vals[seg_kept].min()
            assert bool(vals[~seg_kept].max() <= threshold), f"seq {b}: an evicted score exceeds a kept one"
            idx = torch.arange(start, stop, device=dev)
            tie_kept = idx[seg_kept & (vals == threshold)]
            tie_evicted = idx[~seg_kept & (vals == threshold)]
            if tie_evicted.numel():
                assert int(tie_evicted.min()) > int(tie_kept.max()), f"seq {b}: threshold ties not lowest-index first"


def _slots(table: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    return table[rows // 128] * 128 + rows % 128


def _front_snapshot(cache, spec):
    """Rows of the pages an in-place step overwrites, per (layer, kind, sequence)."""
    nb = -(-spec.budget // 128)
    out = {}
    for kind, caches in (("k", cache.k_caches), ("v", cache.v_caches)):
        for layer, c in enumerate(caches):
            rows = c.view(-1, spec.num_kv_heads, spec.head_dim)
            for b, src in enumerate(cache.source_tables):
                out[(kind, layer, b)] = rows[_slots(src, torch.arange(nb * 128, device=src.device))].clone()
    return out


def _check_compaction(cache, spec, keep: torch.Tensor, snapshot) -> None:
    nb = -(-spec.budget // 128)
    for b, src in enumerate(cache.source_tables):
        k = keep[b]
        dst = src[:nb] if spec.inplace else cache.destination_tables[b]
        dst_slots = _slots(dst, torch.arange(spec.budget, device=k.device))
        src_slots = _slots(src, k)
        from_front = k < nb * 128
        for kind, caches in (("k", cache.k_caches), ("v", cache.v_caches)):
            for layer, c in enumerate(caches):
                rows = c.view(-1, spec.num_kv_heads, spec.head_dim)
                want = rows[src_slots]
                if spec.inplace:
                    want[from_front] = snapshot[(kind, layer, b)][k[from_front]]
                assert torch.equal(rows[dst_slots], want), f"{kind.upper()} layer {layer} seq {b} differs"


def _check_tables(cache, spec, tables, freed) -> None:
    for b, src in enumerate(cache.source_tables):
        dst = None if spec.inplace else cache.destination_tables[b].tolist()
        want_table, want_freed = ref.rewrite_block_table(src.tolist(), dst, spec.budget)
        assert tables[b].cpu().tolist() == want_table
        assert freed[b].cpu().tolist() == want_freed


def _host_keys(cache, spec, b: int):
    """Host copies of sequence b's pages in the scoring layers (taken before
    the compaction, which may overwrite them) and its table into them."""
    src = cache.source_tables[b]
    pages = src.unique()
    remap = {int(p): i for i, p in enumerate(pages.tolist())}
    h_src = torch.tensor([remap[int(p)] for p in src.tolist()])
    return [cache.k_caches[layer][pages].cpu() for layer in spec.scoring_layers], h_src


def _oracle_sequence(cache, spec, pipeline, batch, b: int, host_keys) -> int:
    """Oracle on sequence b over its host key copies."""
    k_host, h_src = host_keys
    cfg = ref.MethodConfig(
        budget=spec.budget, recent=spec.recent, prefix=spec.prefix, segments=spec.segments, policy=spec.policy,
        score_aggregation=pipeline.score_aggregation, score_chunk_size=8192, score_layer_stride=spec.score_layer_stride,
    )
    n = spec.seq_lens[b]
    out = ref.method_select(
        k_host,
        oracle_layer_stats(cache.calibration, spec.model_shape(), spec.scoring_layers),
        h_src,
        n,
        cache.round_starts[b],
        ref.build_geometric_offsets(spec.max_model_len),
        cfg,
    )
    start = sum(spec.seq_lens[:b])
    h_q = spec.num_attention_heads
    head_mean, head_var = pipeline.head_statistics(batch)
    for s_idx in range(len(spec.scoring_layers)):
        got = pipeline.raw_scores()[s_idx, start : start + n, :h_q].t()
        assert_scores_close(got, out["raw"][s_idx].reshape(h_q, n))
        var, mean = out["stats"][s_idx]
        torch.testing.assert_close(head_mean[s_idx, b].cpu(), mean.reshape(-1), rtol=1e-4, atol=1e-4)
        torch.testing.assert_close(head_var[s_idx, b].cpu(), var.reshape(-1), rtol=1e-3, atol=1e-4)
    assert_agg_close(pipeline.agg[start : start + n], out["agg"])
    protected = torch.zeros(n, dtype=torch.bool)
    p = min(spec.prefix, n)
    r = min(spec.recent, n - p)
    protected[:p] = True
    if r:
        protected[n - r :] = True
    return assert_keep_matches(pipeline.keep[b], out["keep"], out["agg"], spec.budget, protected)


def _run_full(spec, hip_device, oracle_seqs, score_aggregation: str = "mean") -> None:
    from kvcompress_mi355x import workloads

    gc.collect()
    torch.cuda.empty_cache()  # earlier tests' cached blocks: these workloads take 60-120 GB
    print(f"full-size workload {spec.name}: {len(spec.seq_lens)} sequences, {spec.total_tokens} tokens, "
          f"{spec.n_layers} layers", flush=True)
    cache = workloads.build_synthetic_cache(spec, hip_device, seed=0)
    pipeline, batch = workloads.build_pipeline(cache, score_aggregation=score_aggregation)
    keep = pipeline.select_step(batch)
    host_keys = {b: _host_keys(cache, spec, b) for b in oracle_seqs}
    snapshot = _front_snapshot(cache, spec) if spec.inplace else None
    pipeline.compact(batch)
    tables, freed = pipeline.rewrite(batch)
    torch.cuda.synchronize()
    near = 0
    for b in oracle_seqs:
        near += _oracle_sequence(cache, spec, pipeline, batch, b, host_keys[b])
    assert near <= 8, f"{near} near-tie differences against the oracle"
    _check_selection(spec, batch, pipeline.agg, keep)
    _check_compaction(cache, spec, keep, snapshot)
    _check_tables(cache, spec, tables, freed)


def test_fullsize_qwen2_5_14b_16x16384(hip_device) -> None:
    from kvcompress_mi355x import workloads

    _run_full(workloads.config_spec(2), hip_device, oracle_seqs=(0, 15))


def test_fullsize_qwen3_5_hybrid_v3(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(3)
    longest = max(range(len(spec.seq_lens)), key=lambda i: spec.seq_lens[i])
    _run_full(spec, hip_device, oracle_seqs=(longest,))


def test_fullsize_inplace_4x131072(hip_device) -> None:
    from kvcompress_mi355x import workloads

    _run_full(workloads.config_spec(4), hip_device, oracle_seqs=(1,))


def test_fullsize_decode_batch_fp16(hip_device) -> None:
    from kvcompress_mi355x import workloads

    # Every triggered sequence at its full length; 12 of the 24 benchmark
    # layers materialised (two scoring layers) to leave room for the checks.
    _run_full(workloads.config_spec(5, n_layers=12), hip_device, oracle_seqs=(0,))


def test_fullsize_qwen3_5_hybrid_score_max(hip_device) -> None:
    from kvcompress_mi355x import workloads

    # score_aggregation="max" (19 offsets); the oracle's per-offset torch loop
    # runs on the shortest sequence.
    spec = workloads.config_spec(3)
    shortest = min(range(len(spec.seq_lens)), key=lambda i: spec.seq_lens[i])
    _run_full(spec, hip_device, oracle_seqs=(shortest,), score_aggregation="max")
