"""End-to-end parity of the batched compression step and the method API (GPU)."""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import assert_agg_close, assert_keep_matches, assert_scores_close, oracle_layer_stats
from oracle import triattention_ref as ref

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _oracle_for(host, spec, b, score_aggregation="mean", layer_aggregation="mean"):
    layer_stats = oracle_layer_stats(host.calibration, spec.model_shape(), spec.scoring_layers)
    cfg = ref.MethodConfig(
        budget=spec.budget, recent=spec.recent, prefix=spec.prefix, segments=spec.segments, policy=spec.policy,
        score_aggregation=score_aggregation, layer_aggregation=layer_aggregation,
        score_chunk_size=8192, score_layer_stride=spec.score_layer_stride,
    )
    return ref.method_select(
        [host.k_caches[layer] for layer in spec.scoring_layers],
        layer_stats,
        host.source_tables[b],
        spec.seq_lens[b],
        host.round_starts[b],
        ref.build_geometric_offsets(spec.max_model_len),
        cfg,
    )


def _protected(n, spec):
    mask = torch.zeros(n, dtype=torch.bool)
    p = min(spec.prefix, n)
    r = min(spec.recent, n - p)
    mask[:p] = True
    if r:
        mask[n - r :] = True
    return mask


def _run_and_check(spec, hip_device, *, check_layers=None, score_aggregation="mean", layer_aggregation="mean",
                   compaction_order="auto"):
    from kvcompress_mi355x import workloads

    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    cache = workloads.move_cache(host, hip_device)
    pipeline, batch = workloads.build_pipeline(
        cache, score_aggregation=score_aggregation, layer_aggregation=layer_aggregation,
        compaction_order=compaction_order,
    )
    keep, tables, freed = pipeline.step(batch)
    if compaction_order != "auto":
        assert pipeline.compaction_form.chosen == compaction_order
    torch.cuda.synchronize()
    offs = [0]
    for n in spec.seq_lens:
        offs.append(offs[-1] + n)
    h_q = spec.num_attention_heads
    near_ties = 0
    oracle_keeps = []
    head_mean, head_var = pipeline.head_statistics(batch)
    for b, n in enumerate(spec.seq_lens):
        out = _oracle_for(host, spec, b, score_aggregation, layer_aggregation)
        for s_idx in range(len(spec.scoring_layers)):
            got_raw = pipeline.raw_scores()[s_idx, offs[b] : offs[b + 1], :h_q].t()
            assert_scores_close(got_raw, out["raw"][s_idx].reshape(h_q, n))
            var, mean = out["stats"][s_idx]
            torch.testing.assert_close(head_mean[s_idx, b].cpu(), mean.reshape(-1), rtol=1e-4, atol=1e-4)
            torch.testing.assert_close(head_var[s_idx, b].cpu(), var.reshape(-1), rtol=1e-3, atol=1e-4)
        assert_agg_close(pipeline.agg[offs[b] : offs[b + 1]], out["agg"])
        near_ties += assert_keep_matches(keep[b], out["keep"], out["agg"], spec.budget, _protected(n, spec))
        oracle_keeps.append(out["keep"])
    # Compaction is bit-exact given the kernel's own keep set.
    layers = range(spec.n_layers) if check_layers is None else check_layers
    nb = -(-spec.budget // 128)
    for b in range(len(spec.seq_lens)):
        gkeep = keep[b].cpu()
        src = host.source_tables[b]
        dst = src[:nb] if spec.inplace else host.destination_tables[b]
        slots = ref.token_slots(src, gkeep, 128)
        for layer in layers:
            want_k = ref.gather_slots(host.k_caches[layer], slots)
            want_v = ref.gather_slots(host.v_caches[layer], slots)
            dslots = ref.token_slots(dst.to(hip_device), torch.arange(spec.budget, device=hip_device), 128)
            got_k = ref.gather_slots(cache.k_caches[layer], dslots).cpu()
            got_v = ref.gather_slots(cache.v_caches[layer], dslots).cpu()
            assert torch.equal(got_k, want_k), f"K layer {layer} seq {b}"
            assert torch.equal(got_v, want_v), f"V layer {layer} seq {b}"
        want_table, want_freed = ref.rewrite_block_table(src.tolist(), None if spec.inplace else dst.tolist(), spec.budget)
        assert tables[b].cpu().tolist() == want_table
        assert freed[b].cpu().tolist() == want_freed
    if cache.kv_buffers is not None:
        _assert_padding_untouched(cache)
    return pipeline, keep, oracle_keeps, near_ties


def _assert_padding_untouched(cache) -> None:
    """Every page's padding of the shared K/V buffers still holds its fill
    (NaN, compared bit for bit)."""
    from kvcompress_mi355x import workloads

    num_pages = int(cache.k_caches[0].shape[0])
    fill = torch.full((1,), workloads.PAD_VALUE, dtype=cache.spec.dtype).view(torch.int16)
    for layer, buf in enumerate(cache.kv_buffers):
        pad = workloads.padding_view(buf, num_pages, cache.spec)
        assert torch.equal(pad.view(torch.int16).cpu(), fill.expand_as(pad)), f"layer {layer} padding was written"


def test_config1_end_to_end(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(1)
    pipeline, keep, oracle_keeps, near = _run_and_check(spec, hip_device)
    assert near <= 2
    fixture = json.loads((GOLDEN / "config1_expected.json").read_text())
    assert fixture["keep_sha256"] is not None
    assert sorted(keep[0].cpu().tolist()) == keep[0].cpu().tolist()
    golden_keep = np.load(GOLDEN / "config1_keep.npy", allow_pickle=False)
    diff = set(keep[0].cpu().tolist()) ^ set(golden_keep.tolist())
    assert len(diff) <= 2 * near


def test_ragged_batch_private(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(
        2, n_layers=4, score_layer_stride=2, seq_lens=(4224, 5000, 8192, 4351), budget=4096, recent=128, max_model_len=32768
    )
    _run_and_check(spec, hip_device)


def test_partial_rope_v3_hybrid_pages(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(3, n_layers=4, seq_lens=(9000, 6000))
    _run_and_check(spec, hip_device)


def test_inplace_front_pages_with_outliers(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(4, n_layers=2, score_layer_stride=1, seq_lens=(12000, 20000), pool_pages=300, max_model_len=32768)
    _run_and_check(spec, hip_device)


@pytest.mark.parametrize(
    "config, overrides, layer_aggregation",
    [
        # 18 offsets: two 16-offset chunks, query heads split over two workgroups.
        (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(5000, 8192), budget=4096, max_model_len=131072), "max"),
        # Partial RoPE (F = 32), 19 offsets, v3 selection.
        (3, dict(n_layers=4, seq_lens=(9000, 6000)), "mean"),
        # fp16 keys, 16 offsets.
        (5, dict(n_layers=2, score_layer_stride=1, seq_lens=(4300, 7000)), "mean"),
    ],
    ids=["qwen2.5-14b-o18-layer-max", "qwen3.5-o19", "fp16-o16"],
)
def test_score_aggregation_max(hip_device, config, overrides, layer_aggregation) -> None:
    # score_aggregation="max" (tri/scoring.py:84-97) through the batched step.
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(config, **overrides)
    _, _, _, near = _run_and_check(spec, hip_device, score_aggregation="max", layer_aggregation=layer_aggregation)
    assert near <= 4


@pytest.mark.parametrize("score_aggregation", ["mean", "max"])
def test_vector_alu_scorer_shape(hip_device, score_aggregation) -> None:
    # head_dim 96 (F = 48): the vector-ALU scorers and token-major raw scores.
    from kvcompress_mi355x import _native, workloads

    spec = workloads.config_spec(
        2, n_layers=2, score_layer_stride=1, seq_lens=(3000, 4500), budget=1024, recent=64, head_dim=96, rotary_dim=96,
        num_attention_heads=12, num_kv_heads=4, max_model_len=65536,
    )
    assert _native.load().kvc_score_raw_layout(0, 0, 4, 96, 96, 3) == _native.RAW_TOKEN_MAJOR
    _, _, _, near = _run_and_check(spec, hip_device, score_aggregation=score_aggregation)
    assert near <= 4


def test_fp16_decode_shape(hip_device) -> None:
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(5, n_layers=2, score_layer_stride=1, seq_lens=(4300, 7000, 4224))
    _run_and_check(spec, hip_device)


@pytest.mark.parametrize("order", ["layer_major", "interleaved"])
def test_pinned_compaction_order(hip_device, order) -> None:
    """A pipeline whose compaction layer order is pinned runs no trials and
    compacts every layer bit-exactly in that order (private and in place)."""
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(2, n_layers=4, score_layer_stride=2, seq_lens=(4224, 6000), budget=2048, max_model_len=16384)
    _run_and_check(spec, hip_device, compaction_order=order)
    spec = workloads.config_spec(4, n_layers=2, score_layer_stride=1, seq_lens=(12000, 7000), pool_pages=200, max_model_len=32768)
    _run_and_check(spec, hip_device, compaction_order=order)


SHARED_BUFFER_CASES = [
    # (config, overrides, score aggregation); K and V interleaved in one buffer
    # per layer, pages padded by page_pad elements (a multiple of 8: 16 bytes).
    (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(4224, 6000), budget=2048, max_model_len=16384, page_pad=0), "mean"),
    (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(4224, 6000), budget=2048, max_model_len=16384, page_pad=8), "mean"),
    (5, dict(n_layers=2, score_layer_stride=1, seq_lens=(4300, 5000), page_pad=64), "mean"),
    (3, dict(n_layers=4, seq_lens=(9000, 6000), page_pad=8), "mean"),
    (4, dict(n_layers=2, score_layer_stride=1, seq_lens=(12000, 7000), pool_pages=200, max_model_len=32768, page_pad=8), "mean"),
    (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(5000, 4300), budget=2048, max_model_len=131072, page_pad=8), "max"),
]


@pytest.mark.parametrize(
    "config, overrides, score_aggregation",
    SHARED_BUFFER_CASES,
    ids=["bf16-pad0", "bf16-pad8", "fp16-pad64", "qwen3.5-v3-pad8", "inplace-pad8", "max-o18-pad8"],
)
def test_shared_kv_buffer_layouts(hip_device, config, overrides, score_aggregation) -> None:
    """The step on the reference's shared-buffer cache layout: K and V of a
    layer are interleaved views of one buffer, each page followed by its
    padding (tests/test_cache.py:50-94; pkg/provider.py:1201-1230).  Scores,
    statistics, aggregate and keep set against the oracle, compaction bit-exact
    in every layer, the padding untouched."""
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(config, kv_layout="interleaved", **overrides)
    _, _, _, near = _run_and_check(spec, hip_device, score_aggregation=score_aggregation)
    assert near <= 4


@pytest.mark.parametrize("layout", [("separate", 0), ("interleaved", 0), ("interleaved", 24)], ids=["separate", "shared-kv", "shared-kv-pad24"])
def test_method_api_compress(hip_device, tmp_path, layout) -> None:
    """TriAttentionMethod through method API v1 on a bound synthetic cache:
    one tensor per layer and kind, or K and V as interleaved views of one
    (padded) buffer per layer as the reference's cache contract allows
    (pkg/provider.py:1201-1230)."""
    from kvcompress_mi355x.methods import create_method
    from kvcompress_mi355x.methods.base import CompressionRequest, LayerCache
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(2, n_layers=4, score_layer_stride=2, seq_lens=(6000,), budget=2048, recent=128,
                                 max_model_len=16384, kv_layout=layout[0], page_pad=layout[1])
    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    cache = workloads.move_cache(host, hip_device)
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
    vllm_config = SimpleNamespace(
        parallel_config=SimpleNamespace(tensor_parallel_size=1),
        model_config=SimpleNamespace(max_model_len=spec.max_model_len),
        speculative_config=None,
    )
    method = create_method(
        "triattention",
        {"stats_path": str(stats_path), "kv_budget": 2048, "score_layer_stride": 2, "protected_recent_window": 128},
        vllm_config,
        spec.model_shape(),
    )
    assert method.compatibility_reasons(None) == ()
    assert method.runtime_spec.compression_threshold_tokens == 2176
    layers = tuple(LayerCache(f"model.layers.{i}.self_attn.attn", i, cache.k_caches[i], cache.v_caches[i]) for i in range(spec.n_layers))
    method.bind_model_runner(SimpleNamespace(device=hip_device), layers)
    src = cache.source_tables[0]
    dst = cache.destination_tables[0]
    request = CompressionRequest(
        request_id="r0",
        semantic_num_tokens=6000,
        physical_num_tokens=6000,
        source_block_ids=(tuple(src.cpu().tolist()),),
        destination_block_ids=(tuple(dst.cpu().tolist()),),
        source_block_ids_device=src,
        destination_block_ids_device=dst,
    )
    keep_only = method.select_keep_indices(src, 6000, 6000)
    result = method.compress(request)
    torch.cuda.synchronize()
    assert result.physical_num_tokens == 2048
    assert result.per_layer_physical_num_tokens == tuple((layer.name, 2048) for layer in layers)
    out = _oracle_for(host, spec, 0)
    assert_keep_matches(keep_only, out["keep"], out["agg"], 2048, _protected(6000, spec))
    slots = ref.token_slots(src.cpu(), keep_only.cpu(), 128)
    dslots = ref.token_slots(dst, torch.arange(2048, device=hip_device), 128)
    for i in range(spec.n_layers):
        assert torch.equal(ref.gather_slots(cache.k_caches[i], dslots).cpu(), ref.gather_slots(host.k_caches[i], slots))
        assert torch.equal(ref.gather_slots(cache.v_caches[i], dslots).cpu(), ref.gather_slots(host.v_caches[i], slots))
    if cache.kv_buffers is not None:
        _assert_padding_untouched(cache)


def test_pipeline_reused_with_a_smaller_batch(hip_device) -> None:
    """A pipeline grown by a two-sequence batch then scores one sequence: the
    head statistics of every scoring layer must come from that call (a stale
    stride once made layer 1 read the previous batch's sequence 0)."""
    from kvcompress_mi355x import workloads
    from kvcompress_mi355x.methods.triattention.pipeline import Batch

    spec = workloads.config_spec(2, n_layers=4, score_layer_stride=2, seq_lens=(3000, 5000), budget=2048, recent=128, max_model_len=16384)
    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    cache = workloads.move_cache(host, hip_device)
    pipeline, batch = workloads.build_pipeline(cache)
    pipeline.select_step(batch)
    for b in (1, 0):
        n = spec.seq_lens[b]
        one = Batch.build(pipeline.device, [n], [n], [cache.source_tables[b]])
        keep = pipeline.select_step(one)[0]
        out = _oracle_for(host, spec, b)
        assert_agg_close(pipeline.agg[:n], out["agg"])
        mean, var = pipeline.head_statistics(one)
        for s_idx in range(len(spec.scoring_layers)):
            want_var, want_mean = out["stats"][s_idx]
            torch.testing.assert_close(mean[s_idx, 0].cpu(), want_mean.reshape(-1), rtol=1e-4, atol=1e-4)
            torch.testing.assert_close(var[s_idx, 0].cpu(), want_var.reshape(-1), rtol=1e-3, atol=1e-4)
        assert_keep_matches(keep, out["keep"], out["agg"], spec.budget, _protected(n, spec))


@pytest.mark.parametrize("order", ["layer_major", "interleaved"])
def test_compaction_order_choice_and_forced_order(hip_device, order) -> None:
    """settle_compaction times both layer orders and keeps one of them; a
    step in either order compacts bit-exactly (the check of _run_and_check
    after the order is forced), and an in-place batch is refused unless the
    caller accepts repeated compaction."""
    from kvcompress_mi355x import workloads

    spec = workloads.config_spec(2, n_layers=3, score_layer_stride=2, seq_lens=(3000, 5000, 2100), budget=2048,
                                 recent=128, max_model_len=16384)
    cache = workloads.move_cache(workloads.build_synthetic_cache(spec, "cpu", seed=1), hip_device)
    pipeline, batch = workloads.build_pipeline(cache)
    pipeline.select_step(batch)
    chosen = pipeline.settle_compaction(batch)
    assert chosen in ("layer_major", "interleaved")
    assert set(pipeline.compaction_form.per_row_ms) == {"layer_major", "interleaved"}

    _run_and_check(spec, hip_device, compaction_order=order)

    ispec = workloads.config_spec(4, n_layers=2, score_layer_stride=1, seq_lens=(6000,), pool_pages=60, max_model_len=16384)
    icache = workloads.move_cache(workloads.build_synthetic_cache(ispec, "cpu", seed=2), hip_device)
    ipipe, ibatch = workloads.build_pipeline(icache)
    ipipe.select_step(ibatch)
    with pytest.raises(ValueError, match="repeat_in_place"):
        ipipe.settle_compaction(ibatch)
