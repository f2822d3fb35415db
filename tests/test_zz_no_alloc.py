"""kvc_score_paged_noalloc (static device scratch) against kvc_score_paged +
kvc_head_stats (caller workspace): identical raw scores and head statistics on
two calls in a row, the second with a smaller batch; oversized batches are
rejected before anything runs."""

from __future__ import annotations

import ctypes

import pytest
import torch

from kvcompress_mi355x import _native, workloads
from kvcompress_mi355x.methods.triattention import _device as dev
from kvcompress_mi355x.methods.triattention.pipeline import Batch


def _noalloc(pipeline, batch, raw, mean, var) -> int:
    """The pipeline's scoring call (kvc_score_paged arguments for this batch)
    with the workspace replaced by the head-statistics outputs."""
    t = pipeline.tables
    layer_stride = int(raw.stride(0))
    strides = (layer_stride, 1, int(raw.stride(1))) if pipeline.head_major else (layer_stride, int(raw.stride(1)), 1)
    return _native.load().kvc_score_paged_noalloc(
        dev.stream_handle(pipeline.device),
        dev.cache_dtype_code(pipeline.dtype),
        t.n_layers,
        dev.ptr(pipeline.scoring_ptrs),
        pipeline.num_pages,
        pipeline.page_stride,
        pipeline.kv_heads,
        pipeline.head_dim,
        t.rotary_dim,
        t.qpk,
        dev.rope_style_code(t.rope_style),
        batch.n_seq,
        max(batch.seq_lens_host),
        dev.ptr(batch.seq_lens),
        dev.ptr(batch.token_offsets),
        dev.ptr(batch.src_offsets),
        dev.ptr(batch.src_ids),
        dev.ptr(t.q_real),
        dev.ptr(t.q_imag),
        dev.ptr(t.freq_scale),
        dev.ptr(t.extra),
        dev.ptr(t.q_pass),
        dev.ptr(pipeline.phase_cos),
        dev.ptr(pipeline.phase_sin),
        t.n_layers * t.freq,
        dev.ptr(raw),
        *strides,
        dev.ptr(mean),
        dev.ptr(var),
    )


def _check_call(pipeline, batch) -> None:
    """Workspace path first (phases, scores, statistics), then the no-alloc
    entry point on the same phase tables into separate outputs."""
    pipeline.score(batch)
    total = batch.total_tokens
    s, h = pipeline.tables.n_layers, pipeline.n_heads
    raw2 = torch.full_like(pipeline.raw, float("nan"))
    mean2 = torch.full((s, batch.n_seq, h), float("nan"), device=pipeline.device)
    var2 = torch.full_like(mean2, float("nan"))
    rc = _noalloc(pipeline, batch, raw2, mean2, var2)
    assert rc == 0, _native.load().kvc_last_error().decode()
    torch.cuda.synchronize()
    want_mean, want_var = pipeline.head_statistics(batch)
    got_raw = raw2.transpose(1, 2) if pipeline.head_major else raw2
    assert torch.equal(got_raw[:, :total], pipeline.raw_scores()[:, :total])
    assert torch.equal(mean2, want_mean)
    assert torch.equal(var2, want_var)


@pytest.mark.gpu
@pytest.mark.parametrize("config", [2, 3])
def test_noalloc_scorer_matches_workspace_scorer_twice(hip_device, config):
    # Two sequences of the workload at full length, then a smaller batch of two
    # shorter ones on the same caches: the second call reuses the device's
    # scratch with a different shape.
    full = workloads.config_spec(config)
    spec = workloads.config_spec(config, n_layers=4 if config == 3 else 16, seq_lens=full.seq_lens[:2])
    cache = workloads.build_synthetic_cache(spec, hip_device, seed=3)
    pipeline, batch = workloads.build_pipeline(cache)
    _check_call(pipeline, batch)
    small_lens = [max(spec.budget + spec.recent + 1, n // 3) for n in spec.seq_lens[:2]]
    small = Batch.build(
        hip_device,
        small_lens,
        small_lens,
        [t[: -(-n // 128)] for t, n in zip(cache.source_tables[:2], small_lens)],
        None if cache.destination_tables is None else cache.destination_tables[:2],
        budget=spec.budget,
    )
    _check_call(pipeline, small)


@pytest.mark.gpu
def test_noalloc_scorer_under_graph_capture(hip_device):
    """The entry point captured into a HIP graph on a side stream (after one
    eager call on the device, which takes the scratch array's address):
    two replays, each after the outputs are overwritten with NaN by eager
    work, give the workspace path's raw scores and statistics bit for bit."""
    spec = workloads.config_spec(2, n_layers=16, seq_lens=(16384, 9000))
    cache = workloads.build_synthetic_cache(spec, hip_device, seed=4)
    pipeline, batch = workloads.build_pipeline(cache)
    pipeline.score(batch)
    total = batch.total_tokens
    want_raw = pipeline.raw_scores()[:, :total].clone()
    want_mean, want_var = (t.clone() for t in pipeline.head_statistics(batch))
    s, h = pipeline.tables.n_layers, pipeline.n_heads
    raw2 = torch.full_like(pipeline.raw, float("nan"))
    mean2 = torch.full((s, batch.n_seq, h), float("nan"), device=pipeline.device)
    var2 = torch.full_like(mean2, float("nan"))

    def check() -> None:
        got_raw = raw2.transpose(1, 2) if pipeline.head_major else raw2
        assert torch.equal(got_raw[:, :total], want_raw)
        assert torch.equal(mean2, want_mean)
        assert torch.equal(var2, want_var)

    assert _noalloc(pipeline, batch, raw2, mean2, var2) == 0, _native.load().kvc_last_error().decode()
    torch.cuda.synchronize()
    check()
    side = torch.cuda.Stream(device=pipeline.device)
    side.wait_stream(torch.cuda.current_stream(pipeline.device))
    graph = torch.cuda.CUDAGraph()
    codes = []
    with torch.cuda.graph(graph, stream=side):
        codes.append(_noalloc(pipeline, batch, raw2, mean2, var2))
    assert codes == [0], _native.load().kvc_last_error().decode()
    for _ in range(2):
        for t in (raw2, mean2, var2):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check()


def test_noalloc_scorer_rejects_batches_beyond_its_scratch():
    lib = _native.load()
    # 6 scoring layers x 64 sequences of 131072 tokens x 40 query heads: the
    # per-tile partial sums alone are 126 MiB, beyond the 64 MiB scratch.
    need = lib.kvc_score_workspace_bytes(6, 8, 128, 128, 5, 64, 131072)
    assert need > 64 << 20
    rc = lib.kvc_score_paged_noalloc(
        None, 0, 6, None, 100, 128 * 8 * 128, 8, 128, 128, 5, 0, 64, 131072, None, None, None, None,
        None, None, None, None, None, None, None, 0, None, 0, 1, 131072, None, None,
    )
    assert rc == _native.EINVAL
    assert "64 MiB" in lib.kvc_last_error().decode()
    small = lib.kvc_score_workspace_bytes(6, 8, 128, 128, 5, 16, 16384)
    assert small <= 64 << 20
    assert isinstance(small, int) and ctypes.sizeof(ctypes.c_size_t) == 8
