"""The compression step captured as one HIP graph replays to the eager step's
results: every replay is checked against an eager step run on the same cache
contents, with eager work, cache edits and synchronisations between replays."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

SPECS = {
    "private": (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(3000, 1500, 4096), budget=1024, recent=64, max_model_len=8192)),
    "inplace": (4, dict(n_layers=2, score_layer_stride=1, seq_lens=(6000, 9000), pool_pages=160, max_model_len=16384)),
    # score_aggregation="max": per-offset phase table, both folds and the max scorer in the graph.
    "private-max": (2, dict(n_layers=4, score_layer_stride=2, seq_lens=(3000, 4096), budget=1024, recent=64, max_model_len=131072)),
}


@pytest.mark.parametrize("mode", sorted(SPECS))
def test_graph_replays_match_eager_steps(hip_device, mode) -> None:
    from kvcompress_mi355x import workloads

    index, overrides = SPECS[mode]
    spec = workloads.config_spec(index, **overrides)
    assert spec.inplace == (mode == "inplace")
    cache = workloads.build_synthetic_cache(spec, hip_device, seed=3)
    pipeline, batch = workloads.build_pipeline(cache, score_aggregation="max" if mode.endswith("-max") else "mean")
    pristine_k = [k.clone() for k in cache.k_caches]
    pristine_v = [v.clone() for v in cache.v_caches]
    g = torch.Generator(device=hip_device).manual_seed(11)
    noise = [torch.randn(pristine_k[layer].shape, generator=g, device=hip_device).to(spec.dtype) for layer in spec.scoring_layers]

    def load_inputs(replay: int) -> None:
        # New keys in the same pages: replay r perturbs the scoring layers by r * noise.
        for layer in range(spec.n_layers):
            cache.k_caches[layer].copy_(pristine_k[layer])
            cache.v_caches[layer].copy_(pristine_v[layer])
        for i, layer in enumerate(spec.scoring_layers):
            cache.k_caches[layer].add_(noise[i] * replay)

    load_inputs(0)
    step_graph = pipeline.capture(batch)
    keeps = []
    for replay in range(4):
        load_inputs(replay)
        torch.cuda.synchronize()
        step_graph.replay()
        torch.cuda.synchronize()
        got_keep = step_graph.keep.clone()
        got_tables = step_graph.tables.clone()
        got_freed = [f.clone() for f in step_graph.freed]
        got_k = [k.clone() for k in cache.k_caches]
        got_v = [v.clone() for v in cache.v_caches]

        load_inputs(replay)
        keep, tables, freed = pipeline.step(batch)
        torch.cuda.synchronize()
        assert torch.equal(got_keep, keep), f"replay {replay}: keep"
        assert torch.equal(got_tables, tables), f"replay {replay}: tables"
        assert all(torch.equal(a, b) for a, b in zip(got_freed, freed)), f"replay {replay}: freed"
        for layer in range(spec.n_layers):
            assert torch.equal(got_k[layer], cache.k_caches[layer]), f"replay {replay}: K layer {layer}"
            assert torch.equal(got_v[layer], cache.v_caches[layer]), f"replay {replay}: V layer {layer}"
        keeps.append(keep.cpu())
    # The perturbed inputs change the selection, so the replays did recompute.
    assert any(not torch.equal(keeps[0], k) for k in keeps[1:])
