"""The whole compression transaction on the GPU: the scheduler arms plans over
a real page pool, the worker compresses every armed request in one batched
launch through TriAttentionMethod, the scheduler commits (table swap, reverse
release of the source pages), and the next decode token of each request is
written through the fused physical slot mapping into the compacted table."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from helpers import assert_keep_matches, oracle_layer_stats
from oracle import brute
from oracle import triattention_ref as ref

pytestmark = pytest.mark.gpu


def test_transaction_round_trip(hip_device, tmp_path) -> None:
    from kvcompress_mi355x import workloads
    from kvcompress_mi355x.methods import create_method
    from kvcompress_mi355x.methods.base import LayerCache
    from kvcompress_mi355x.methods.triattention.kernels import compute_physical_slot_mapping
    from kvcompress_mi355x.transaction import PLAN_ATTRIBUTE
    from kvcompress_mi355x.transactions import BlockPool, SchedulerTransactions
    from kvcompress_mi355x.worker import CompressionWorker

    budget, recent = 2048, 128
    spec = workloads.config_spec(
        2, n_layers=4, score_layer_stride=2, seq_lens=(3000, 5000), budget=budget, recent=recent, max_model_len=16384
    )
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
        {"stats_path": str(stats_path), "kv_budget": budget, "score_layer_stride": 2, "protected_recent_window": recent},
        vllm_config,
        spec.model_shape(),
    )
    layers = tuple(
        LayerCache(f"model.layers.{i}.self_attn.attn", i, cache.k_caches[i], cache.v_caches[i]) for i in range(spec.n_layers)
    )
    method.bind_model_runner(SimpleNamespace(device=hip_device), layers)

    # Host state: each request holds its prompt pages; every other pool page is free.
    num_pages = int(cache.k_caches[0].shape[0])
    req_to_blocks = {f"r{b}": [int(p) for p in host.source_tables[b].tolist()] for b in range(2)}
    used = {p for blocks in req_to_blocks.values() for p in blocks}
    pool = BlockPool([p for p in range(num_pages) if p not in used])
    free_before = pool.get_num_free_blocks()
    prompts = {f"r{b}": spec.seq_lens[b] for b in range(2)}
    last_chunk = 64
    sched_requests = {
        r: SimpleNamespace(num_computed_tokens=n, num_prompt_tokens=n, max_tokens=256, next_decode_eligible_step=0)
        for r, n in prompts.items()
    }
    runner_requests = {
        r: SimpleNamespace(num_computed_tokens=n - last_chunk, num_prompt_tokens=n, max_tokens=256, block_ids=(list(req_to_blocks[r]),))
        for r, n in prompts.items()
    }
    spec_rt = method.runtime_spec
    state = SchedulerTransactions(
        threshold=spec_rt.compression_threshold_tokens,
        budget=spec_rt.max_physical_num_tokens,
        page_tokens=128,
        pool=pool,
        req_to_blocks=req_to_blocks,
        requests=sched_requests,
        required_recompute_tokens=spec_rt.required_recompute_tokens,
    )
    worker = CompressionWorker(method, requests=runner_requests, page_tokens=128, device=hip_device)

    # Step: schedule the last prompt chunk of both requests, arm, execute.
    output = SimpleNamespace(num_scheduled_tokens={r: last_chunk for r in prompts}, finished_req_ids=set(), preempted_req_ids=set())
    plans = state.after_schedule(output)
    assert set(plans) == set(prompts)
    assert pool.get_num_free_blocks() == free_before - 2 * (budget // 128)
    results = worker.compress_scheduled_requests(output)
    torch.cuda.synchronize()
    assert {r: res.physical_num_tokens for r, res in results.items()} == {r: budget for r in prompts}

    # The compacted rows equal the oracle's materialisation of its keep set.
    for b, r in enumerate(sorted(prompts)):
        out = ref.method_select(
            [host.k_caches[layer] for layer in spec.scoring_layers],
            oracle_layer_stats(host.calibration, spec.model_shape(), spec.scoring_layers),
            host.source_tables[b],
            spec.seq_lens[b],
            host.round_starts[b],
            ref.build_geometric_offsets(spec.max_model_len),
            ref.MethodConfig(budget=budget, recent=recent, score_chunk_size=8192, score_layer_stride=2),
        )
        got_keep = method.select_keep_indices(host.source_tables[b].to(hip_device), spec.seq_lens[b], spec.seq_lens[b])
        protected = torch.zeros(spec.seq_lens[b], dtype=torch.bool)
        protected[spec.seq_lens[b] - recent :] = True
        assert_keep_matches(got_keep, out["keep"], out["agg"], budget, protected)
        dst = torch.tensor(plans[r].destination_block_ids)
        src_slots = ref.token_slots(host.source_tables[b], got_keep.cpu(), 128)
        for layer in range(spec.n_layers):
            want_k = ref.gather_slots(host.k_caches[layer], src_slots)
            want_v = ref.gather_slots(host.v_caches[layer], src_slots)
            got_k = cache.k_caches[layer][dst.to(hip_device)].cpu().reshape(want_k.shape)
            got_v = cache.v_caches[layer][dst.to(hip_device)].cpu().reshape(want_v.shape)
            assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)

    # Output acknowledged; the next schedule commits on both sides.
    state.after_output(output)
    state.before_schedule()
    for r in prompts:
        assert req_to_blocks[r] == list(plans[r].destination_block_ids)
        runner_requests[r].num_computed_tokens = prompts[r]
    assert pool.free_ids()[-len(plans["r1"].source_block_ids) :] == tuple(reversed(plans["r1"].source_block_ids))
    decode = SimpleNamespace(num_scheduled_tokens={r: 1 for r in prompts}, finished_req_ids=set())
    worker.before_update_states(decode)
    assert all(runner_requests[r].block_ids[0] == list(plans[r].destination_block_ids) for r in prompts)

    # Decode token at semantic position = prompt length: physical length
    # budget + 1 needs one more page, which the host allocates from the pool.
    order = sorted(prompts)
    for r in order:
        assert state.physical_tokens(r, prompts[r] + 1) == budget + 1
        req_to_blocks[r].append(pool.get_new_blocks(1)[0])
    table = torch.full((2, 32), -1, dtype=torch.int32)
    for i, r in enumerate(order):
        table[i, : len(req_to_blocks[r])] = torch.tensor(req_to_blocks[r], dtype=torch.int32)
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32)
    positions = torch.tensor([prompts[r] for r in order], dtype=torch.int64)
    offsets = worker.request_offsets(order)
    slots = torch.empty(2, dtype=torch.int64, device=hip_device)
    compute_physical_slot_mapping(qsl.to(hip_device), positions.to(hip_device), offsets, table.to(hip_device), 128, slots)
    want, phys = brute.slot_mapping(qsl.tolist(), positions.tolist(), offsets.cpu().tolist(), table.tolist(), 128, 2)
    assert phys == [budget, budget]
    assert slots.cpu().tolist() == want == [req_to_blocks[r][-1] * 128 for r in order]
