"""Scheduler and worker halves of the compression transaction protocol, with
the scenarios of the reference's scheduler tests (tests/test_stateful.py:
404-506, 855-915, 559-583) restated on the host-agnostic API here: one
request "r" of 300 prompt tokens in blocks [3, 4, 5], budget 128 and recompute
window 128 (threshold 256), destination blocks taken from a pool starting at
50."""

from __future__ import annotations

import pickle
from types import SimpleNamespace

import pytest
import torch

from kvcompress_mi355x.methods.base import CompressionResult, MethodRuntimeSpec
from kvcompress_mi355x.transaction import PLAN_ATTRIBUTE, CompressionPlan
from kvcompress_mi355x.transactions import (
    FROZEN_STEP,
    ActiveCompression,
    BlockPool,
    DeferredRelease,
    SchedulerTransactions,
)
from kvcompress_mi355x.worker import CompressionWorker


def _state(*, async_scheduling=False, max_concurrent_batches=None, min_output_tokens=0, speculative=False):
    pool = BlockPool(range(50, 150))
    freed: list[int] = []
    original_free = pool.free_blocks

    def record(ids):
        ids = list(ids)
        freed.extend(ids)
        original_free(ids)

    pool.free_blocks = record
    req_to_blocks = {"r": [3, 4, 5]}
    request = SimpleNamespace(
        request_id="r", num_computed_tokens=300, num_prompt_tokens=300, max_tokens=128, next_decode_eligible_step=7
    )
    requests = {"r": request}
    state = SchedulerTransactions(
        threshold=256,
        budget=128,
        page_tokens=128,
        pool=pool,
        req_to_blocks=req_to_blocks,
        requests=requests,
        required_recompute_tokens=128,
        min_output_tokens=min_output_tokens,
        async_scheduling=async_scheduling,
        max_concurrent_batches=max_concurrent_batches,
        speculative=speculative,
        num_cached_block={"r": 2},
    )
    return state, req_to_blocks, freed, requests


def _output(**kw):
    base = dict(num_scheduled_tokens={"r": 44}, finished_req_ids=set(), preempted_req_ids=set())
    base.update(kw)
    return SimpleNamespace(**base)


def test_plan_survives_pickle() -> None:
    plan = CompressionPlan(300, 128, (3, 4, 5), (50,))
    assert pickle.loads(pickle.dumps(plan)) == plan


def test_commit_only_after_output_ack() -> None:
    state, blocks, freed, _ = _state()
    output = _output()
    state.after_schedule(output)
    state.before_schedule()
    assert blocks["r"] == [3, 4, 5] and not freed
    assert getattr(output, PLAN_ATTRIBUTE)["r"].destination_block_ids == (50,)
    assert getattr(output, PLAN_ATTRIBUTE)["r"] == CompressionPlan(300, 128, (3, 4, 5), (50,))

    state.after_output(output)
    state.before_schedule()
    assert blocks["r"] == [50]
    assert freed == [5, 4, 3]
    assert state.active["r"] == ActiveCompression(300, 128)
    assert state.num_cached_block["r"] == 0
    assert state.physical_tokens("r", 301) == 129


def test_async_request_frozen_until_ack() -> None:
    state, blocks, _, requests = _state(async_scheduling=True)
    output = _output()
    state.after_schedule(output)
    assert requests["r"].next_decode_eligible_step == FROZEN_STEP
    state.before_schedule()
    assert blocks["r"] == [3, 4, 5]

    state.after_output(SimpleNamespace(num_scheduled_tokens={"other": 1}))
    state.before_schedule()
    assert blocks["r"] == [3, 4, 5]
    assert requests["r"].next_decode_eligible_step == FROZEN_STEP

    state.after_output(output)
    state.before_schedule()
    assert blocks["r"] == [50]
    assert requests["r"].next_decode_eligible_step == 7


def test_async_sources_wait_for_queued_batches() -> None:
    state, blocks, freed, _ = _state(async_scheduling=True, max_concurrent_batches=3)
    output = _output()
    state.after_schedule(output)
    state.after_output(output)
    assert blocks["r"] == [50] and not freed
    state.after_output(SimpleNamespace(num_scheduled_tokens={"other": 1}))
    assert not freed
    state.after_output(SimpleNamespace(num_scheduled_tokens={"other": 1}))
    assert freed == [5, 4, 3]


def test_finished_request_discards_pending() -> None:
    state, _, freed, _ = _state()
    state.after_schedule(_output())
    state.before_schedule(finished_req_ids={"r"})
    assert not state.pending
    assert freed == [50]


def test_short_output_request_is_not_armed() -> None:
    state, _, _, requests = _state(min_output_tokens=64)
    requests["r"].max_tokens = 32
    state.after_schedule(_output())
    assert not state.pending


def test_invalid_max_tokens_fails_closed() -> None:
    state, _, _, requests = _state()
    requests["r"].max_tokens = -1
    with pytest.raises(RuntimeError, match="max_tokens"):
        state.after_schedule(_output())


def test_preempted_request_discards_active_state() -> None:
    state, _, _, _ = _state()
    state.active["r"] = ActiveCompression(300, 128)
    state.after_schedule(_output(num_scheduled_tokens={}, preempted_req_ids={"r"}))
    assert not state.active


def test_free_releases_async_tail_on_abort() -> None:
    state, _, freed, _ = _state()
    state.deferred_releases["r"] = [DeferredRelease("r", (5, 4), 1)]
    state.free_request("r")
    assert freed == [5, 4]
    assert not state.deferred_releases


def test_first_compression_waits_for_prompt_boundary_and_threshold() -> None:
    state, _, _, requests = _state()
    requests["r"].num_computed_tokens = 200  # mid-prompt chunk
    assert state.after_schedule(_output()) == {}
    requests["r"].num_computed_tokens = 300
    requests["r"].num_prompt_tokens = 300
    state.threshold = 301
    assert state.after_schedule(_output()) == {}


def test_recompression_uses_the_current_physical_window() -> None:
    state, blocks, _, requests = _state()
    state.active["r"] = ActiveCompression(300, 128)
    requests["r"].num_computed_tokens = 427  # 128 + 127 decoded tokens: physical 255 < 256
    assert state.after_schedule(_output()) == {}
    requests["r"].num_computed_tokens = 428  # physical 256 reaches the threshold
    plans = state.after_schedule(_output())
    assert plans["r"].semantic_anchor == 428 and plans["r"].physical_anchor == 128


def test_speculative_decode_steps_are_not_armed() -> None:
    state, _, _, _ = _state()
    assert state.after_schedule(_output(scheduled_spec_decode_tokens={"r": [1, 2]})) == {}
    state, _, _, requests = _state(speculative=True)
    state.active["r"] = ActiveCompression(300, 128)
    requests["r"].num_computed_tokens = 500
    assert state.after_schedule(_output()) == {}


def test_pool_exhaustion_skips_instead_of_failing() -> None:
    state, _, _, _ = _state()
    state.pool.get_new_blocks(state.pool.get_num_free_blocks())
    assert state.after_schedule(_output()) == {}


def test_changed_block_table_fails_at_commit() -> None:
    state, blocks, freed, _ = _state()
    output = _output()
    state.after_schedule(output)
    state.after_output(output)
    blocks["r"].append(6)
    with pytest.raises(RuntimeError, match="changed before compression commit"):
        state.before_schedule()
    assert freed == [50] and not state.pending


def test_budget_must_be_page_aligned() -> None:
    with pytest.raises(RuntimeError, match="divisible"):
        SchedulerTransactions(
            threshold=4736, budget=4608, page_tokens=2048, pool=BlockPool([]), req_to_blocks={}, requests={}
        )


def test_prefix_cache_hit_cap() -> None:
    state, _, _, requests = _state()
    assert state.prefix_cache_hit_cap(requests["r"]) == 172  # 300 - recompute 128
    requests["r"].num_prompt_tokens = 200
    assert state.prefix_cache_hit_cap(requests["r"]) is None


# ------------------------------------------------------------------ worker --


class _FakeMethod:
    name = "fake"

    def __init__(self) -> None:
        self.batches: list[list] = []
        self.runtime_spec = MethodRuntimeSpec(
            requires_private_destination=True,
            compression_threshold_tokens=256,
            required_recompute_tokens=128,
            max_physical_num_tokens=128,
            min_output_tokens_for_compression=0,
        )

    def compress_batch(self, requests):
        self.batches.append(list(requests))
        return [CompressionResult(128) for _ in requests]


def _worker_setup():
    state, blocks, freed, sched_requests = _state()
    runner_request = SimpleNamespace(num_computed_tokens=256, num_prompt_tokens=300, max_tokens=128, block_ids=([3, 4, 5],))
    method = _FakeMethod()
    worker = CompressionWorker(method, requests={"r": runner_request}, page_tokens=128, device="cpu")
    return state, blocks, freed, sched_requests, runner_request, method, worker


def test_worker_executes_plan_and_commits_on_next_schedule() -> None:
    state, blocks, freed, _, runner_request, method, worker = _worker_setup()
    output = _output()
    state.after_schedule(output)
    # The worker sees the pre-step count plus this step's 44 tokens = 300.
    results = worker.compress_scheduled_requests(output)
    assert set(results) == {"r"} and len(method.batches) == 1
    sent = method.batches[0][0]
    assert sent.semantic_num_tokens == 300 and sent.physical_num_tokens == 300
    assert sent.source_block_ids == ((3, 4, 5),) and sent.destination_block_ids == ((50,),)
    assert torch.equal(sent.destination_block_ids_device, torch.tensor([50]))
    assert runner_request.block_ids == ([3, 4, 5],)  # nothing changes before the barrier
    state.after_output(output)
    state.before_schedule()
    worker.before_update_states(SimpleNamespace(num_scheduled_tokens={"r": 1}, finished_req_ids=set()))
    assert runner_request.block_ids == ([50],) and blocks["r"] == [50] and freed == [5, 4, 3]
    assert worker.active["r"] == ActiveCompression(300, 128)
    assert worker.request_offsets(["r", "other"]).tolist() == [172, 0]


def test_worker_rejects_plans_that_disagree_with_its_state() -> None:
    state, _, _, _, runner_request, _, worker = _worker_setup()
    output = _output()
    state.after_schedule(output)
    runner_request.num_computed_tokens = 257  # semantic 301 != plan's 300
    runner_request.num_prompt_tokens = 301
    with pytest.raises(RuntimeError, match="semantic length disagrees"):
        worker.compress_scheduled_requests(output)
    runner_request.num_computed_tokens, runner_request.num_prompt_tokens = 256, 300
    runner_request.block_ids = ([3, 4, 9],)
    with pytest.raises(RuntimeError, match="source block table disagrees"):
        worker.compress_scheduled_requests(output)
    runner_request.block_ids = ([3, 4, 50],)
    bad = CompressionPlan(300, 128, (3, 4, 50), (50,))
    setattr(output, PLAN_ATTRIBUTE, {"r": bad})
    with pytest.raises(RuntimeError, match="private destination"):
        worker.compress_scheduled_requests(output)


def test_worker_batches_every_authorised_request_in_one_call() -> None:
    method = _FakeMethod()
    requests = {
        f"r{i}": SimpleNamespace(num_computed_tokens=296, num_prompt_tokens=300, max_tokens=64, block_ids=([10 * i, 10 * i + 1, 10 * i + 2],))
        for i in range(1, 4)
    }
    worker = CompressionWorker(method, requests=requests, page_tokens=128, device="cpu")
    output = SimpleNamespace(num_scheduled_tokens={k: 4 for k in requests}, finished_req_ids=set())
    setattr(
        output,
        PLAN_ATTRIBUTE,
        {k: CompressionPlan(300, 128, tuple(r.block_ids[0]), (900 + i,)) for i, (k, r) in enumerate(requests.items())},
    )
    assert set(worker.compress_scheduled_requests(output)) == set(requests)
    assert len(method.batches) == 1 and len(method.batches[0]) == 3
    # Finished requests drop their pending state at the next update.
    worker.before_update_states(SimpleNamespace(num_scheduled_tokens={}, finished_req_ids={"r1"}))
    assert "r1" not in worker.pending and set(worker.pending) == {"r2", "r3"}
