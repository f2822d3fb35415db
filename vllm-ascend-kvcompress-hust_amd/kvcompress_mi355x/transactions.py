"""Scheduler-side compression transactions: arm, acknowledge, commit, release.

A compression is a two-sided transaction between the scheduler, which owns
the block pool and every request's block table, and the worker, which moves
the kept K/V rows on the GPU (pkg/stateful.py:66-561, pkg/transaction.py):

  arm (after a schedule)   a request whose physical length reached the
                           threshold gets ceil(budget / page) private
                           destination blocks from the pool and a
                           CompressionPlan that travels to the worker with
                           the scheduler output; under async scheduling the
                           request is frozen until the plan is acknowledged.
  acknowledge (output)     the worker's output for that step carries the
                           plan back; the plan becomes ready.
  commit (next barrier)    the request's table becomes the destination
                           blocks and every source block is released in
                           reverse order -- immediately, or after
                           max_concurrent_batches - 1 further outputs when
                           batches already queued may still read them.
  discard                  a finished, preempted or vanished request returns
                           its reserved destination blocks instead.

The host here is whatever object keeps these in step: the block pool
(``get_num_free_blocks``, ``get_new_blocks``, ``free_blocks`` over integer
block ids), ``req_to_blocks`` (request id -> mutable list of block ids of the
full-attention group) and ``requests`` (request id -> object with
``num_computed_tokens``, ``num_prompt_tokens``, ``max_tokens`` and a mutable
``next_decode_eligible_step``).  Scheduler outputs are read by attribute
(``num_scheduled_tokens``, ``finished_req_ids``, ``preempted_req_ids``,
``scheduled_spec_decode_tokens``) as the host's SchedulerOutput carries them,
and plans are attached under PLAN_ATTRIBUTE.
"""

from __future__ import annotations

import logging
from collections import deque
from collections.abc import Iterable, Mapping, MutableMapping
from dataclasses import dataclass
from typing import Any

from .transaction import PLAN_ATTRIBUTE, CompressionPlan

logger = logging.getLogger(__name__)

# Eligibility step that keeps a frozen request out of async scheduling.
FROZEN_STEP = 1 << 62


def blocks_for_tokens(tokens: int, page_tokens: int) -> int:
    """Scheduler blocks that hold ``tokens`` tokens."""
    return -(-int(tokens) // int(page_tokens))


def request_max_tokens(request: Any) -> int:
    """The request's output limit, validated as the reference does
    (pkg/stateful.py:564-570)."""
    value = getattr(request, "max_tokens", None)
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise RuntimeError("Request.max_tokens must be a non-negative integer")
    return value


class BlockPool:
    """Free-block queue over integer ids: allocation takes from the front,
    release appends at the back (the order in which the host's pool reuses
    blocks)."""

    def __init__(self, block_ids: Iterable[int]) -> None:
        self._free: deque[int] = deque(int(b) for b in block_ids)
        if len(set(self._free)) != len(self._free):
            raise ValueError("block ids must be unique")

    def get_num_free_blocks(self) -> int:
        return len(self._free)

    def get_new_blocks(self, count: int) -> list[int]:
        if count < 0 or count > len(self._free):
            raise RuntimeError(f"cannot allocate {count} blocks ({len(self._free)} free)")
        return [self._free.popleft() for _ in range(count)]

    def free_blocks(self, block_ids: Iterable[int]) -> None:
        self._free.extend(int(b) for b in block_ids)

    def free_ids(self) -> tuple[int, ...]:
        return tuple(self._free)


@dataclass
class PendingTransaction:
    plan: CompressionPlan
    reserved_blocks: tuple[int, ...]
    ready: bool = False
    previous_eligible_step: int | None = None


@dataclass(frozen=True)
class ActiveCompression:
    semantic_anchor: int
    physical_anchor: int

    @property
    def removed_tokens(self) -> int:
        return self.semantic_anchor - self.physical_anchor


@dataclass
class DeferredRelease:
    request_id: str
    blocks: tuple[int, ...]
    remaining_outputs: int


class SchedulerTransactions:
    """Scheduler half of the compression protocol (pkg/stateful.py:75-561).

    ``threshold``, ``budget``, ``required_recompute_tokens`` and
    ``min_output_tokens`` come from the method's runtime spec
    (pkg/methods/base.py:44-52); ``page_tokens`` is the full-attention
    group's scheduler block size.
    """

    def __init__(
        self,
        *,
        threshold: int,
        budget: int,
        page_tokens: int,
        pool: Any,
        req_to_blocks: MutableMapping[str, list[int]],
        requests: Mapping[str, Any],
        required_recompute_tokens: int = 0,
        min_output_tokens: int = 0,
        async_scheduling: bool = False,
        max_concurrent_batches: int | None = None,
        speculative: bool = False,
        num_cached_block: MutableMapping[str, int] | None = None,
    ) -> None:
        if page_tokens <= 0:
            raise ValueError("page_tokens must be positive")
        if budget <= 0 or budget % page_tokens:
            raise RuntimeError(
                f"compression target must be divisible by full-attention logical block size {page_tokens}"
            )
        if threshold < budget:
            raise ValueError("the compression threshold cannot be below the budget")
        batches = (2 if async_scheduling else 1) if max_concurrent_batches is None else int(max_concurrent_batches)
        if batches < 1:
            raise RuntimeError("max_concurrent_batches must be positive")
        self.threshold = int(threshold)
        self.budget = int(budget)
        self.page_tokens = int(page_tokens)
        self.required_recompute_tokens = int(required_recompute_tokens)
        self.min_output_tokens = int(min_output_tokens)
        self.async_scheduling = bool(async_scheduling)
        self.max_concurrent_batches = batches
        self.speculative = bool(speculative)
        self.pool = pool
        self.req_to_blocks = req_to_blocks
        self.requests = requests
        self.num_cached_block = num_cached_block
        self.pending: dict[str, PendingTransaction] = {}
        self.active: dict[str, ActiveCompression] = {}
        self.deferred_releases: dict[str, list[DeferredRelease]] = {}

    # ------------------------------------------------------------ lengths --
    def physical_tokens(self, request_id: str, tokens: int) -> int:
        """Token count of the full-attention group for a semantic count
        (the length translation of pkg/stateful.py:432-487)."""
        active = self.active.get(request_id)
        return max(0, int(tokens) - active.removed_tokens) if active else int(tokens)

    def prefix_cache_hit_cap(self, request: Any) -> int | None:
        """Longest prefix-cache hit that still leaves the method its query
        suffix (pkg/stateful.py:165-178)."""
        prompt = int(request.num_prompt_tokens)
        if prompt < self.threshold or request_max_tokens(request) < self.min_output_tokens:
            return None
        return max(0, min(prompt - 1, prompt - self.required_recompute_tokens))

    # ------------------------------------------------------------- phases --
    def after_schedule(self, output: Any) -> dict[str, CompressionPlan]:
        """Arm plans for the requests of this schedule (pkg/stateful.py:489-561)."""
        reset = set(getattr(output, "preempted_req_ids", ()) or ())
        reset.update(getattr(output, "finished_req_ids", ()) or ())
        for request_id in reset:
            self._discard_pending(request_id)
            self.active.pop(request_id, None)
        speculative_tokens = getattr(output, "scheduled_spec_decode_tokens", {}) or {}
        keep = blocks_for_tokens(self.budget, self.page_tokens)
        plans: dict[str, CompressionPlan] = {}
        for request_id in output.num_scheduled_tokens:
            if speculative_tokens.get(request_id) or request_id in self.pending:
                continue
            request = self.requests.get(request_id)
            if request is None or request_max_tokens(request) < self.min_output_tokens:
                continue
            # The pre-step count: the worker adds this step's scheduled tokens.
            semantic = int(request.num_computed_tokens)
            active = self.active.get(request_id)
            if active is None:
                if semantic != int(request.num_prompt_tokens):
                    continue  # the first compression happens at the prompt boundary
                physical = semantic
            else:
                physical = active.physical_anchor + semantic - active.semantic_anchor
            if physical < self.threshold:
                continue
            if self.speculative and active is not None:
                continue  # draft KV of a decode step may still roll back
            blocks = self.req_to_blocks.get(request_id, ())
            if len(blocks) < keep:
                raise RuntimeError(f"request {request_id!r} has too few scheduler blocks")
            if self.pool.get_num_free_blocks() < keep:
                logger.warning(
                    "skipping KV compression for request %s: %d private destination blocks unavailable",
                    request_id,
                    keep,
                )
                continue
            destination = tuple(int(b) for b in self.pool.get_new_blocks(keep))
            plan = CompressionPlan(
                semantic_anchor=semantic,
                physical_anchor=self.budget,
                source_block_ids=tuple(int(b) for b in blocks),
                destination_block_ids=destination,
            )
            previous = None
            if self.async_scheduling:
                previous = int(request.next_decode_eligible_step)
                request.next_decode_eligible_step = FROZEN_STEP
            self.pending[request_id] = PendingTransaction(plan, destination, previous_eligible_step=previous)
            plans[request_id] = plan
        if plans:
            setattr(output, PLAN_ATTRIBUTE, plans)
        return plans

    def before_schedule(self, finished_req_ids: Iterable[str] = ()) -> None:
        """Drop finished requests, then commit acknowledged plans when
        scheduling is synchronous (pkg/stateful.py:282-290)."""
        for request_id in tuple(finished_req_ids):
            self._discard_pending(request_id)
            self.active.pop(request_id, None)
        if not self.async_scheduling:
            self._commit_pending(defer_release_outputs=0)

    def after_output(self, output: Any) -> None:
        """The worker's output acknowledges the plans it executed
        (pkg/stateful.py:362-368)."""
        for request_id, plan in (getattr(output, PLAN_ATTRIBUTE, None) or {}).items():
            pending = self.pending.get(request_id)
            if pending is not None and pending.plan == plan:
                pending.ready = True
        self.after_model_output()

    def after_model_output(self) -> None:
        """Async scheduling commits at the output barrier; sources stay
        allocated until the batches already queued have produced output
        (pkg/stateful.py:292-299)."""
        if not self.async_scheduling:
            return
        self._drain_deferred_releases()
        self._commit_pending(defer_release_outputs=max(0, self.max_concurrent_batches - 1))

    def free_request(self, request_id: str) -> None:
        """The host released a request (finished or aborted): return its
        reserved and deferred blocks now (the KVCacheManager.free hook,
        pkg/stateful.py:628-640)."""
        self._discard_pending(request_id)
        for release in self.deferred_releases.pop(request_id, ()):
            self.pool.free_blocks(release.blocks)
        self.active.pop(request_id, None)

    # ------------------------------------------------------------ helpers --
    def _commit_pending(self, *, defer_release_outputs: int) -> None:
        for request_id, pending in tuple(self.pending.items()):
            if not pending.ready:
                continue
            if request_id not in self.requests:
                self._discard_pending(request_id)
                continue
            blocks = self.req_to_blocks.get(request_id)
            if blocks is None:
                self._discard_pending(request_id)
                continue
            plan = pending.plan
            if tuple(int(b) for b in blocks) != plan.source_block_ids:
                self._discard_pending(request_id)
                raise RuntimeError(f"request {request_id!r} block table changed before compression commit")
            released = tuple(reversed(tuple(blocks)))
            blocks[:] = list(pending.reserved_blocks)
            if defer_release_outputs:
                self.deferred_releases.setdefault(request_id, []).append(
                    DeferredRelease(request_id, released, defer_release_outputs)
                )
            else:
                self.pool.free_blocks(released)
            if self.num_cached_block is not None and request_id in self.num_cached_block:
                # Compacted KV no longer matches the prefix hashes of the
                # request's original tokens.
                self.num_cached_block[request_id] = 0
            self.active[request_id] = ActiveCompression(plan.semantic_anchor, plan.physical_anchor)
            if pending.previous_eligible_step is not None:
                self.requests[request_id].next_decode_eligible_step = pending.previous_eligible_step
            del self.pending[request_id]

    def _drain_deferred_releases(self) -> None:
        for request_id, releases in tuple(self.deferred_releases.items()):
            kept: list[DeferredRelease] = []
            for release in releases:
                release.remaining_outputs -= 1
                if release.remaining_outputs <= 0:
                    self.pool.free_blocks(release.blocks)
                else:
                    kept.append(release)
            if kept:
                self.deferred_releases[request_id] = kept
            else:
                del self.deferred_releases[request_id]

    def _discard_pending(self, request_id: str) -> None:
        pending = self.pending.pop(request_id, None)
        if pending is None:
            return
        self.pool.free_blocks(reversed(pending.reserved_blocks))
        request = self.requests.get(request_id)
        if request is not None and pending.previous_eligible_step is not None:
            request.next_decode_eligible_step = pending.previous_eligible_step
