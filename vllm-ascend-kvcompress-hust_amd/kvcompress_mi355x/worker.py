"""Worker-side compression transactions: execute armed plans, then commit.

The worker half of the protocol in transactions.py (pkg/provider.py:321-371,
471-601).  After the model step of a scheduler output, every request that
carries a plan and passes the same gates the scheduler applied is compressed
-- all of them in one batched launch per kernel through the method's
``compress_batch`` (the reference loops the requests one at a time).  The new
physical state waits as pending until the next scheduler output that
schedules the request again, which is the commit boundary on the worker: the
request's full-attention block table becomes the destination blocks and its
semantic -> physical offset becomes active for the decode-side position shift
(kernels.shift_positions / compute_physical_slot_mapping).

Host objects are duck-typed as the host's runner exposes them: ``requests``
maps a request id to an object with ``num_computed_tokens``,
``num_prompt_tokens``, ``max_tokens`` and ``block_ids`` (one block-id list per
cache group); scheduler outputs carry ``num_scheduled_tokens``,
``finished_req_ids``, ``preempted_req_ids`` and, optionally,
``scheduled_cached_reqs.resumed_req_ids``.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from .config import KERNEL_BLOCK_SIZE
from .methods.base import CompressionRequest, CompressionResult, KVCompressionMethod
from .methods.triattention.cache import expand_scheduler_block_ids
from .transaction import PLAN_ATTRIBUTE, CompressionPlan
from .transactions import ActiveCompression, blocks_for_tokens, request_max_tokens


@dataclass(frozen=True)
class PendingCompression:
    """Physical state written by the worker, not yet committed
    (pkg/provider.py:38-43)."""

    semantic_anchor: int
    physical_anchor: int
    block_ids: tuple[int, ...]


class CompressionWorker:
    """Runs scheduler-authorised compressions for one model runner."""

    def __init__(
        self,
        method: KVCompressionMethod,
        *,
        requests: Mapping[str, Any],
        page_tokens: int,
        device: torch.device | str,
        attention_group_index: int = 0,
    ) -> None:
        if page_tokens <= 0 or page_tokens % KERNEL_BLOCK_SIZE:
            raise ValueError(f"scheduler pages must be a multiple of {KERNEL_BLOCK_SIZE} tokens")
        self.method = method
        self.spec = method.runtime_spec
        self.requests = requests
        self.page_tokens = int(page_tokens)
        self.cache_blocks_per_page = self.page_tokens // KERNEL_BLOCK_SIZE
        self.device = torch.device(device)
        self.attention_group_index = int(attention_group_index)
        self.pending: dict[str, PendingCompression] = {}
        self.active: dict[str, ActiveCompression] = {}

    # ----------------------------------------------------------- compress --
    def compress_scheduled_requests(self, output: Any) -> dict[str, CompressionResult]:
        """Execute the plans of a scheduler output (pkg/provider.py:471-601)."""
        plans: Mapping[str, CompressionPlan] = getattr(output, PLAN_ATTRIBUTE, None) or {}
        required = blocks_for_tokens(self.spec.max_physical_num_tokens, self.page_tokens)
        batch: list[tuple[str, CompressionRequest]] = []
        for request_id, scheduled in output.num_scheduled_tokens.items():
            plan = plans.get(request_id)
            if plan is None or request_id in self.pending:
                continue
            request = self.requests.get(request_id)
            if request is None:
                continue
            if request_max_tokens(request) < self.spec.min_output_tokens_for_compression:
                continue
            semantic = int(request.num_computed_tokens) + int(scheduled)
            active = self.active.get(request_id)
            if active is None:
                if semantic != int(request.num_prompt_tokens):
                    continue
                physical = semantic
            else:
                physical = active.physical_anchor + semantic - active.semantic_anchor
            if semantic != plan.semantic_anchor:
                raise RuntimeError(
                    f"request {request_id!r} semantic length disagrees with the scheduler compression plan"
                )
            if physical < self.spec.compression_threshold_tokens:
                continue
            if self.attention_group_index >= len(request.block_ids):
                raise RuntimeError("request has no full-attention block table")
            source = tuple(int(b) for b in request.block_ids[self.attention_group_index])
            if len(source) < required:
                raise RuntimeError(f"request {request_id!r} has too few blocks for compression")
            if source != plan.source_block_ids:
                raise RuntimeError(
                    f"request {request_id!r} source block table disagrees with the scheduler compression plan"
                )
            destination = plan.destination_block_ids
            if len(destination) != required or set(destination) & set(source):
                raise RuntimeError(f"request {request_id!r} requires private destination blocks")
            batch.append(
                (
                    request_id,
                    CompressionRequest(
                        request_id=request_id,
                        semantic_num_tokens=semantic,
                        physical_num_tokens=physical,
                        source_block_ids=(source,),
                        destination_block_ids=(destination,),
                        source_block_ids_device=self._expand(source),
                        destination_block_ids_device=self._expand(destination),
                        plan=plan,
                    ),
                )
            )
        if not batch:
            return {}
        requests = [request for _, request in batch]
        compress_batch = getattr(self.method, "compress_batch", None)
        if compress_batch is not None:
            results = list(compress_batch(requests))
        else:  # a method without a batched entry point: one call per request
            results = [self.method.compress(request) for request in requests]
        if len(results) != len(batch):
            raise RuntimeError("method returned a result count that does not match the batch")
        done: dict[str, CompressionResult] = {}
        for (request_id, request), result in zip(batch, results):
            compacted = result.physical_num_tokens
            if isinstance(compacted, bool) or not isinstance(compacted, int):
                raise RuntimeError("method returned a non-integer physical length")
            if compacted != self.spec.max_physical_num_tokens:
                raise RuntimeError(f"method {self.method.name!r} returned unexpected length {compacted}")
            self.pending[request_id] = PendingCompression(
                request.semantic_num_tokens, compacted, request.destination_block_ids[0]
            )
            done[request_id] = result
        return done

    # ------------------------------------------------------------- commit --
    def before_update_states(self, output: Any) -> None:
        """Commit pending compressions of requests scheduled again
        (pkg/provider.py:321-371)."""
        reset = set(getattr(output, "finished_req_ids", ()) or ())
        reset.update(getattr(output, "preempted_req_ids", ()) or ())
        cached = getattr(output, "scheduled_cached_reqs", None)
        reset.update(getattr(cached, "resumed_req_ids", ()) or ())
        for request_id in reset:
            self.pending.pop(request_id, None)
            self.active.pop(request_id, None)
        for request_id, pending in tuple(self.pending.items()):
            if request_id not in output.num_scheduled_tokens:
                continue  # still frozen by the scheduler
            request = self.requests.get(request_id)
            if request is None:
                del self.pending[request_id]
                continue
            groups = list(request.block_ids)
            groups[self.attention_group_index] = list(pending.block_ids)
            request.block_ids = tuple(groups)
            self.active[request_id] = ActiveCompression(pending.semantic_anchor, pending.physical_anchor)
            del self.pending[request_id]

    def request_offsets(self, request_ids: Sequence[str]) -> torch.Tensor:
        """Semantic minus physical length per request row (0 when the request
        was never compressed), int64 on the device: the offsets of the
        decode-side position shift (pkg/provider.py:980-1010)."""
        values = [self.active[r].removed_tokens if r in self.active else 0 for r in request_ids]
        return torch.tensor(values, dtype=torch.int64, device=self.device)

    # ------------------------------------------------------------ helpers --
    def _expand(self, block_ids: tuple[int, ...]) -> torch.Tensor:
        ids = torch.tensor(block_ids, dtype=torch.int64, device=self.device)
        if self.cache_blocks_per_page == 1:
            return ids
        return expand_scheduler_block_ids(ids, self.cache_blocks_per_page)
