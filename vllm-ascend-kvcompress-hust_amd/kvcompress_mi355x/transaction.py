"""Scheduler-to-worker compression plan (pkg/transaction.py:8-18)."""

from __future__ import annotations

from dataclasses import dataclass

PLAN_ATTRIBUTE = "_ascend_kvcompress_plans_v4"


@dataclass(frozen=True)
class CompressionPlan:
    """Source blocks stay immutable until the destination blocks are written."""

    semantic_anchor: int
    physical_anchor: int
    source_block_ids: tuple[int, ...]
    destination_block_ids: tuple[int, ...]
