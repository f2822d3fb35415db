"""Method API v1: the contract between the compression step and a method.

Mirrors pkg/methods/base.py:15-189 of the reference plugin (same type names,
fields, defaults and abstract members) so a method written against the
reference contract binds here unchanged.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any

import torch

from ..transaction import CompressionPlan


@dataclass(frozen=True)
class ModelShape:
    """Transformer shape a method needs (pkg/methods/base.py:15-41)."""

    model_type: str
    num_layers: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float
    has_rope_scaling: bool
    rotary_dim: int | None = None
    attention_layer_indices: tuple[int, ...] | None = None

    @property
    def effective_rotary_dim(self) -> int:
        return self.head_dim if self.rotary_dim is None else self.rotary_dim

    @property
    def full_attention_layer_indices(self) -> tuple[int, ...]:
        if self.attention_layer_indices is None:
            return tuple(range(self.num_layers))
        return self.attention_layer_indices

    @property
    def is_hybrid(self) -> bool:
        return len(self.full_attention_layer_indices) != self.num_layers


@dataclass(frozen=True)
class MethodRuntimeSpec:
    """Scheduler-visible limits of a method (pkg/methods/base.py:44-52)."""

    requires_private_destination: bool
    compression_threshold_tokens: int
    required_recompute_tokens: int
    max_physical_num_tokens: int
    min_output_tokens_for_compression: int = 0


@dataclass(frozen=True)
class LayerCache:
    """One full-attention K/V cache binding (pkg/methods/base.py:55-62)."""

    name: str
    layer_index: int
    k_cache: torch.Tensor
    v_cache: torch.Tensor


@dataclass(frozen=True)
class CompressionRequest:
    """One scheduler-authorised compression transaction (pkg/methods/base.py:65-77)."""

    request_id: str
    semantic_num_tokens: int
    physical_num_tokens: int
    source_block_ids: tuple[tuple[int, ...], ...]
    destination_block_ids: tuple[tuple[int, ...], ...]
    source_block_ids_device: torch.Tensor
    destination_block_ids_device: torch.Tensor
    plan: CompressionPlan | None = None
    per_layer_physical_num_tokens: tuple[tuple[str, int], ...] | None = None


@dataclass(frozen=True)
class CompressionResult:
    """Physical state after compression (pkg/methods/base.py:80-85)."""

    physical_num_tokens: int
    per_layer_physical_num_tokens: tuple[tuple[str, int], ...] | None = None


@dataclass(frozen=True)
class QueryBatchSpan:
    """Query rows of one request in a forward batch (pkg/methods/base.py:88-94)."""

    request_id: str
    start: int
    end: int


@dataclass(frozen=True)
class QueryObservation:
    """A completed final-prefill transaction (pkg/methods/base.py:97-110)."""

    request_id: str
    plan: CompressionPlan
    semantic_num_tokens: int
    window_tokens: int
    layer_indices: tuple[int, ...]


class KVCompressionMethod(ABC):
    """Algorithm boundary under the lifecycle adapter (pkg/methods/base.py:113-189)."""

    @property
    @abstractmethod
    def name(self) -> str:
        """Stable configuration name."""

    @property
    @abstractmethod
    def runtime_spec(self) -> MethodRuntimeSpec:
        """Scheduler-visible limits, known before KV allocation."""

    @abstractmethod
    def compatibility_reasons(self, worker: Any) -> tuple[str, ...]:
        """Method-specific incompatibilities, without side effects."""

    @abstractmethod
    def bind_model_runner(self, runner: Any, layer_caches: tuple[LayerCache, ...]) -> None:
        """Bind runtime state after the host has allocated its KV cache."""

    @abstractmethod
    def compress(self, request: CompressionRequest) -> CompressionResult:
        """Materialise one compression transaction."""

    @property
    def query_window_tokens(self) -> int:
        """Trailing prefill query rows the method observes; 0 installs no hooks."""
        return 0

    @property
    def query_layer_indices(self) -> tuple[int, ...] | None:
        """Model-layer indices whose queries are observed; None = all bound layers."""
        return None

    @property
    def requires_per_layer_physical_state(self) -> bool:
        """Whether per-layer physical lengths may differ after compression."""
        return False

    def capture_query(
        self, layer: LayerCache, query: torch.Tensor, spans: tuple[QueryBatchSpan, ...]
    ) -> None:
        """Copy prefill query rows into method-owned buffers (default: none)."""
        return None

    def complete_query_observation(self, observation: QueryObservation) -> None:
        """Publish buffered queries after a successful forward (default: none)."""
        return None

    def discard_query_observation(self, request_id: str) -> None:
        """Release one request's uncommitted observation (default: none)."""
        return None
