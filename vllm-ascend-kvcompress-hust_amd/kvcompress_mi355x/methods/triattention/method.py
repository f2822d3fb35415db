"""TriAttentionMethod: the method API v1 implementation on MI355X.

Keeps the reference's lifecycle and contracts (tri/method.py:57-515):
``runtime_spec`` advertises private destinations, the compression threshold
(budget + recompute window) and the physical budget; ``bind_model_runner``
validates the bound caches against the calibration, precomputes the scoring
tables for every ``score_layer_stride``-th layer and allocates address-stable
device buffers; ``compress`` scores the sampled layers, selects the keep set
and materialises it into the destination blocks of every bound layer,
returning ``CompressionResult(budget, ((layer, budget), ...))``.

``compress_batch`` runs many requests in one batched step (one launch per
kernel for the whole batch); ``compress`` is the one-request case of it.
"""

from __future__ import annotations

import os
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from ...config import KERNEL_BLOCK_SIZE, JsonScalar
from ..base import (
    CompressionRequest,
    CompressionResult,
    KVCompressionMethod,
    LayerCache,
    MethodRuntimeSpec,
    ModelShape,
)
from . import _device as dev
from .config import TriAttentionConfig
from .pipeline import COMPACTION_ORDERS, Batch, CompressionPipeline, ScoringTables, max_all_reducer
from .scoring import build_geometric_offsets
from .stats import CalibrationStats, DeviceLayerCalibrationStats

METHOD_NAME = "triattention"
MTP_LAYER_NAME = "mtp.layers.0.self_attn.attn"


def queries_per_kv_head(model_shape: ModelShape) -> int:
    if model_shape.num_attention_heads % model_shape.num_kv_heads:
        raise RuntimeError("TriAttention requires query heads divisible by KV heads")
    return model_shape.num_attention_heads // model_shape.num_kv_heads


def scoring_layer_indices(n_layers: int, stride: int) -> tuple[int, ...]:
    """The layers whose keys are scored: every ``stride``-th attention layer
    from the first, and no other (tri/method.py:188,312 sample
    ``layer_caches[::score_layer_stride]``; the last layer is not added)."""
    if stride <= 0:
        raise ValueError("method option 'score_layer_stride' must be positive")
    return tuple(range(0, n_layers, stride))


COMPACTION_ORDER_ENV = "KVCOMPRESS_MI355X_COMPACTION_ORDER"


def compaction_order_setting() -> str:
    """The compaction layer order a bound cache uses: the environment's
    KVCOMPRESS_MI355X_COMPACTION_ORDER ("layer_major" or "interleaved" pins
    it), else "auto", which times both orders on the cache's first
    compactions and keeps the faster.  The method options stay the
    reference's, so this deployment setting is not one of them."""
    value = os.environ.get(COMPACTION_ORDER_ENV, "auto").strip() or "auto"
    if value not in COMPACTION_ORDERS:
        raise ValueError(f"{COMPACTION_ORDER_ENV} must be one of {', '.join(COMPACTION_ORDERS)}, got {value!r}")
    return value


def is_mtp_cache_layer(layer_name: str) -> bool:
    return ".mtp.layers." in f".{layer_name}."


@dataclass(frozen=True)
class TriAttentionLayerCache:
    name: str
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    stats: DeviceLayerCalibrationStats


class TriAttentionMethod(KVCompressionMethod):
    """TriAttention KV selection with MI355X HIP kernels behind method API v1."""

    def __init__(self, options: Mapping[str, JsonScalar], vllm_config: Any, model_shape: ModelShape) -> None:
        self.config = TriAttentionConfig.from_method_config(options)
        self.vllm_config = vllm_config
        self.model_shape = model_shape
        self.calibration = CalibrationStats.load(self.config.stats_path)
        self.layer_caches: tuple[TriAttentionLayerCache, ...] = ()
        self.materialization_caches: tuple[LayerCache, ...] = ()
        self.cache_block_size = KERNEL_BLOCK_SIZE
        self.offsets: torch.Tensor | None = None
        self.pipeline: CompressionPipeline | None = None
        self.tensor_parallel_size = 1
        self.all_reduce_max = None  # the TP group's MAX all-reduce when tensor_parallel_size > 1

    @property
    def name(self) -> str:
        return METHOD_NAME

    @property
    def runtime_spec(self) -> MethodRuntimeSpec:
        return MethodRuntimeSpec(
            requires_private_destination=True,
            compression_threshold_tokens=self.config.compression_threshold_tokens,
            required_recompute_tokens=self.config.recompute_window,
            max_physical_num_tokens=self.config.kv_budget,
            min_output_tokens_for_compression=self.config.min_output_tokens_for_compression,
        )

    def compatibility_reasons(self, worker: Any) -> tuple[str, ...]:
        del worker
        return self.calibration.validate(self.model_shape)

    # ---------------------------------------------------------------- bind --
    def bind_model_runner(self, runner: Any, layer_caches: tuple[LayerCache, ...]) -> None:
        tp_size = int(getattr(getattr(self.vllm_config, "parallel_config", None), "tensor_parallel_size", 1))
        if tp_size < 1:
            raise RuntimeError(f"invalid tensor_parallel_size {tp_size}")
        tp_rank = 0
        self.tensor_parallel_size = tp_size
        self.all_reduce_max = None
        if tp_size > 1:
            # KV heads are sharded over the TP group (tri/method.py:111-122): this
            # rank scores its own heads and the per-layer head maxima meet in one
            # MAX all-reduce per step (tri/method.py:447-461).
            group = tensor_parallel_group()
            tp_rank = int(group.rank_in_group)
            self.all_reduce_max = max_all_reducer(group.device_group)
        device = torch.device(runner.device)
        if device.type != "cuda":
            raise RuntimeError("TriAttention on MI355X requires a HIP device")
        max_len = int(self.vllm_config.model_config.max_model_len)
        device_stats = self.calibration.to_device(
            self.model_shape, device, tensor_parallel_rank=tp_rank, tensor_parallel_size=tp_size
        )
        self.offsets = build_geometric_offsets(max_len, device)

        mtp = tuple(layer for layer in layer_caches if is_mtp_cache_layer(layer.name))
        target = tuple(layer for layer in layer_caches if not is_mtp_cache_layer(layer.name))
        speculative = getattr(self.vllm_config, "speculative_config", None)
        if mtp and (
            len(mtp) != 1
            or mtp[0].name != MTP_LAYER_NAME
            or getattr(speculative, "method", None) != "mtp"
            or getattr(speculative, "num_speculative_tokens", None) != 2
        ):
            raise RuntimeError("uncalibrated MTP cache requires Qwen3.5 MTP2")
        if len(target) != len(self.model_shape.full_attention_layer_indices):
            raise RuntimeError("allocated full-attention layer count does not match calibration")
        bound: list[TriAttentionLayerCache] = []
        seen: set[int] = set()
        for layer in target:
            if layer.layer_index not in device_stats:
                raise RuntimeError(
                    f"attention layer {layer.name!r} resolves to invalid model layer index {layer.layer_index}"
                )
            if layer.layer_index in seen:
                raise RuntimeError(f"multiple cache layers resolve to model layer index {layer.layer_index}")
            seen.add(layer.layer_index)
            bound.append(TriAttentionLayerCache(layer.name, layer.k_cache, layer.v_cache, device_stats[layer.layer_index]))
        expected = set(self.model_shape.full_attention_layer_indices)
        if seen != expected:
            raise RuntimeError(
                "allocated target full-attention layers do not match calibration: "
                f"allocated={sorted(seen)} expected={sorted(expected)}"
            )
        self.layer_caches = tuple(bound)
        self.materialization_caches = tuple(layer_caches)
        cache = self.layer_caches[0].k_cache
        self.cache_block_size = int(cache.shape[1])
        if self.cache_block_size != KERNEL_BLOCK_SIZE:
            raise RuntimeError("TriAttention requires 128-token kernel cache blocks")
        local_kv_heads = self.model_shape.num_kv_heads // tp_size
        if int(cache.shape[2]) != local_kv_heads:
            raise RuntimeError(
                "local KV-cache head count does not match tensor-parallel model shape: "
                f"expected {local_kv_heads}, got {cache.shape[2]}"
            )
        queries_per_kv_head(self.model_shape)
        scoring = [self.layer_caches[i] for i in scoring_layer_indices(len(self.layer_caches), self.config.score_layer_stride)]
        tables = ScoringTables.from_layer_stats([layer.stats for layer in scoring], self.offsets)
        self.pipeline = CompressionPipeline(
            scoring_k_caches=[layer.k_cache for layer in scoring],
            k_caches=[layer.k_cache for layer in self.materialization_caches],
            v_caches=[layer.v_cache for layer in self.materialization_caches],
            tables=tables,
            budget=self.config.kv_budget,
            protected_prefix=self.config.protected_prefix_window,
            protected_recent=self.config.protected_recent_window,
            segments=self.config.position_segments,
            policy=self.config.position_policy,
            layer_aggregation=self.config.layer_aggregation,
            max_seqs=1,
            max_seq_len=max_len,
            score_aggregation=self.config.score_aggregation,
            compaction_order=compaction_order_setting(),
        )

    # ------------------------------------------------------------ compress --
    def _result(self) -> CompressionResult:
        return CompressionResult(
            physical_num_tokens=self.config.kv_budget,
            per_layer_physical_num_tokens=tuple(
                (layer.name, self.config.kv_budget) for layer in self.materialization_caches
            ),
        )

    def compress(self, request: CompressionRequest) -> CompressionResult:
        return self.compress_batch((request,))[0]

    def compress_batch(self, requests: Sequence[CompressionRequest]) -> list[CompressionResult]:
        """Compress many scheduler-authorised requests in one batched step."""
        if self.pipeline is None or self.offsets is None or not self.layer_caches:
            raise RuntimeError("TriAttention method is not bound to KV cache")
        if not requests:
            return []
        for request in requests:
            dev.require_hip(request.source_block_ids_device, "source_block_ids_device")
            dev.require_hip(request.destination_block_ids_device, "destination_block_ids_device")
        batch = Batch.build(
            self.pipeline.device,
            [int(r.physical_num_tokens) for r in requests],
            [int(r.semantic_num_tokens) for r in requests],
            [r.source_block_ids_device for r in requests],
            [r.destination_block_ids_device for r in requests],
            block_size=self.cache_block_size,
            budget=self.config.kv_budget,
        )
        self._select(batch)
        self.pipeline.compact(batch)
        return [self._result() for _ in requests]

    def _select(self, batch: Batch) -> torch.Tensor:
        if self.all_reduce_max is not None:
            return self.pipeline.select_step_sharded(batch, self.all_reduce_max)
        return self.pipeline.select_step(batch)

    def select_keep_indices(self, source_block_ids: torch.Tensor, physical_num_tokens: int, round_start: int) -> torch.Tensor:
        """Keep indices of one request without materialising (tri/method.py:297-475)."""
        if self.pipeline is None:
            raise RuntimeError("TriAttention method is not bound to KV cache")
        batch = Batch.build(self.pipeline.device, [int(physical_num_tokens)], [int(round_start)], [source_block_ids])
        return self._select(batch)[0].clone()


def tensor_parallel_group() -> Any:
    """vLLM's tensor-parallel group coordinator (``rank_in_group``,
    ``device_group``), imported only when tensor_parallel_size > 1, as the
    reference does (tri/method.py:113-116)."""
    try:
        from vllm.distributed import get_tp_group
    except ImportError as exc:
        raise RuntimeError("tensor_parallel_size > 1 needs vLLM's tensor-parallel group (vllm.distributed)") from exc
    return get_tp_group()


def create_triattention_method(
    options: Mapping[str, JsonScalar], vllm_config: Any, model_shape: ModelShape
) -> KVCompressionMethod:
    return TriAttentionMethod(options, vllm_config, model_shape)


# Import name of the options type before the method registry existed
# (tri/method.py:518-519); callers that still import it get the same class.
TriAttentionAscendConfig = TriAttentionConfig
