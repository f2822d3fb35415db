"""TriAttention calibration artifacts: load, validate, lay out for the device.

Reads both artifact formats of the reference (tri/stats.py:59-86):
  * schema-3 ``layer_stats``: {layer: {q_mean_complex | q_mean_real/q_mean_imag,
    q_abs_mean, freq_scale_sq?, inv_freq?, q_pass_mean?}}  (tri/stats.py:420-464)
  * legacy flat ``stats``: {"layerLL_headHH": {q_mean_real, q_mean_imag,
    q_abs_mean}} with complete, contiguous head indices  (tri/stats.py:374-417)
Only ``torch.load(weights_only=True)`` touches the file.  ``validate`` returns
the same incompatibility reasons as tri/stats.py:88-260; ``to_device`` groups
query-head rows by KV head (tri/stats.py:345-360), takes one tensor-parallel
shard of KV heads (tri/stats.py:315-323) and resolves omega from inv_freq or
1/theta^(2i/R) (tri/stats.py:325-331).
"""

from __future__ import annotations

import math
import re
from collections.abc import Mapping
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch

from ..base import ModelShape

_FLAT_KEY = re.compile(r"^layer(?P<layer>\d+)_head(?P<head>\d+)$")
SUPPORTED_MODEL_TYPES = frozenset(
    {
        "llama",
        "mistral",
        "qwen2",
        "qwen2_moe",
        "qwen3",
        "qwen3_moe",
        "qwen3_5_text",
        "qwen3_5_moe_text",
    }
)


@dataclass(frozen=True)
class LayerCalibrationStats:
    q_mean_real: torch.Tensor
    q_mean_imag: torch.Tensor
    q_abs_mean: torch.Tensor
    freq_scale_sq: torch.Tensor | None = None
    inv_freq: torch.Tensor | None = None
    q_pass_mean: torch.Tensor | None = None


@dataclass(frozen=True)
class DeviceLayerCalibrationStats:
    """Per-layer statistics grouped as [kv_heads, queries_per_kv, width]."""

    q_mean_real: torch.Tensor
    q_mean_imag: torch.Tensor
    q_abs_mean: torch.Tensor
    freq_scale_sq: torch.Tensor
    omega: torch.Tensor
    rope_style: str
    rotary_dim: int | None = None
    q_pass_mean: torch.Tensor | None = None


def _matrix(value: Any, name: str) -> torch.Tensor:
    if not isinstance(value, torch.Tensor):
        raise ValueError(f"calibration field {name!r} must be a tensor")
    tensor = value.detach().to(device="cpu", dtype=torch.float32)
    if tensor.ndim == 1:
        tensor = tensor.unsqueeze(0)
    if tensor.ndim != 2:
        raise ValueError(f"calibration field {name!r} must be rank two")
    return tensor.contiguous()


def _vector(value: Any) -> torch.Tensor | None:
    if isinstance(value, torch.Tensor):
        return value.detach().to(device="cpu", dtype=torch.float32).flatten()
    if isinstance(value, (list, tuple)):
        return torch.tensor(value, dtype=torch.float32).flatten()
    return None


def _flat_layers(entries: Mapping[str, Any]) -> dict[int, LayerCalibrationStats]:
    by_layer: dict[int, dict[int, Mapping[str, Any]]] = {}
    for key, entry in entries.items():
        match = _FLAT_KEY.match(str(key))
        if match is None:
            continue
        if not isinstance(entry, Mapping):
            raise ValueError(f"calibration entry {key!r} must be a mapping")
        by_layer.setdefault(int(match["layer"]), {})[int(match["head"])] = entry
    if not by_layer:
        raise ValueError("flat calibration statistics contain no layer/head entries")
    layers: dict[int, LayerCalibrationStats] = {}
    for layer, heads in by_layer.items():
        order = list(range(max(heads) + 1))
        if sorted(heads) != order:
            raise ValueError(
                f"layer {layer} calibration heads must be complete and contiguous; got {sorted(heads)}"
            )

        def rows(field: str) -> torch.Tensor:
            return torch.stack([_matrix(heads[h][field], field)[0] for h in order])

        layers[layer] = LayerCalibrationStats(
            rows("q_mean_real"), rows("q_mean_imag"), rows("q_abs_mean")
        )
    return layers


def _structured_layers(entries: Mapping[Any, Any]) -> dict[int, LayerCalibrationStats]:
    layers: dict[int, LayerCalibrationStats] = {}
    for raw_index, entry in entries.items():
        if not isinstance(entry, Mapping):
            raise ValueError(f"layer statistics {raw_index!r} must be a mapping")
        q_mean = entry.get("q_mean_complex")
        if isinstance(q_mean, torch.Tensor) and q_mean.is_complex():
            real = _matrix(q_mean.real, "q_mean_complex.real")
            imag = _matrix(q_mean.imag, "q_mean_complex.imag")
        elif isinstance(q_mean, torch.Tensor) and q_mean.ndim == 3:
            if q_mean.shape[-1] != 2:
                raise ValueError("q_mean_complex final dimension must equal two")
            real = _matrix(q_mean[..., 0], "q_mean_complex.real")
            imag = _matrix(q_mean[..., 1], "q_mean_complex.imag")
        else:
            real = _matrix(entry.get("q_mean_real"), "q_mean_real")
            imag = _matrix(entry.get("q_mean_imag"), "q_mean_imag")
        scale = entry.get("freq_scale_sq")
        pass_mean = entry.get("q_pass_mean")
        layers[int(raw_index)] = LayerCalibrationStats(
            q_mean_real=real,
            q_mean_imag=imag,
            q_abs_mean=_matrix(entry.get("q_abs_mean"), "q_abs_mean"),
            freq_scale_sq=_matrix(scale, "freq_scale_sq") if scale is not None else None,
            inv_freq=_vector(entry.get("inv_freq")) if isinstance(entry.get("inv_freq"), torch.Tensor) else None,
            q_pass_mean=_matrix(pass_mean, "q_pass_mean") if pass_mean is not None else None,
        )
    return layers


def _metadata_inv_freq(metadata: Mapping[str, Any], layer: int) -> torch.Tensor | None:
    per_layer = metadata.get("layer_inv_freqs")
    value: Any = None
    if isinstance(per_layer, Mapping):
        value = per_layer.get(layer, per_layer.get(str(layer)))
    elif isinstance(per_layer, (list, tuple)) and layer < len(per_layer):
        value = per_layer[layer]
    if value is None:
        value = metadata.get("inv_freq")
    return _vector(value)


def group_query_stats(tensor: torch.Tensor, model: ModelShape, group: int, width: int) -> torch.Tensor:
    """[H_q, w] -> [H_kv, group, w] (consecutive query heads per KV head);
    [H_kv, w] rows are repeated across the group."""
    shape = tuple(tensor.shape)
    if shape == (model.num_attention_heads, width):
        return tensor.reshape(model.num_kv_heads, group, width).contiguous()
    if shape == (model.num_kv_heads, width):
        return tensor.unsqueeze(1).expand(model.num_kv_heads, group, width).contiguous()
    raise ValueError(
        f"calibration tensor shape {shape} cannot be grouped for "
        f"{model.num_attention_heads} query heads and {model.num_kv_heads} KV heads"
    )


@dataclass(frozen=True)
class CalibrationStats:
    metadata: Mapping[str, Any]
    layers: Mapping[int, LayerCalibrationStats]

    @classmethod
    def load(cls, path: Path) -> CalibrationStats:
        path = Path(path)
        if not path.is_file():
            raise ValueError(f"calibration statistics file does not exist: {path}")
        payload = torch.load(path, map_location="cpu", weights_only=True)
        if not isinstance(payload, Mapping):
            raise ValueError("calibration statistics payload must be a mapping")
        metadata = payload.get("metadata", {})
        if not isinstance(metadata, Mapping):
            raise ValueError("calibration metadata must be a mapping")
        flat = payload.get("stats")
        if isinstance(flat, Mapping) and flat:
            layers = _flat_layers(flat)
        else:
            structured = payload.get("layer_stats")
            if not isinstance(structured, Mapping) or not structured:
                raise ValueError("calibration payload must contain non-empty 'stats' or 'layer_stats'")
            layers = _structured_layers(structured)
        return cls(metadata=dict(metadata), layers=layers)

    # ------------------------------------------------------------ validate --
    def _metadata_reasons(self, model: ModelShape) -> list[str]:
        md = self.metadata
        reasons: list[str] = []
        if model.model_type not in SUPPORTED_MODEL_TYPES:
            reasons.append(f"model_type {model.model_type!r} has no verified RoPE layout")
        expected = set(model.full_attention_layer_indices)
        if set(self.layers) != expected:
            reasons.append(
                "calibration layer set does not match the model: "
                f"expected {sorted(expected)}, got {sorted(self.layers)}"
            )
        style = str(md.get("rope_style", "half"))
        if style != "half":
            reasons.append(f"calibration rope_style {style!r} is unsupported; expected 'half'")

        def mismatch(key: str, actual: Any, label: str | None = None) -> None:
            value = md.get(key)
            if value is not None and int(value) != actual:
                reasons.append(
                    f"calibration {label or key} {value} does not match model {label or key} {actual}"
                )

        mismatch("head_dim", model.head_dim)
        mismatch("rotary_dim", model.effective_rotary_dim)
        layers_md = md.get("attention_layer_indices")
        if layers_md is not None and tuple(int(v) for v in layers_md) != model.full_attention_layer_indices:
            reasons.append("calibration attention_layer_indices do not match the model")
        model_type = md.get("model_type")
        if model_type is not None and str(model_type) != model.model_type:
            reasons.append(
                f"calibration model_type {model_type!r} does not match model_type {model.model_type!r}"
            )
        mismatch("num_layers", model.num_layers)
        mismatch("num_attention_heads", model.num_attention_heads)
        kv = md.get("num_kv_heads", md.get("num_key_value_heads"))
        if kv is not None and int(kv) != model.num_kv_heads:
            reasons.append(f"calibration num_kv_heads {kv} does not match model value {model.num_kv_heads}")
        theta = md.get("rope_theta")
        if theta is not None and not math.isclose(float(theta), model.rope_theta, rel_tol=1e-7, abs_tol=0.0):
            reasons.append(
                f"calibration rope_theta {theta} does not match model rope_theta {model.rope_theta}"
            )
        return reasons

    def validate(self, model: ModelShape) -> tuple[str, ...]:
        reasons = self._metadata_reasons(model)
        rope_type = self.metadata.get("rope_type", "default") or "default"
        freq = model.effective_rotary_dim // 2
        pass_dim = model.head_dim - model.effective_rotary_dim
        q_shape = (model.num_attention_heads, freq)
        kv_shape = (model.num_kv_heads, freq)
        for index, layer in self.layers.items():
            for name, tensor in (
                ("q_mean_real", layer.q_mean_real),
                ("q_mean_imag", layer.q_mean_imag),
                ("q_abs_mean", layer.q_abs_mean),
            ):
                if tuple(tensor.shape) not in {q_shape, kv_shape}:
                    reasons.append(
                        f"layer {index} {name} has shape {tuple(tensor.shape)}; "
                        f"expected {q_shape} or {kv_shape}"
                    )
                if not bool(torch.isfinite(tensor).all()):
                    reasons.append(f"layer {index} {name} contains non-finite values")
            if bool((layer.q_abs_mean < 0).any()):
                reasons.append(f"layer {index} q_abs_mean contains negative values")
            if pass_dim:
                pq, pk = (model.num_attention_heads, pass_dim), (model.num_kv_heads, pass_dim)
                if layer.q_pass_mean is None:
                    reasons.append(f"layer {index} partial RoPE requires q_pass_mean")
                elif tuple(layer.q_pass_mean.shape) not in {pq, pk}:
                    reasons.append(
                        f"layer {index} q_pass_mean has shape {tuple(layer.q_pass_mean.shape)}; "
                        f"expected {pq} or {pk}"
                    )
                elif not bool(torch.isfinite(layer.q_pass_mean).all()):
                    reasons.append(f"layer {index} q_pass_mean contains non-finite values")
            scale = layer.freq_scale_sq
            if scale is not None:
                if tuple(scale.shape) not in {(1, freq), q_shape, kv_shape}:
                    reasons.append(
                        f"layer {index} freq_scale_sq has incompatible shape {tuple(scale.shape)}"
                    )
                if not bool(torch.isfinite(scale).all()):
                    reasons.append(f"layer {index} freq_scale_sq contains non-finite values")
                if bool((scale <= 0).any()):
                    reasons.append(f"layer {index} freq_scale_sq must be positive")
            elif model.has_rope_scaling:
                reasons.append(f"layer {index} scaled RoPE requires freq_scale_sq calibration values")
            inv_freq = layer.inv_freq if layer.inv_freq is not None else _metadata_inv_freq(self.metadata, index)
            if inv_freq is None and (model.has_rope_scaling or rope_type != "default"):
                reasons.append(
                    f"layer {index} scaled or non-default RoPE requires exact inv_freq calibration values"
                )
            if inv_freq is not None:
                if inv_freq.numel() != freq:
                    reasons.append(f"layer {index} inv_freq has {inv_freq.numel()} values; expected {freq}")
                if not bool(torch.isfinite(inv_freq).all()):
                    reasons.append(f"layer {index} inv_freq contains non-finite values")
                if bool((inv_freq <= 0).any()):
                    reasons.append(f"layer {index} inv_freq must be positive")
        return tuple(reasons)

    # ----------------------------------------------------------- to_device --
    def to_device(
        self,
        model: ModelShape,
        device: torch.device,
        *,
        tensor_parallel_rank: int = 0,
        tensor_parallel_size: int = 1,
    ) -> dict[int, DeviceLayerCalibrationStats]:
        if tensor_parallel_size <= 0 or not 0 <= tensor_parallel_rank < tensor_parallel_size:
            raise ValueError("invalid tensor-parallel rank or size")
        if model.num_kv_heads % tensor_parallel_size:
            raise ValueError(
                "TriAttention tensor parallelism requires KV heads divisible by tensor-parallel size"
            )
        group = model.num_attention_heads // model.num_kv_heads
        rotary = model.effective_rotary_dim
        freq = rotary // 2
        style = str(self.metadata.get("rope_style", "half"))
        local = model.num_kv_heads // tensor_parallel_size
        lo, hi = tensor_parallel_rank * local, (tensor_parallel_rank + 1) * local
        result: dict[int, DeviceLayerCalibrationStats] = {}
        for index, layer in self.layers.items():

            def grouped(tensor: torch.Tensor, width: int) -> torch.Tensor:
                full = group_query_stats(tensor.to(device=device, dtype=torch.float32), model, group, width)
                return full[lo:hi].contiguous()

            scale = layer.freq_scale_sq
            if scale is None:
                scale = torch.ones(model.num_attention_heads, freq, dtype=torch.float32)
            if scale.shape[0] == 1:
                scale = scale.expand(model.num_attention_heads, -1)
            inv_freq = layer.inv_freq if layer.inv_freq is not None else _metadata_inv_freq(self.metadata, index)
            if inv_freq is None:
                exponents = torch.arange(0, rotary, 2, dtype=torch.float32)
                inv_freq = 1.0 / (model.rope_theta ** (exponents / float(rotary)))
            result[index] = DeviceLayerCalibrationStats(
                q_mean_real=grouped(layer.q_mean_real, freq),
                q_mean_imag=grouped(layer.q_mean_imag, freq),
                q_abs_mean=grouped(layer.q_abs_mean, freq),
                freq_scale_sq=grouped(scale, freq),
                omega=inv_freq.to(device=device, dtype=torch.float32).contiguous(),
                rope_style=style,
                rotary_dim=rotary,
                q_pass_mean=(
                    grouped(layer.q_pass_mean, model.head_dim - rotary)
                    if layer.q_pass_mean is not None
                    else None
                ),
            )
        return result
