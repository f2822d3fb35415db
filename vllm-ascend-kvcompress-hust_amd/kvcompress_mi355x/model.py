"""Method-facing model shape from a Hugging Face text configuration.

Mirrors model_shape_from_config (pkg/model.py:12-109): head counts, head
dimension (``head_dim`` or hidden_size / heads), layer count, RoPE theta (from
``rope_theta`` or ``rope_parameters``, default 10000), rotary dimension
(``rotary_dim``, ``rope_parameters["rope_dim"]`` or ``partial_rotary_factor``),
the full-attention layers of a hybrid model (``layer_types``) and whether RoPE
is scaled.  The same configurations are rejected with ValueError.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

from .methods.base import ModelShape

_LAYER_TYPES = frozenset({"full_attention", "linear_attention"})
_UNSCALED_ROPE_KEYS = frozenset({"rope_theta", "rope_type", "type"})


def model_shape_from_config(model_config: Any) -> ModelShape:
    """ModelShape of a host model config exposing ``hf_text_config`` or ``hf_config``."""
    text = getattr(model_config, "hf_text_config", None)
    if text is None:
        text = getattr(model_config, "hf_config", None)
    if text is None:
        raise ValueError("model has no Hugging Face text configuration")
    heads = int(text.num_attention_heads)
    kv_heads = int(getattr(text, "num_key_value_heads", heads))
    head_dim = getattr(text, "head_dim", None)
    head_dim = int(text.hidden_size) // heads if head_dim is None else int(head_dim)
    layers = int(getattr(text, "num_hidden_layers", getattr(text, "num_layers", 0)))
    if layers <= 0:
        raise ValueError("model text configuration has no positive layer count")
    if heads <= 0 or kv_heads <= 0:
        raise ValueError("model attention head counts must be positive")
    if heads % kv_heads:
        raise ValueError("model query heads are not divisible by KV heads")
    if head_dim <= 0 or head_dim % 2:
        raise ValueError("model attention head dimension must be positive and even")

    parameters = getattr(text, "rope_parameters", None)
    theta = getattr(text, "rope_theta", None)
    if theta is None and isinstance(parameters, Mapping):
        theta = parameters.get("rope_theta")
    theta = 10000.0 if theta is None else float(theta)

    return ModelShape(
        model_type=str(getattr(text, "model_type", "")),
        num_layers=layers,
        num_attention_heads=heads,
        num_kv_heads=kv_heads,
        head_dim=head_dim,
        rope_theta=theta,
        has_rope_scaling=_scaled(getattr(text, "rope_scaling", None)) or _scaled(parameters),
        rotary_dim=_rotary_dim(text, head_dim, parameters),
        attention_layer_indices=_attention_layers(getattr(text, "layer_types", None), layers),
    )


def _rotary_dim(text: Any, head_dim: int, parameters: Any) -> int:
    value = getattr(text, "rotary_dim", None)
    if value is None and isinstance(parameters, Mapping):
        value = parameters.get("rope_dim")
    if value is None:
        factor = getattr(text, "partial_rotary_factor", None)
        if factor is None and isinstance(parameters, Mapping):
            factor = parameters.get("partial_rotary_factor")
        value = head_dim if factor is None else int(head_dim * float(factor))
    value = int(value)
    if value <= 0 or value > head_dim or value % 2:
        raise ValueError(
            "model rotary dimension must be positive, even, and no larger than the attention head dimension"
        )
    return value


def _attention_layers(layer_types: Any, layers: int) -> tuple[int, ...]:
    if layer_types is None:
        return tuple(range(layers))
    if len(layer_types) != layers:
        raise ValueError("model layer_types length does not match layer count")
    unknown = sorted(set(layer_types) - _LAYER_TYPES)
    if unknown:
        raise ValueError("unsupported model layer types: " + ", ".join(unknown))
    full = tuple(i for i, kind in enumerate(layer_types) if kind == "full_attention")
    if not full:
        raise ValueError("model exposes no full-attention layers")
    return full


def _scaled(parameters: Any) -> bool:
    """Whether a rope_scaling / rope_parameters entry changes the default RoPE."""
    if not parameters:
        return False
    if not isinstance(parameters, Mapping):
        return True
    kind = parameters.get("rope_type", parameters.get("type", "default")) or "default"
    return str(kind) != "default" or bool(set(parameters) - _UNSCALED_ROPE_KEYS)
