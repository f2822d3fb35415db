"""Method-facing model shape from a Hugging Face text configuration.

The shape a compression method binds against (ModelShape) is read from the
host's model config, which exposes the Hugging Face text config as
``hf_text_config`` (or ``hf_config``).  Which configuration keys feed which
field is the interface of model_shape_from_config (pkg/model.py:12-109):

  num_attention_heads   num_attention_heads
  num_kv_heads          num_key_value_heads, else the query head count
  head_dim              head_dim, else hidden_size // num_attention_heads
  num_layers            num_hidden_layers, else num_layers
  rope_theta            rope_theta, else rope_parameters["rope_theta"], else 10000
  rotary_dim            rotary_dim, else rope_parameters["rope_dim"], else
                        head_dim * partial_rotary_factor (attribute, then
                        rope_parameters), else head_dim
  layer indices         the "full_attention" entries of layer_types (hybrid
                        models also have "linear_attention"), else every layer
  has_rope_scaling      rope_scaling or rope_parameters names a RoPE type other
                        than "default" or carries any key besides rope_theta,
                        rope_type and type (a non-mapping value counts too)

Inconsistent configurations raise ValueError.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

from .methods.base import ModelShape

_KNOWN_LAYER_TYPES = ("full_attention", "linear_attention")
_PLAIN_ROPE_KEYS = frozenset({"rope_theta", "rope_type", "type"})


class _TextConfigView:
    """Lookups over a Hugging Face text config: attributes first, then the keys
    of its ``rope_parameters`` mapping (transformers v5 moved RoPE settings
    there); None counts as absent."""

    def __init__(self, text: Any) -> None:
        self.text = text
        rope = getattr(text, "rope_parameters", None)
        self.rope = rope if isinstance(rope, Mapping) else {}

    def attr(self, *names: str) -> Any:
        for name in names:
            value = getattr(self.text, name, None)
            if value is not None:
                return value
        return None

    def setting(self, attribute: str, rope_key: str | None = None) -> Any:
        value = self.attr(attribute)
        if value is None and rope_key is not None:
            value = self.rope.get(rope_key)
        return value


def _rope_entry_is_scaled(entry: Any) -> bool:
    if not entry:
        return False
    if not isinstance(entry, Mapping):
        return True
    kind = entry.get("rope_type", entry.get("type", "default")) or "default"
    return str(kind) != "default" or any(key not in _PLAIN_ROPE_KEYS for key in entry)


def _full_attention_layers(layer_types: Any, num_layers: int) -> tuple[int, ...]:
    if layer_types is None:
        return tuple(range(num_layers))
    kinds = list(layer_types)
    if len(kinds) != num_layers:
        raise ValueError("model layer_types length does not match layer count")
    unknown = sorted({kind for kind in kinds if kind not in _KNOWN_LAYER_TYPES})
    if unknown:
        raise ValueError("unsupported model layer types: " + ", ".join(unknown))
    full = tuple(index for index, kind in enumerate(kinds) if kind == "full_attention")
    if not full:
        raise ValueError("model exposes no full-attention layers")
    return full


def _rotary_dim(view: _TextConfigView, head_dim: int) -> int:
    explicit = view.setting("rotary_dim", "rope_dim")
    if explicit is not None:
        rotary = int(explicit)
    else:
        factor = view.setting("partial_rotary_factor", "partial_rotary_factor")
        rotary = head_dim if factor is None else int(head_dim * float(factor))
    if not (0 < rotary <= head_dim and rotary % 2 == 0):
        raise ValueError("model rotary dimension must be positive, even and no larger than the attention head dimension")
    return rotary


def model_shape_from_config(model_config: Any) -> ModelShape:
    """ModelShape of a host model config exposing ``hf_text_config`` or ``hf_config``."""
    text = getattr(model_config, "hf_text_config", None)
    if text is None:
        text = getattr(model_config, "hf_config", None)
    if text is None:
        raise ValueError("model has no Hugging Face text configuration")
    view = _TextConfigView(text)
    heads = int(text.num_attention_heads)
    kv_heads = view.attr("num_key_value_heads")
    kv_heads = heads if kv_heads is None else int(kv_heads)
    head_dim = view.attr("head_dim")
    head_dim = int(text.hidden_size) // heads if head_dim is None else int(head_dim)
    layers = view.attr("num_hidden_layers", "num_layers")
    num_layers = 0 if layers is None else int(layers)

    for broken, message in (
        (num_layers <= 0, "model text configuration has no positive layer count"),
        (heads <= 0 or kv_heads <= 0, "model attention head counts must be positive"),
        (heads > 0 and kv_heads > 0 and heads % kv_heads != 0, "model query heads are not divisible by KV heads"),
        (head_dim <= 0 or head_dim % 2 != 0, "model attention head dimension must be positive and even"),
    ):
        if broken:
            raise ValueError(message)

    theta = view.setting("rope_theta", "rope_theta")
    return ModelShape(
        model_type=str(view.attr("model_type") or ""),
        num_layers=num_layers,
        num_attention_heads=heads,
        num_kv_heads=kv_heads,
        head_dim=head_dim,
        rope_theta=10000.0 if theta is None else float(theta),
        has_rope_scaling=any(
            _rope_entry_is_scaled(entry)
            for entry in (getattr(text, "rope_scaling", None), getattr(text, "rope_parameters", None))
        ),
        rotary_dim=_rotary_dim(view, head_dim),
        attention_layer_indices=_full_attention_layers(getattr(text, "layer_types", None), num_layers),
    )
