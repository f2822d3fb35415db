"""TriAttention method options (the option contract of tri/config.py:18-198).

The options, their defaults and what each accepts are the reference's: the
budget, recompute window and score chunk are positive multiples of the
128-token block, the protected windows are non-negative and fit in the budget
together, segments and layer stride are positive.  Here they are one schema
table, parsed in table order, followed by the cross-option rules in a fixed
order, so the first problem found is the one reported and its message is the
reference's.  Calibration-generation options are parsed and stored for the
calibration step.
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from dataclasses import dataclass
from pathlib import Path
from typing import Literal

from ...config import KERNEL_BLOCK_SIZE, JsonScalar, require_bool, require_choice, require_int

ScoreAggregation = Literal["mean", "max"]
LayerAggregation = Literal["mean", "max"]
PositionPolicy = Literal["global", "v3"]


@dataclass(frozen=True)
class _Option:
    """One method option: how its value is read and what it defaults to."""

    name: str
    kind: str  # "path", "optional_path", "text", "bool", "int" or "choice"
    default: JsonScalar = None
    choices: frozenset[str] = frozenset()

    def read(self, options: Mapping[str, JsonScalar]) -> object:
        if self.kind in ("path", "optional_path", "text"):
            value = options.get(self.name, self.default)
            if value is None and self.kind == "optional_path":
                return None
            if not isinstance(value, str) or not value.strip():
                raise ValueError(f"method option {self.name!r} must be a non-empty string")
            return value.strip() if self.kind == "text" else Path(value).expanduser()
        if self.kind == "bool":
            return require_bool(options, self.name, bool(self.default))
        if self.kind == "int":
            return require_int(options, self.name, int(self.default))
        return require_choice(options, self.name, str(self.default), set(self.choices))


_SCHEMA: tuple[_Option, ...] = (
    _Option("stats_path", "path"),
    _Option("calibration_input_path", "optional_path"),
    _Option("calibration_device", "text", "auto"),
    _Option("auto_calibrate", "bool", True),
    _Option("calibration_max_length", "int", 4096),
    _Option("calibration_attn_implementation", "choice", "eager", frozenset({"eager", "sdpa", "flash_attention_2"})),
    _Option("calibration_local_files_only", "bool", False),
    _Option("kv_budget", "int", 2048),
    _Option("recompute_window", "int", KERNEL_BLOCK_SIZE),
    _Option("position_policy", "choice", "global", frozenset({"global", "v3"})),
    _Option("protected_prefix_window", "int", 0),
    _Option("protected_recent_window", "int", KERNEL_BLOCK_SIZE),
    _Option("position_segments", "int", 8),
    _Option("score_aggregation", "choice", "mean", frozenset({"mean", "max"})),
    _Option("layer_aggregation", "choice", "mean", frozenset({"mean", "max"})),
    _Option("score_chunk_size", "int", 512),
    _Option("score_layer_stride", "int", 8),
    _Option("min_output_tokens_for_compression", "int", 0),
)

KNOWN_OPTIONS = frozenset(option.name for option in _SCHEMA)

# Options that count tokens in whole 128-token kernel blocks.
_BLOCK_MULTIPLES = ("kv_budget", "recompute_window", "score_chunk_size")
_PROTECTED_WINDOWS = ("protected_prefix_window", "protected_recent_window")


@dataclass(frozen=True)
class TriAttentionConfig:
    stats_path: Path
    auto_calibrate: bool = True
    calibration_input_path: Path | None = None
    calibration_max_length: int = 4096
    calibration_device: str = "auto"
    calibration_attn_implementation: str = "eager"
    calibration_local_files_only: bool = False
    kv_budget: int = 2048
    recompute_window: int = KERNEL_BLOCK_SIZE
    position_policy: PositionPolicy = "global"
    protected_prefix_window: int = 0
    protected_recent_window: int = KERNEL_BLOCK_SIZE
    position_segments: int = 8
    score_aggregation: ScoreAggregation = "mean"
    layer_aggregation: LayerAggregation = "mean"
    score_chunk_size: int = 512
    score_layer_stride: int = 8
    min_output_tokens_for_compression: int = 0

    @property
    def compression_threshold_tokens(self) -> int:
        return self.kv_budget + self.recompute_window

    @classmethod
    def from_method_config(cls, method_config: Mapping[str, JsonScalar]) -> TriAttentionConfig:
        unknown = sorted(set(method_config) - KNOWN_OPTIONS)
        if unknown:
            raise ValueError("unknown TriAttention method options: " + ", ".join(unknown))
        config = cls(**{option.name: option.read(method_config) for option in _SCHEMA})
        config.validate()
        return config

    def problems(self) -> Iterator[str]:
        """The rules the options break, in the order they are checked."""
        for name in _BLOCK_MULTIPLES:
            value = getattr(self, name)
            if value <= 0 or value % KERNEL_BLOCK_SIZE:
                yield f"method option {name!r} must be a positive multiple of {KERNEL_BLOCK_SIZE}"
        for name in _PROTECTED_WINDOWS:
            value = getattr(self, name)
            if value < 0:
                yield f"method option {name!r} must be non-negative"
            if value > self.kv_budget:
                yield f"method option {name!r} cannot exceed 'kv_budget'"
        if self.protected_prefix_window + self.protected_recent_window > self.kv_budget:
            yield "protected prefix and recent windows cannot exceed 'kv_budget'"
        if self.position_segments <= 0:
            yield "method option 'position_segments' must be positive"
        if self.score_layer_stride <= 0:
            yield "method option 'score_layer_stride' must be positive"
        if self.min_output_tokens_for_compression < 0:
            yield "method option 'min_output_tokens_for_compression' must be non-negative"
        if self.calibration_max_length < 128:
            yield "method option 'calibration_max_length' must be at least 128"

    def validate(self) -> None:
        for problem in self.problems():
            raise ValueError(problem)
