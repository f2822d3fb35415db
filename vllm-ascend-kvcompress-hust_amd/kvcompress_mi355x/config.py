"""Shared constants and option parsing helpers (pkg/config.py:13-22,173-190)."""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any, TypeAlias

# Tokens per kernel cache block.  The reference calls it ASCEND_BLOCK_SIZE
# (pkg/config.py:18); the name is kept so reference-side code imports unchanged.
KERNEL_BLOCK_SIZE = 128
ASCEND_BLOCK_SIZE = KERNEL_BLOCK_SIZE
PROVIDER_NAME = "ascend_kvcompress"
DEFAULT_METHOD = "triattention"

JsonScalar: TypeAlias = str | int | float | bool | None


def require_int(options: Mapping[str, Any], name: str, default: int) -> int:
    """Integer option; booleans are rejected even though bool subclasses int."""
    value = options.get(name, default)
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError(f"method option {name!r} must be an integer")
    return value


def require_choice(options: Mapping[str, Any], name: str, default: str, choices: set[str]) -> str:
    value = options.get(name, default)
    if not isinstance(value, str) or value not in choices:
        raise ValueError(f"method option {name!r} must be one of: {', '.join(sorted(choices))}")
    return value


def require_bool(options: Mapping[str, Any], name: str, default: bool) -> bool:
    value = options.get(name, default)
    if not isinstance(value, bool):
        raise ValueError(f"method option {name!r} must be a boolean")
    return value
