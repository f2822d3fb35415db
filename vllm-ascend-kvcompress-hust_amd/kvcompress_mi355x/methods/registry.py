"""Name -> factory registry of compression methods (pkg/methods/registry.py:13-106).

Same fail-closed behaviour as the reference: duplicate names, unknown names,
factories returning something that is not a KVCompressionMethod, and methods
whose ``name`` differs from the registered name are all rejected.  Methods
may also be published through the reference's entry-point group.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from importlib.metadata import entry_points
from typing import Any, TypeAlias

from ..config import JsonScalar
from .base import KVCompressionMethod, ModelShape

MethodFactory: TypeAlias = Callable[[Mapping[str, JsonScalar], Any, ModelShape], KVCompressionMethod]
METHOD_ENTRY_POINT_GROUP = "vllm_ascend_kvcompress.methods"


def _normalize_name(name: str) -> str:
    if not isinstance(name, str) or not name.strip():
        raise ValueError("compression method name must be a non-empty string")
    normalized = name.strip().lower()
    if not normalized.replace("_", "").replace("-", "").isalnum():
        raise ValueError("compression method names may contain only letters, digits, '-' and '_'")
    return normalized


class MethodRegistry:
    """Registry used by the compression step to create its method."""

    def __init__(self) -> None:
        self._factories: dict[str, MethodFactory] = {}

    def register(self, name: str, factory: MethodFactory) -> None:
        key = _normalize_name(name)
        if key in self._factories:
            raise ValueError(f"compression method {key!r} is already registered")
        if not callable(factory):
            raise TypeError("compression method factory must be callable")
        self._factories[key] = factory

    def create(
        self,
        name: str,
        options: Mapping[str, JsonScalar],
        vllm_config: Any,
        model_shape: ModelShape,
    ) -> KVCompressionMethod:
        key = _normalize_name(name)
        factory = self._factories.get(key)
        if factory is None:
            known = ", ".join(self.names()) or "<none>"
            raise ValueError(f"unknown compression method {key!r}; available: {known}")
        method = factory(options, vllm_config, model_shape)
        if not isinstance(method, KVCompressionMethod):
            raise TypeError(
                f"compression method factory {key!r} returned {type(method).__name__}, "
                "expected KVCompressionMethod"
            )
        if method.name != key:
            raise ValueError(
                f"compression method factory {key!r} returned method named {method.name!r}"
            )
        return method

    def names(self) -> tuple[str, ...]:
        return tuple(sorted(self._factories))


METHOD_REGISTRY = MethodRegistry()
_entry_points_loaded = False


def register_method(name: str, factory: MethodFactory) -> None:
    """Register an in-process method factory."""
    METHOD_REGISTRY.register(name, factory)


def load_method_entry_points() -> None:
    """Load third-party methods of the public entry-point group once."""
    global _entry_points_loaded
    if _entry_points_loaded:
        return
    _entry_points_loaded = True
    for entry in entry_points(group=METHOD_ENTRY_POINT_GROUP):
        METHOD_REGISTRY.register(entry.name, entry.load())


def create_method(
    name: str,
    options: Mapping[str, JsonScalar],
    vllm_config: Any,
    model_shape: ModelShape,
) -> KVCompressionMethod:
    load_method_entry_points()
    return METHOD_REGISTRY.create(name, options, vllm_config, model_shape)


def available_methods() -> tuple[str, ...]:
    load_method_entry_points()
    return METHOD_REGISTRY.names()
