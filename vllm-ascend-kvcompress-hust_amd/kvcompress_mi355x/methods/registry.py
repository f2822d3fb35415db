"""Compression methods by name, failing closed (the contract of
pkg/methods/registry.py:13-106).

A name is canonicalised once (stripped, lower-cased, letters, digits, '-' and
'_' only) and can be registered once.  Creating a method checks what the
factory produced: an unknown name, an object that is not a
KVCompressionMethod, or a method reporting a different name is an error.
Third-party methods arrive through the reference's entry-point group, read
the first time a method is created or listed.  The error types and messages
are the reference's, since callers match on them.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass
from importlib.metadata import entry_points
from typing import Any, TypeAlias

from ..config import JsonScalar
from .base import KVCompressionMethod, ModelShape

MethodFactory: TypeAlias = Callable[[Mapping[str, JsonScalar], Any, ModelShape], KVCompressionMethod]
METHOD_ENTRY_POINT_GROUP = "vllm_ascend_kvcompress.methods"

_NAME_PUNCTUATION = frozenset("-_")


def canonical_method_name(name: object) -> str:
    """The registry key of ``name``: at least one letter or digit, nothing
    but letters, digits, '-' and '_', compared lower-cased."""
    text = name.strip().lower() if isinstance(name, str) else ""
    if not text:
        raise ValueError("compression method name must be a non-empty string")
    has_alnum = any(ch.isalnum() for ch in text)
    if not has_alnum or any(not ch.isalnum() and ch not in _NAME_PUNCTUATION for ch in text):
        raise ValueError("compression method names may contain only letters, digits, '-' and '_'")
    return text


@dataclass(frozen=True)
class _Registration:
    factory: MethodFactory
    origin: str  # "in-process", or the entry point that published it


def _checked(key: str, method: object) -> KVCompressionMethod:
    """What a factory returned, accepted only as a method carrying its key."""
    if not isinstance(method, KVCompressionMethod):
        raise TypeError(
            f"compression method factory {key!r} returned {type(method).__name__}, expected KVCompressionMethod"
        )
    if method.name != key:
        raise ValueError(f"compression method factory {key!r} returned method named {method.name!r}")
    return method


class MethodRegistry:
    """Registry used by the compression step to create its method."""

    def __init__(self) -> None:
        self._entries: dict[str, _Registration] = {}

    def register(self, name: str, factory: MethodFactory, *, origin: str = "in-process") -> None:
        key = canonical_method_name(name)
        if key in self._entries:
            raise ValueError(f"compression method {key!r} is already registered")
        if not callable(factory):
            raise TypeError("compression method factory must be callable")
        self._entries[key] = _Registration(factory, origin)

    def names(self) -> tuple[str, ...]:
        return tuple(sorted(self._entries))

    def origin(self, name: str) -> str:
        """Where the method registered under ``name`` came from."""
        return self._entries[canonical_method_name(name)].origin

    def create(
        self,
        name: str,
        options: Mapping[str, JsonScalar],
        vllm_config: Any,
        model_shape: ModelShape,
    ) -> KVCompressionMethod:
        key = canonical_method_name(name)
        entry = self._entries.get(key)
        if entry is None:
            listed = ", ".join(self.names()) or "<none>"
            raise ValueError(f"unknown compression method {key!r}; available: {listed}")
        return _checked(key, entry.factory(options, vllm_config, model_shape))


class _EntryPointLoader:
    """Reads the entry-point group into a registry, once per process."""

    def __init__(self, group: str) -> None:
        self.group = group
        self.done = False

    def load_into(self, registry: MethodRegistry) -> None:
        if self.done:
            return
        self.done = True
        for entry in entry_points(group=self.group):
            registry.register(entry.name, entry.load(), origin=f"entry point {entry.value}")


METHOD_REGISTRY = MethodRegistry()
_ENTRY_POINTS = _EntryPointLoader(METHOD_ENTRY_POINT_GROUP)


def register_method(name: str, factory: MethodFactory) -> None:
    """Register an in-process method factory."""
    METHOD_REGISTRY.register(name, factory)


def load_method_entry_points() -> None:
    """Register the methods third parties publish through the entry-point group."""
    _ENTRY_POINTS.load_into(METHOD_REGISTRY)


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
