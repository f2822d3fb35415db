"""Small helpers shared by the HIP wrappers: device checks, streams, descriptors."""

from __future__ import annotations

from collections import OrderedDict

import torch

from ... import _native


def require_hip(tensor: torch.Tensor, name: str) -> None:
    """The compression path runs only on the GPU; there is no host fallback."""
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tensor.device.type != "cuda":
        raise ValueError(
            f"{name} is on {tensor.device}; the MI355X compression path needs HIP device tensors"
        )


def require_dtype(tensor: torch.Tensor, name: str, *dtypes: torch.dtype) -> None:
    if tensor.dtype not in dtypes:
        raise ValueError(f"{name} must have dtype {' or '.join(map(str, dtypes))}, got {tensor.dtype}")


def require_contiguous(tensor: torch.Tensor, name: str) -> None:
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else int(tensor.data_ptr())


def cache_dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _native.DTYPE_BF16
    if dtype == torch.float16:
        return _native.DTYPE_FP16
    raise ValueError(f"cache dtype {dtype} is unsupported (bf16 or fp16 only)")


def rope_style_code(style: str) -> int:
    if style == "half":
        return _native.ROPE_HALF
    if style == "interleaved":
        return _native.ROPE_INTERLEAVED
    raise ValueError(f"unsupported rope style {style!r}")


def validate_cache(cache: torch.Tensor, name: str, block_size: int = 128) -> None:
    """Reference cache contract (pkg/provider.py:1201-1230): [pages, 128, H, D]
    bf16/fp16, contiguous inner block, page stride at least one page."""
    require_hip(cache, name)
    if cache.ndim != 4 or cache.shape[1] != block_size:
        raise ValueError(f"{name} must have shape [pages, {block_size}, kv_heads, head_dim]")
    cache_dtype_code(cache.dtype)
    _, blk, heads, dim = cache.shape
    if cache.stride()[1:] != (heads * dim, dim, 1) or cache.stride(0) < blk * heads * dim:
        raise ValueError(f"{name} must have contiguous inner blocks and a non-overlapping page stride")


def require_16_byte_pages(cache: torch.Tensor, name: str) -> None:
    """The scorers read keys in 16-byte words, so every page must start on a
    16-byte boundary: the base address and the page stride in bytes must be
    multiples of 16.  The reference accepts any page stride of at least one
    page (pkg/provider.py:1224-1230); a stride padded by a multiple of 8
    elements (bf16/fp16), e.g. K and V interleaved in one [pages, 2, ...]
    buffer, passes; an odd padding such as 4 elements does not."""
    if cache.data_ptr() % 16 or (cache.stride(0) * cache.element_size()) % 16:
        raise ValueError(
            f"{name}: the HIP scorer reads 16-byte words; the cache base address and its page stride "
            f"({cache.stride(0)} elements) must be multiples of 16 bytes"
        )


def pointer_table(tensors: list[torch.Tensor], device: torch.device) -> torch.Tensor:
    """Device array of base addresses (uint64 stored in int64)."""
    values = [int(t.data_ptr()) for t in tensors]
    signed = [v - (1 << 64) if v >= (1 << 63) else v for v in values]
    return torch.tensor(signed, dtype=torch.int64, device=device)


def ragged(rows: list[torch.Tensor | list[int] | tuple[int, ...]], device: torch.device) -> tuple[torch.Tensor, torch.Tensor, list[int]]:
    """Concatenate int64 rows; return (offsets [n+1], flat ids, host lengths)."""
    lengths: list[int] = []
    parts: list[torch.Tensor] = []
    for row in rows:
        t = row if isinstance(row, torch.Tensor) else torch.tensor(list(row), dtype=torch.int64)
        t = t.to(device=device, dtype=torch.int64).reshape(-1)
        parts.append(t)
        lengths.append(int(t.numel()))
    offsets = [0]
    for n in lengths:
        offsets.append(offsets[-1] + n)
    flat = torch.cat(parts) if parts else torch.empty(0, dtype=torch.int64, device=device)
    return torch.tensor(offsets, dtype=torch.int64, device=device), flat.contiguous(), lengths


class DescriptorCache:
    """Device descriptors of one-sequence launches, one per distinct value.

    A descriptor is a small device tensor whose address goes into kernel
    launches; it must outlive every launch that reads it.  Entries made or
    used while the current stream is capturing a graph are pinned for the
    life of the cache (a replay reads the captured address at any later
    time); the others are kept least-recently-used, ``maxsize`` of them.  A
    descriptor used on a stream other than the one it was allocated on is
    recorded on that stream, so that evicting it cannot hand its memory to a
    new allocation while a kernel queued there still reads it.  ``make``,
    ``capturing`` and ``current_stream`` are injectable for host-only tests."""

    def __init__(self, maxsize: int = 256, *, make=None, capturing=None, current_stream=None) -> None:
        self.maxsize = int(maxsize)
        self._lru: OrderedDict = OrderedDict()
        self._pinned: dict = {}
        self._make = make or _make_descriptor
        self._capturing = capturing or torch.cuda.is_current_stream_capturing
        self._current_stream = current_stream or (lambda device: torch.cuda.current_stream(device))

    def __len__(self) -> int:
        return len(self._lru) + len(self._pinned)

    def pinned(self, key) -> bool:
        return key in self._pinned

    def get(self, key: tuple) -> torch.Tensor:
        entry = self._pinned.get(key)
        if entry is None:
            entry = self._lru.pop(key, None)
            if entry is None:
                tensor = self._make(key)
                entry = (tensor, self._current_stream(tensor.device))
            if self._capturing():
                self._pinned[key] = entry
            else:
                self._lru[key] = entry
                while len(self._lru) > self.maxsize:
                    self._lru.popitem(last=False)
        tensor, made_on = entry
        stream = self._current_stream(tensor.device)
        if stream != made_on:
            tensor.record_stream(stream)
        return tensor


def _make_descriptor(key: tuple) -> torch.Tensor:
    device_index, layer_ptr, num_tokens, n_blocks = key
    signed = layer_ptr - (1 << 64) if layer_ptr >= (1 << 63) else layer_ptr
    # int64 words: [layer pointer, token offsets (0, n), block offsets (0, blocks), sequence length in the low half]
    return torch.tensor([signed, 0, num_tokens, 0, n_blocks, num_tokens], dtype=torch.int64,
                        device=torch.device("cuda", device_index))


_DESCRIPTORS = DescriptorCache()


def one_sequence_descriptor(layer: torch.Tensor, num_tokens: int, n_blocks: int) -> dict:
    """Device addresses of the batch descriptor of a one-layer, one-sequence
    launch (layer pointer table, token and block offsets, int32 sequence
    length), kept on the device per distinct value so that repeated calls
    copy nothing to the device; ``"tensor"`` is the descriptor itself, for
    callers that hold on to their launch arguments.  The words are immutable
    once made."""
    t = _DESCRIPTORS.get((layer.device.index, int(layer.data_ptr()), int(num_tokens), int(n_blocks)))
    base = int(t.data_ptr())
    return {"tensor": t, "layer_ptrs": base, "token_offsets": base + 8, "block_offsets": base + 24, "seq_lens": base + 40}
