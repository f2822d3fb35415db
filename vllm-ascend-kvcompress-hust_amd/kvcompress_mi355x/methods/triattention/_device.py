"""Small helpers shared by the HIP wrappers: device checks, streams, descriptors."""

from __future__ import annotations

import functools

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


@functools.lru_cache(maxsize=256)
def _one_sequence_descriptor(device_index: int, layer_ptr: int, num_tokens: int, n_blocks: int) -> torch.Tensor:
    signed = layer_ptr - (1 << 64) if layer_ptr >= (1 << 63) else layer_ptr
    # int64 words: [layer pointer, token offsets (0, n), block offsets (0, blocks), sequence length in the low half]
    return torch.tensor([signed, 0, num_tokens, 0, n_blocks, num_tokens], dtype=torch.int64,
                        device=torch.device("cuda", device_index))


def one_sequence_descriptor(layer: torch.Tensor, num_tokens: int, n_blocks: int) -> dict[str, int]:
    """Device addresses of the batch descriptor of a one-layer, one-sequence
    launch (layer pointer table, token and block offsets, int32 sequence
    length), kept on the device per distinct value so that repeated calls
    copy nothing to the device.  The words are immutable once made."""
    t = _one_sequence_descriptor(layer.device.index, int(layer.data_ptr()), int(num_tokens), int(n_blocks))
    base = int(t.data_ptr())
    return {"layer_ptrs": base, "token_offsets": base + 8, "block_offsets": base + 24, "seq_lens": base + 40}
