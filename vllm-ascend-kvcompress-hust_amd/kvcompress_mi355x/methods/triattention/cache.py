"""Paged-cache slot arithmetic and K/V materialisation on the GPU (tri/cache.py).

``token_slots``, ``gather_paged_tokens`` / ``gather_paged_range`` and
``materialize_token_slots`` keep the reference names and contracts
(tri/cache.py:9-15,48-76,100-112); ``materialize_selected_tokens`` keeps
tri/cache.py:79-97.  The fast path used by the compression step is
``compact_layers``: one launch moves the kept rows of every layer.
"""

from __future__ import annotations

import torch

from ... import _native
from . import _device as dev


def token_slots(block_ids: torch.Tensor, token_indices: torch.Tensor, block_size: int) -> torch.Tensor:
    """Logical token -> flat physical slot (tri/cache.py:9-15)."""
    dev.require_hip(block_ids, "block_ids")
    dev.require_hip(token_indices, "token_indices")
    blocks = block_ids.to(torch.int64).contiguous()
    tokens = token_indices.to(torch.int64).contiguous()
    if tokens.numel() and int(tokens.max()) >= blocks.numel() * block_size:
        raise IndexError("token index outside the block table")
    out = torch.empty_like(tokens)
    _native.call(
        "kvc_token_slots",
        dev.stream_handle(tokens.device),
        dev.ptr(blocks),
        int(blocks.numel()),
        dev.ptr(tokens),
        int(tokens.numel()),
        int(block_size),
        dev.ptr(out),
    )
    return out


def gather_paged_tokens(
    cache: torch.Tensor, block_ids: torch.Tensor, token_indices: torch.Tensor, block_size: int
) -> torch.Tensor:
    """Rows of logical tokens from ``[blocks, block, heads, dim]`` storage as a
    dense ``[tokens, heads, dim]`` tensor (tri/cache.py:48-58).  A helper for
    callers of the reference's torch path: the compression step reads pages in
    its kernels and never gathers."""
    if cache.ndim != 4 or cache.shape[1] != block_size:
        raise ValueError("cache must use [blocks, block, heads, dim] layout")
    dev.require_hip(cache, "cache")
    slots = token_slots(block_ids, token_indices, block_size)
    return cache[torch.div(slots, block_size, rounding_mode="floor"), torch.remainder(slots, block_size)]


def gather_paged_range(
    cache: torch.Tensor, block_ids: torch.Tensor, *, start: int, count: int, block_size: int
) -> torch.Tensor:
    """One contiguous logical range of tokens (tri/cache.py:61-76)."""
    indices = torch.arange(start, start + count, device=block_ids.device, dtype=torch.long)
    return gather_paged_tokens(cache, block_ids, indices, block_size)


def _cache_geometry(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int]:
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride() or k_cache.dtype != v_cache.dtype:
        raise ValueError("K and V caches must share shape, strides and dtype")
    dev.validate_cache(k_cache, "k_cache", int(k_cache.shape[1]))
    dev.validate_cache(v_cache, "v_cache", int(v_cache.shape[1]))
    row_elems = int(k_cache.shape[2] * k_cache.shape[3])
    return int(k_cache.shape[0]), int(k_cache.stride(0)), row_elems


def materialize_token_slots(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    k_workspace: torch.Tensor,
    v_workspace: torch.Tensor,
) -> None:
    """Gather rows into the workspaces, then scatter them: safe for any overlap."""
    num_pages, page_stride, row_elems = _cache_geometry(k_cache, v_cache)
    if int(k_cache.shape[1]) != 128:
        raise ValueError("the HIP materialiser addresses 128-token cache blocks")
    src = source_slots.to(torch.int64).contiguous()
    dst = destination_slots.to(torch.int64).contiguous()
    n = int(src.numel())
    if int(dst.numel()) != n:
        raise ValueError("source and destination slot counts differ")
    for name, ws in (("k_workspace", k_workspace), ("v_workspace", v_workspace)):
        dev.require_hip(ws, name)
        if not ws.is_contiguous() or ws.numel() * ws.element_size() < n * row_elems * 2:
            raise ValueError(f"{name} must be contiguous and hold every gathered row")
    _native.call(
        "kvc_materialize_slots",
        dev.stream_handle(k_cache.device),
        dev.ptr(k_cache),
        dev.ptr(v_cache),
        num_pages,
        page_stride,
        row_elems,
        2,
        dev.ptr(src),
        dev.ptr(dst),
        n,
        dev.ptr(k_workspace),
        dev.ptr(v_workspace),
    )


def materialize_selected_tokens(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    source_block_ids: torch.Tensor,
    destination_block_ids: torch.Tensor,
    keep_indices: torch.Tensor,
    block_size: int,
) -> None:
    """Write kept tokens densely into the destination blocks (tri/cache.py:79-97)."""
    src = token_slots(source_block_ids, keep_indices, block_size)
    dense = torch.arange(keep_indices.numel(), device=keep_indices.device, dtype=torch.int64)
    dst = token_slots(destination_block_ids, dense, block_size)
    row = (keep_indices.numel(),) + tuple(k_cache.shape[2:])
    k_ws = torch.empty(row, dtype=k_cache.dtype, device=k_cache.device)
    v_ws = torch.empty_like(k_ws)
    materialize_token_slots(k_cache, v_cache, src, dst, k_ws, v_ws)


def compact_layers(
    k_layer_ptrs: torch.Tensor,
    v_layer_ptrs: torch.Tensor,
    *,
    num_pages: int,
    page_stride: int,
    row_elems: int,
    seq_lens: torch.Tensor,
    src_block_offsets: torch.Tensor,
    src_block_ids: torch.Tensor,
    dst_block_offsets: torch.Tensor | None,
    dst_block_ids: torch.Tensor | None,
    keep: torch.Tensor,
    budget: int,
    workspace: torch.Tensor | None = None,
    layer_order: str = "layer_major",
) -> None:
    """Move every layer's kept K/V rows (``dst_block_ids`` None = in place).

    ``workspace`` (uint8, at least :func:`compact_workspace_bytes`) lets a
    batch of up to 32 sequences resolve its rows once and move them one layer
    per workgroup (in place: the rows after the ordered walk), dispatched
    ``layer_order`` = "layer_major" (one layer after the other) or
    "interleaved" (every layer's workgroups interleaved); without it every
    workgroup walks all layers.  The caches end up identical either way."""
    orders = {"layer_major": _native.COMPACT_LAYER_MAJOR, "interleaved": _native.COMPACT_LAYERS_INTERLEAVED}
    if layer_order not in orders:
        raise ValueError(f"unknown layer order {layer_order!r}")
    n_layers = int(k_layer_ptrs.numel())
    if int(v_layer_ptrs.numel()) != n_layers:
        raise ValueError("K and V layer tables differ in length")
    n_seq = int(seq_lens.numel())
    _native.call(
        "kvc_compact",
        dev.stream_handle(keep.device),
        n_layers,
        dev.ptr(k_layer_ptrs),
        dev.ptr(v_layer_ptrs),
        int(num_pages),
        int(page_stride),
        int(row_elems),
        2,
        n_seq,
        dev.ptr(seq_lens),
        dev.ptr(src_block_offsets),
        dev.ptr(src_block_ids),
        dev.ptr(dst_block_offsets),
        dev.ptr(dst_block_ids),
        dev.ptr(keep),
        int(keep.stride(0)),
        int(budget),
        dev.ptr(workspace),
        0 if workspace is None else int(workspace.numel() * workspace.element_size()),
        orders[layer_order],
    )


def compact_workspace_bytes(n_seq: int, budget: int) -> int:
    """Bytes of the optional :func:`compact_layers` workspace for a batch."""
    return int(_native.load().kvc_compact_workspace_bytes(int(n_seq), int(budget)))


def rewrite_block_tables(
    *,
    budget: int,
    src_block_offsets: torch.Tensor,
    src_block_ids: torch.Tensor,
    src_lengths: list[int],
    dst_block_offsets: torch.Tensor | None,
    dst_block_ids: torch.Tensor | None,
    block_size: int = 128,
    buffers: dict | None = None,
) -> tuple[torch.Tensor, list[torch.Tensor]]:
    """New per-sequence tables and released pages (reversed, as the scheduler
    frees them).  ``buffers`` (a dict owned by the caller) keeps the output
    buffers of a batch alive across calls so repeated steps allocate nothing."""
    n_seq = len(src_lengths)
    device = src_block_ids.device
    nb = (budget + block_size - 1) // block_size
    inplace = dst_block_ids is None
    key = (budget, inplace)
    if buffers is not None and key in buffers:
        tables, freed, freed_offsets, offsets = buffers[key]
    else:
        freed_counts = [(n - min(nb, n)) if inplace else n for n in src_lengths]
        offsets = [0]
        for c in freed_counts:
            offsets.append(offsets[-1] + c)
        freed_offsets = torch.tensor(offsets, dtype=torch.int64, device=device)
        freed = torch.empty(max(offsets[-1], 1), dtype=torch.int64, device=device)
        tables = torch.empty((n_seq, nb), dtype=torch.int64, device=device)
        if buffers is not None:
            buffers[key] = (tables, freed, freed_offsets, offsets)
    _native.call(
        "kvc_rewrite_block_tables",
        dev.stream_handle(device),
        n_seq,
        int(budget),
        dev.ptr(src_block_offsets),
        dev.ptr(src_block_ids),
        dev.ptr(dst_block_offsets),
        dev.ptr(dst_block_ids),
        dev.ptr(tables),
        dev.ptr(freed_offsets),
        dev.ptr(freed),
    )
    return tables, [freed[offsets[i] : offsets[i + 1]] for i in range(n_seq)]


def expand_scheduler_block_ids(block_ids: torch.Tensor, cache_blocks_per_scheduler_block: int) -> torch.Tensor:
    """Scheduler page id -> consecutive 128-token cache blocks (pkg/provider.py:1273-1287)."""
    dev.require_hip(block_ids, "block_ids")
    ids = block_ids.to(torch.int64).contiguous()
    k = int(cache_blocks_per_scheduler_block)
    if k <= 0:
        raise ValueError("cache blocks per scheduler block must be positive")
    if k == 1:
        return ids
    out = torch.empty(ids.numel() * k, dtype=torch.int64, device=ids.device)
    _native.call("kvc_expand_block_ids", dev.stream_handle(ids.device), dev.ptr(ids), int(ids.numel()), k, dev.ptr(out))
    return out
