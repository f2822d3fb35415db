"""Keep-set selection on the GPU (select_keep_indices, tri/selection.py:108-196).

Same signature, validation and result contract as the reference: ``budget``
sorted int64 indices, protected prefix/recent windows always kept, ``global``
keeps the top scores of the rest, ``v3`` distributes eviction over equal
middle segments with integer quotas.  Ties at the selection threshold are
broken towards the lower index (torch.topk leaves tie order unspecified).
"""

from __future__ import annotations

import torch

from ... import _native
from . import _device as dev

POLICY_CODES = {"global": _native.POLICY_GLOBAL, "v3": _native.POLICY_V3}


def validate_selection(
    token_count: int, *, budget: int, protected_prefix: int, protected_recent: int, segments: int, policy: str
) -> None:
    """Host-side checks of tri/selection.py:123-133,161-163."""
    if budget <= 0 or budget > token_count:
        raise ValueError("budget must be in [1, token_count]")
    if protected_prefix < 0 or protected_recent < 0:
        raise ValueError("protected windows must be non-negative")
    if protected_prefix + protected_recent > budget:
        raise ValueError("protected windows cannot exceed the selection budget")
    if segments <= 0:
        raise ValueError("segments must be positive")
    if policy not in POLICY_CODES:
        raise ValueError(f"unsupported position policy: {policy}")
    if policy == "v3":
        prefix = min(protected_prefix, token_count)
        recent = min(protected_recent, token_count - prefix)
        if token_count - budget > token_count - prefix - recent:
            raise ValueError("selection budget leaves too few slots for protected tokens")


def select_keep_indices(
    scores: torch.Tensor,
    *,
    budget: int,
    protected_prefix: int,
    protected_recent: int,
    segments: int,
    policy: str,
) -> torch.Tensor:
    if scores.ndim != 1:
        raise ValueError("scores must be one-dimensional")
    dev.require_hip(scores, "scores")
    token_count = int(scores.numel())
    validate_selection(
        token_count,
        budget=budget,
        protected_prefix=protected_prefix,
        protected_recent=protected_recent,
        segments=segments,
        policy=policy,
    )
    values = scores.to(dtype=torch.float32).contiguous()
    device = values.device
    keep = torch.empty(budget, dtype=torch.int64, device=device)
    seq_lens = torch.tensor([token_count], dtype=torch.int32, device=device)
    token_offsets = torch.tensor([0, token_count], dtype=torch.int64, device=device)
    _native.call(
        "kvc_select_keep",
        dev.stream_handle(device),
        1,
        token_count,
        dev.ptr(seq_lens),
        dev.ptr(token_offsets),
        dev.ptr(values),
        int(budget),
        int(protected_prefix),
        int(protected_recent),
        int(segments),
        POLICY_CODES[policy],
        dev.ptr(keep),
        int(budget),
    )
    return keep


def select_keep_indices_batched(
    scores: torch.Tensor,
    seq_lens: torch.Tensor,
    token_offsets: torch.Tensor,
    seq_lens_host: list[int],
    keep: torch.Tensor,
    *,
    budget: int,
    protected_prefix: int,
    protected_recent: int,
    segments: int,
    policy: str,
) -> torch.Tensor:
    """All sequences of a batch in one launch; ``keep`` is int64 [n_seq, >= budget]."""
    for n in seq_lens_host:
        validate_selection(
            n,
            budget=budget,
            protected_prefix=protected_prefix,
            protected_recent=protected_recent,
            segments=segments,
            policy=policy,
        )
    n_seq = len(seq_lens_host)
    if keep.ndim != 2 or keep.shape[0] < n_seq or keep.shape[1] < budget or keep.stride(1) != 1:
        raise ValueError("keep must be int64 [n_seq, >= budget] with contiguous rows")
    _native.call(
        "kvc_select_keep",
        dev.stream_handle(scores.device),
        n_seq,
        max(seq_lens_host),
        dev.ptr(seq_lens),
        dev.ptr(token_offsets),
        dev.ptr(scores),
        int(budget),
        int(protected_prefix),
        int(protected_recent),
        int(segments),
        POLICY_CODES[policy],
        dev.ptr(keep),
        int(keep.stride(0)),
    )
    return keep
