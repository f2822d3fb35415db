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

# kvc_select_keep runs one workgroup per (sequence, segment), about 10 us plus
# 0.7 us per 1K scores of the longest segment; kvc_select_keep_split (seven
# launches, chunks spread over the chip) takes 50-65 us for up to a few dozen
# segments: 4 x 130816 scores 66 us against 100 us, 16 x 16256 53 us against
# 23 us.  The crossover is near 64K scores per segment.
SPLIT_MIN_SEGMENT = 65536
SPLIT_MAX_JOBS = 32


def prefers_split(seq_lens_host: list[int], *, protected_prefix: int, protected_recent: int, segments: int, policy: str) -> bool:
    """Whether the chunked launch shape suits this batch: few jobs, long segments."""
    per_seq = segments if policy == "v3" else 1
    longest = max(seq_lens_host) - protected_prefix - protected_recent
    return len(seq_lens_host) * per_seq <= SPLIT_MAX_JOBS and longest // per_seq >= SPLIT_MIN_SEGMENT


def select_workspace(n_seq: int, segments: int, policy: str, device: torch.device) -> torch.Tensor:
    """Scratch of the chunked launch shape for up to ``n_seq`` sequences."""
    size = int(_native.load().kvc_select_workspace_bytes(n_seq, segments, POLICY_CODES[policy]))
    return torch.empty(max(size, 16), dtype=torch.uint8, device=device)


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
    keep = torch.empty((1, budget), dtype=torch.int64, device=device)
    seq_lens = torch.tensor([token_count], dtype=torch.int32, device=device)
    token_offsets = torch.tensor([0, token_count], dtype=torch.int64, device=device)
    select_keep_indices_batched(
        values,
        seq_lens,
        token_offsets,
        [token_count],
        keep,
        budget=budget,
        protected_prefix=protected_prefix,
        protected_recent=protected_recent,
        segments=segments,
        policy=policy,
    )
    return keep[0]


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
    shape: str = "auto",
    workspace: torch.Tensor | None = None,
    validate: bool = True,
) -> torch.Tensor:
    """All sequences of a batch at once; ``keep`` is int64 [n_seq, >= budget].

    ``shape``: "auto" (``prefers_split``), "single" (one workgroup per
    sequence segment) or "split" (chunked; ``workspace`` from
    ``select_workspace``, allocated here when None).  Both shapes return the
    same indices.  ``validate=False`` skips the per-sequence host checks for a
    caller that has made them already."""
    for n in seq_lens_host if validate else ():
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
    if shape not in ("auto", "single", "split"):
        raise ValueError(f"unknown selection launch shape {shape!r}")
    if shape == "auto":
        shape = "split" if prefers_split(
            seq_lens_host, protected_prefix=protected_prefix, protected_recent=protected_recent,
            segments=segments, policy=policy,
        ) else "single"
    args = (
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
    if shape == "single":
        _native.call("kvc_select_keep", *args)
        return keep
    if workspace is None:
        workspace = select_workspace(n_seq, segments, policy, scores.device)
    _native.call("kvc_select_keep_split", *args, dev.ptr(workspace), int(workspace.numel()))
    return keep
