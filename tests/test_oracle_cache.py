"""Pin the oracle's slot arithmetic, materialisation and block-table rewrite
with the reference KATs (tests/test_cache.py:15-94) and commit semantics."""

from __future__ import annotations

import torch

from oracle import triattention_ref as ref


def test_gather_maps_tokens_through_block_table() -> None:
    cache = torch.arange(12, dtype=torch.float32).view(3, 4, 1, 1)
    got = ref.gather_paged_tokens(cache, torch.tensor([2, 0]), torch.tensor([0, 3, 4, 7]), 4)
    assert got.flatten().tolist() == [8.0, 11.0, 0.0, 3.0]


def test_overlapping_destination_is_gathered_first() -> None:
    k = torch.arange(16, dtype=torch.float32).view(4, 4, 1, 1)
    v = k.clone() + 100
    src, keep = torch.tensor([2, 0, 3]), torch.tensor([1, 4, 6, 9])
    want_k = ref.gather_paged_tokens(k, src, keep, 4).clone()
    want_v = ref.gather_paged_tokens(v, src, keep, 4).clone()
    ref.materialize_selected_tokens(k, v, src, torch.tensor([2]), keep, 4)
    assert torch.equal(k[2], want_k) and torch.equal(v[2], want_v)


def test_padded_pages_keep_unused_storage() -> None:
    bs, pages, heads, dim = 4, 4, 1, 2
    logical = bs * heads * dim
    stride = 2 * logical + 4
    raw = torch.full((pages * stride,), -1, dtype=torch.float16)
    shape, strides = (pages, bs, heads, dim), (stride, heads * dim, dim, 1)
    k = torch.as_strided(raw, shape, strides)
    v = torch.as_strided(raw, shape, strides, storage_offset=logical)
    k.copy_(torch.arange(pages * logical).view(shape))
    v.copy_(torch.arange(pages * logical).view(shape) + 100)
    src, keep = torch.tensor([2, 0, 3]), torch.tensor([1, 4, 6, 9])
    want_k = ref.gather_paged_tokens(k, src, keep, bs).clone()
    want_v = ref.gather_paged_tokens(v, src, keep, bs).clone()
    ref.materialize_selected_tokens(k, v, src, torch.tensor([2]), keep, bs)
    assert torch.equal(k[2], want_k) and torch.equal(v[2], want_v)
    s = ref.token_slots(torch.tensor([2]), torch.tensor([0, 1, 2, 3]), bs)
    d = ref.token_slots(torch.tensor([1]), torch.tensor([0, 1, 2, 3]), bs)
    ref.materialize_token_slots(k, v, s, d)
    assert torch.equal(k[1], want_k) and torch.equal(v[1], want_v)
    assert torch.equal(raw.view(pages, stride)[:, -4:], torch.full((pages, 4), -1, dtype=torch.float16))


def test_token_slots_closed_form() -> None:
    blocks = torch.tensor([7, 3, 9])
    tokens = torch.arange(384)
    got = ref.token_slots(blocks, tokens, 128)
    assert torch.equal(got, blocks[tokens // 128] * 128 + tokens % 128)


def test_block_table_rewrite_matches_commit_semantics() -> None:
    src = [11, 4, 7, 2, 9]
    assert ref.rewrite_block_table(src, [20, 21, 22], 256) == ([20, 21], [9, 2, 7, 4, 11])
    assert ref.rewrite_block_table(src, None, 256) == ([11, 4], [9, 2, 7])
    assert ref.rewrite_block_table(src, None, 257) == ([11, 4, 7], [9, 2])
