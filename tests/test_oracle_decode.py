"""Pin the oracle's decode-side arithmetic after compaction: physical
positions and attention lengths (reference KATs) and the slot mapping brute
force (hand-worked block-table cases)."""

from __future__ import annotations

import torch

from oracle import brute
from oracle import triattention_ref as ref


def test_shift_positions_reference_kat() -> None:
    # tests/run_npu_kernel_smoke.py:29-36 of the reference.
    got = ref.shift_positions(
        torch.tensor([300, 20, 301]), torch.tensor([0, 1, 0]), torch.tensor([172, 0])
    )
    assert got.tolist() == [128, 20, 129]


def test_shift_positions_accepts_int32_indices() -> None:
    got = ref.shift_positions(torch.tensor([300, 20]), torch.tensor([0, 1], dtype=torch.int32), torch.tensor([172, 0]))
    assert got.tolist() == [128, 20]


def test_physical_lengths_reference_kat() -> None:
    # tests/test_provider_integration.py:486-514: seq_lens [301, 21], offsets [172, 0].
    got = ref.physical_seq_lens(torch.tensor([301, 21]), torch.tensor([172, 0]), 2)
    assert got.tolist() == [129, 21]
    # Only the first num_reqs rows change.
    got = ref.physical_seq_lens(torch.tensor([301, 21, 50], dtype=torch.int32), torch.tensor([172, 0, 7]), 2)
    assert got.tolist() == [129, 21, 50]


def test_slot_mapping_brute_force_hand_worked() -> None:
    # Request 0 was compacted from 300 to 128 tokens (offset 172) into pages
    # [5, 9]; request 1 is uncompressed in pages [2, 3, 4].  Positions 300 and
    # 301 land on physical 128, 129 = page 9 rows 0, 1; position 20 of request
    # 1 is page 2 row 20; the fourth token is graph padding.
    table = [[5, 9, -1], [2, 3, 4]]
    slots, phys = brute.slot_mapping([0, 2, 3], [300, 301, 20, 7], [172, 0], table, 128, 4)
    assert phys == [128, 129, 20, 7]
    assert slots == [9 * 128 + 0, 9 * 128 + 1, 2 * 128 + 20, -1]


def test_slot_mapping_brute_force_edges() -> None:
    # A position below the offset, past the table row and on a -1 entry all map to -1.
    table = [[5, -1]]
    slots, _ = brute.slot_mapping([0, 4], [10, 72, 300, 150], [20], table, 128, 4)
    assert slots == [-1, 5 * 128 + 52, -1, -1]
    # No offsets: the plain host slot mapping.
    slots, phys = brute.slot_mapping([0, 2], [1, 129], None, [[7, 8]], 128, 2)
    assert slots == [7 * 128 + 1, 8 * 128 + 1] and phys == [1, 129]
