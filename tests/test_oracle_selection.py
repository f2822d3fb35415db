"""Pin the oracle's keep-set selection with the reference KATs, the v3 quota
closed form, a brute-force sort and the batched-v3 equivalence."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import triattention_ref as ref


def test_global_policy_kat() -> None:
    # tests/test_selection.py:144-154
    keep = ref.select_keep_indices(
        torch.tensor([10.0, 9.0, 8.0, 7.0, -5.0, -6.0]),
        budget=4, protected_prefix=0, protected_recent=2, segments=8, policy="global",
    )
    assert keep.tolist() == [0, 1, 4, 5]


def test_v3_kat_evicts_evenly() -> None:
    # tests/test_selection.py:60-75
    keep = ref.select_keep_indices(
        torch.arange(16, dtype=torch.float32), budget=12, protected_prefix=2, protected_recent=2, segments=4, policy="v3"
    )
    assert keep[:2].tolist() == [0, 1] and keep[-2:].tolist() == [14, 15]
    assert set(range(16)) - set(keep.tolist()) == {2, 5, 8, 11}


def test_v3_uneven_quota_is_exact() -> None:
    # tests/test_selection.py:78-91
    keep = ref.select_keep_indices(torch.zeros(19), budget=13, protected_prefix=2, protected_recent=2, segments=8, policy="v3")
    assert keep.numel() == 13 and {0, 1, 17, 18} <= set(keep.tolist())


@pytest.mark.parametrize(
    ("tokens", "budget", "prefix", "recent", "segments"),
    [(32768, 8192, 128, 512, 8), (32768, 8192, 256, 512, 8), (32, 17, 0, 0, 4), (32, 18, 2, 2, 4), (32, 31, 0, 0, 4)],
)
def test_batched_v3_equals_per_segment(tokens, budget, prefix, recent, segments) -> None:
    # tests/test_selection.py:94-125 (randperm seed 28: tie-free scores)
    torch.manual_seed(28)
    scores = torch.randperm(tokens, dtype=torch.long).float()
    expected = ref.select_keep_indices(
        scores, budget=budget, protected_prefix=prefix, protected_recent=recent, segments=segments, policy="v3"
    )
    got = ref.select_v3_batched(scores, budget=budget, prefix=prefix, recent=recent, segments=segments)
    assert got is not None and torch.equal(got, expected)


def test_v3_quota_closed_form_sums_to_budget() -> None:
    # The segment quotas telescope: sum = middle - evict = budget - prefix - recent.
    for n, budget, prefix, recent, segments in [(19, 13, 2, 2, 8), (5000, 4608, 128, 512, 8), (36001, 4608, 128, 512, 8)]:
        p, r = min(prefix, n), min(recent, n - min(prefix, n))
        mc, evict = n - p - r, n - budget
        quotas = []
        for s in range(segments):
            a, b = p + mc * s // segments, p + mc * (s + 1) // segments
            quotas.append((b - a) - (evict * (b - p) // mc - evict * (a - p) // mc))
        assert sum(quotas) == budget - p - r and min(quotas) >= 0


@pytest.mark.parametrize("policy", ["global", "v3"])
@pytest.mark.parametrize("seed", range(4))
def test_oracle_matches_brute_force_sort(policy: str, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    n = 300 + 37 * seed
    scores = torch.randn(n, generator=g)
    args = dict(budget=128 + seed, protected_prefix=3 * seed, protected_recent=10, segments=4)
    got = ref.select_keep_indices(scores, policy=policy, **args)
    want = brute.select_stable(scores.numpy(), args["budget"], args["protected_prefix"], args["protected_recent"], 4, policy)
    np.testing.assert_array_equal(got.numpy(), want)


def test_validation_fails_closed() -> None:
    s = torch.zeros(10)
    with pytest.raises(ValueError):
        ref.select_keep_indices(s, budget=11, protected_prefix=0, protected_recent=0, segments=1, policy="global")
    with pytest.raises(ValueError):
        ref.select_keep_indices(s, budget=4, protected_prefix=3, protected_recent=2, segments=1, policy="global")
    with pytest.raises(ValueError):
        ref.select_keep_indices(s, budget=4, protected_prefix=0, protected_recent=0, segments=0, policy="global")
    with pytest.raises(ValueError):
        ref.select_keep_indices(s, budget=4, protected_prefix=0, protected_recent=0, segments=1, policy="other")


def test_stable_rule_orders_nan_and_signed_zero() -> None:
    # Deterministic tie rule used by the HIP selector: NaN above +inf, +0 above -0,
    # equal keys by ascending index.
    scores = np.array([0.0, -0.0, np.nan, np.inf, 1.0, 1.0, -np.inf], dtype=np.float32)
    assert brute.select_stable(scores, 3, 0, 0, 1, "global").tolist() == [2, 3, 4]
    assert brute.select_stable(scores, 4, 0, 0, 1, "global").tolist() == [2, 3, 4, 5]
    assert brute.select_stable(scores, 5, 0, 0, 1, "global").tolist() == [0, 2, 3, 4, 5]
