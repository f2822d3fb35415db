"""Pin the oracle's cross-layer aggregation (oracle.triattention_ref.aggregate_layers).

The function restates tri/method.py:423-467,477-503: per scoring layer the
normalised scores' maximum over every query head, layers combined in layer
order (copy of layer 0, then += or maximum), division by the number of scoring
layers in mean mode, then nan_to_num(nan=-inf, posinf=1e30, neginf=-inf).

Every expected value here comes from outside that code path:
  - normalised scores of polynomial raw scores from exact power sums
    (fractions.Fraction), not from torch.var_mean;
  - the reference's own two-layer closed form (tests/test_selection.py:199-280,
    expected value at :271-280) without its collective;
  - raw scores passed through with mean 0 / variance 1 (or variance 0, which the
    normalisation clamps to 1e-6), so the per-layer values are chosen directly
    and the layer combination and the NaN / inf mapping follow from IEEE
    arithmetic and the mapping the reference states (tri/method.py:463-467).
Plausible mistakes each fail a case below: dividing by the model's layer count
or by S - 1, dropping or double-counting layer 0, sanitising before the mean, a
NaN-ignoring maximum, a wrong infinity mapping, a sample (not population)
variance, a maximum over one KV head only.
"""

from __future__ import annotations

import math
from fractions import Fraction

import pytest
import torch

from oracle import triattention_ref as ref


def _power_sums(n: int, degree: int) -> list[Fraction]:
    return [Fraction(sum(t**k for t in range(n))) for k in range(degree + 1)]


def _normalised_polynomial(coeffs: list[Fraction], n: int) -> list[float]:
    """z(t) = (p(t) - mean) / sqrt(population variance) over t = 0 .. n-1 for the
    polynomial p with the given coefficients (lowest degree first), with the
    mean and variance from exact power sums."""
    deg = len(coeffs) - 1
    sums = _power_sums(n, 2 * deg)
    mean = sum(c * sums[k] for k, c in enumerate(coeffs)) / n
    second = sum(ci * cj * sums[i + j] for i, ci in enumerate(coeffs) for j, cj in enumerate(coeffs)) / n
    var = second - mean * mean
    sd = math.sqrt(var)
    out = []
    for t in range(n):
        p = sum(c * Fraction(t) ** k for k, c in enumerate(coeffs))
        out.append(float(p - mean) / sd)
    return out


def _layer(values) -> torch.Tensor:
    """One query head's raw scores as [kv=1, qpk=1, N] float32."""
    return torch.tensor(values, dtype=torch.float32).view(1, 1, -1)


def _aggregate(raws: list[torch.Tensor], mode: str = "mean", stats=None) -> torch.Tensor:
    if stats is None:
        stats = [torch.var_mean(r, dim=-1, correction=0) for r in raws]
    cfg = ref.MethodConfig(budget=128, layer_aggregation=mode)
    return ref.aggregate_layers(raws, stats, cfg)


def _passthrough(raws: list[torch.Tensor], var: float = 1.0):
    """(var, mean) that make the normalised scores equal the raw ones
    (var 1) or raw / 1e-3 (var 0, clamped to 1e-6)."""
    return [(torch.full(r.shape[:2], var), torch.zeros(r.shape[:2])) for r in raws]


N = 256
T = [Fraction(t) for t in range(N)]


def test_reference_two_layer_closed_form_mean():
    # tests/test_selection.py:230-280: raw layers t and t^2/256 over 256 tokens,
    # each normalised with its population statistics, mean over the two layers.
    lin = _normalised_polynomial([Fraction(0), Fraction(1)], N)
    quad = _normalised_polynomial([Fraction(0), Fraction(0), Fraction(1, 256)], N)
    want = torch.tensor([(a + b) / 2 for a, b in zip(lin, quad)], dtype=torch.float64)
    raws = [_layer(range(N)), _layer([t * t / 256 for t in range(N)])]
    got = _aggregate(raws, "mean")
    torch.testing.assert_close(got.double(), want, rtol=2e-6, atol=2e-6)
    # The linear layer alone has the textbook closed form (t - (N-1)/2) / sqrt((N^2-1)/12).
    sd = math.sqrt((N * N - 1) / 12)
    assert lin[0] == pytest.approx(-(N - 1) / 2 / sd, rel=1e-12)


def test_reference_two_layer_closed_form_max():
    lin = _normalised_polynomial([Fraction(0), Fraction(1)], N)
    quad = _normalised_polynomial([Fraction(0), Fraction(0), Fraction(1, 256)], N)
    want = torch.tensor([max(a, b) for a, b in zip(lin, quad)], dtype=torch.float64)
    raws = [_layer(range(N)), _layer([t * t / 256 for t in range(N)])]
    got = _aggregate(raws, "max")
    torch.testing.assert_close(got.double(), want, rtol=2e-6, atol=2e-6)


def test_mean_divides_by_scoring_layer_count():
    # Six scoring layers (48 model layers at stride 8): layer l holds
    # sign_l * (l + 1) * t, whose normalised scores are sign_l * u(t) for the
    # linear u; the mean is (sum of signs / 6) * u = u / 3.  Dividing by 48, by
    # 5 or by 7 gives u / 24, 2u / 5 or 2u / 7.
    signs = [1, 1, -1, 1, -1, 1]
    raws = [_layer([s * (l + 1) * t for t in range(N)]) for l, s in enumerate(signs)]
    u = _normalised_polynomial([Fraction(0), Fraction(1)], N)
    want = torch.tensor([x / 3 for x in u], dtype=torch.float64)
    got = _aggregate(raws, "mean")
    torch.testing.assert_close(got.double(), want, rtol=2e-6, atol=2e-6)
    got_max = _aggregate(raws, "max")
    torch.testing.assert_close(got_max.double(), torch.tensor([abs(x) for x in u], dtype=torch.float64), rtol=2e-6, atol=2e-6)


def test_layer_zero_counted_once():
    # Per-layer values chosen directly (mean 0, variance 1): mean of 1, 3, 8 is 4;
    # skipping layer 0 gives 11/3, counting it twice 13/3 (or 13/4).
    raws = [_layer([1.0, -2.0]), _layer([3.0, -4.0]), _layer([8.0, 0.5])]
    got = _aggregate(raws, "mean", _passthrough(raws))
    assert got[0].item() == 4.0
    assert got[1].item() == pytest.approx(-5.5 / 3.0, rel=1e-7)
    got_max = _aggregate(raws, "max", _passthrough(raws))
    assert got_max.tolist() == [8.0, 0.5]


def test_head_maximum_spans_every_kv_head_and_query_head():
    # Two KV heads x two query heads.  Heads t, -t, 2t + 5, -3t normalise to
    # u, -u, u, -u: the maximum over all four is |u|.  Heads t, 2t, -t, -3t put
    # +u only in the first KV head and -u only in the second: the maximum over
    # both is |u|, over the second KV head alone -u.
    u = _normalised_polynomial([Fraction(0), Fraction(1)], N)
    t = torch.arange(N, dtype=torch.float32)
    raw = torch.stack([torch.stack([t, -t]), torch.stack([2 * t + 5, -3 * t])])
    got = _aggregate([raw], "mean")
    torch.testing.assert_close(got.double(), torch.tensor([abs(x) for x in u], dtype=torch.float64), rtol=2e-6, atol=2e-6)
    raw2 = torch.stack([torch.stack([t, 2 * t]), torch.stack([-t, -3 * t])])
    got2 = _aggregate([raw2], "mean")
    torch.testing.assert_close(got2.double(), torch.tensor([abs(x) for x in u], dtype=torch.float64), rtol=2e-6, atol=2e-6)
    only_second = torch.tensor([-x for x in u], dtype=torch.float64)
    assert not torch.allclose(got2.double(), only_second)


def test_population_not_sample_variance():
    # Four tokens 0, 1, 2, 3: population variance 5/4, sample variance 5/3.
    raws = [_layer([0.0, 1.0, 2.0, 3.0])]
    got = _aggregate(raws, "mean")
    want = [(t - 1.5) / math.sqrt(1.25) for t in range(4)]
    torch.testing.assert_close(got.double(), torch.tensor(want, dtype=torch.float64), rtol=1e-6, atol=1e-6)


def test_variance_clamp_and_infinity_mapping():
    # One layer, mean 0, variance 0 (clamped to 1e-6, so z = raw / 1e-3):
    # 1e36 -> 1e39 overflows float32 to +inf -> 1e30; NaN -> -inf; -inf kept;
    # finite values scaled by 1000.
    raws = [_layer([1e36, float("nan"), float("-inf"), 2.0, 3e-3])]
    got = _aggregate(raws, "mean", _passthrough(raws, var=0.0))
    assert got[0].item() == pytest.approx(1e30, rel=1e-6)
    assert got[1].item() == float("-inf")
    assert got[2].item() == float("-inf")
    assert got[3].item() == pytest.approx(2000.0, rel=1e-6)
    assert got[4].item() == pytest.approx(3.0, rel=1e-6)


def test_sanitise_after_the_layer_combination():
    # Layer values chosen directly.  Mean mode: (+inf + 2)/2 = +inf -> 1e30
    # (sanitising first gives (1e30 + 2)/2 = 5e29); (4 + NaN)/2 = NaN -> -inf;
    # (+inf + -inf)/2 = NaN -> -inf (sanitising first: (1e30 - inf)/2 = -inf too,
    # but (1e30 + 3)/2 in the first column already tells them apart).
    raws = [_layer([float("inf"), 4.0, float("inf"), -1.0]), _layer([2.0, float("nan"), float("-inf"), 3.0])]
    got = _aggregate(raws, "mean", _passthrough(raws))
    assert got[0].item() == pytest.approx(1e30, rel=1e-6)
    assert got[1].item() == float("-inf")
    assert got[2].item() == float("-inf")
    assert got[3].item() == 1.0
    # Max mode: NaN propagates through the maximum (torch.maximum), so
    # max(4, NaN) = NaN -> -inf; a NaN-ignoring maximum would give 4.
    got_max = _aggregate(raws, "max", _passthrough(raws))
    assert got_max[0].item() == pytest.approx(1e30, rel=1e-6)
    assert got_max[1].item() == float("-inf")
    assert got_max[2].item() == pytest.approx(1e30, rel=1e-6)
    assert got_max[3].item() == 3.0


def test_nan_in_a_later_layer_of_max_mode():
    # NaN in layer 1 (not layer 0) still wins the maximum: max(2, NaN) -> NaN -> -inf.
    raws = [_layer([2.0, 5.0]), _layer([float("nan"), 1.0])]
    got = _aggregate(raws, "max", _passthrough(raws))
    assert got.tolist() == [float("-inf"), 5.0]
