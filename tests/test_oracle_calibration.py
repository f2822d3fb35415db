"""Pins of the calibration-statistics oracle (oracle/calibration_ref.py) on the CPU.

The restatement of _LayerAccumulator.add (pkg/calibration.py:98-131) is checked
against closed forms that a swapped real/imaginary half, an interleaved pair
layout, a wrong divisor or a gate that leaks into the statistics would break,
and against the float64 loop brute force.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import calibration_ref as cref


def test_constant_pairs_closed_form() -> None:
    # Every pair (re, im) = (3, 4): means 3 and 4, magnitude 5; pass dims 7.
    heads, head_dim, rotary = 2, 10, 8
    q = torch.empty(5, heads, head_dim)
    q[..., :4] = 3.0
    q[..., 4:8] = 4.0
    q[..., 8:] = 7.0
    acc = cref.QueryStatsAccumulator()
    acc.add(q.reshape(5, -1), heads, head_dim, rotary)
    m = acc.means()
    assert acc.count == 5
    assert torch.equal(m["q_mean_real"], torch.full((2, 4), 3.0))
    assert torch.equal(m["q_mean_imag"], torch.full((2, 4), 4.0))
    assert torch.equal(m["q_abs_mean"], torch.full((2, 4), 5.0))
    assert torch.equal(m["q_pass_mean"], torch.full((2, 2), 7.0))


def test_half_layout_not_interleaved() -> None:
    # Dim d of a head holds d: half style pairs (f, F+f), so real means are
    # 0..F-1 and imaginary F..2F-1 (an interleaved reading would give evens/odds).
    heads, head_dim = 1, 8
    q = torch.arange(head_dim, dtype=torch.float32).repeat(3, 1)
    acc = cref.QueryStatsAccumulator()
    acc.add(q, heads, head_dim, head_dim)
    m = acc.means()
    assert m["q_mean_real"].tolist() == [[0.0, 1.0, 2.0, 3.0]]
    assert m["q_mean_imag"].tolist() == [[4.0, 5.0, 6.0, 7.0]]
    want_abs = [float(np.hypot(f, f + 4)) for f in range(4)]
    assert m["q_abs_mean"][0].tolist() == pytest.approx(want_abs, rel=1e-6)
    assert "q_pass_mean" not in m


def test_gate_half_is_ignored_and_head_shaped_input_equals_flat() -> None:
    g = torch.Generator().manual_seed(3)
    heads, head_dim = 3, 8
    q = torch.randn(2, 6, heads * head_dim, generator=g)
    gated = torch.cat([q, torch.full_like(q, float("nan"))], dim=-1)
    a, b, c = cref.QueryStatsAccumulator(), cref.QueryStatsAccumulator(), cref.QueryStatsAccumulator()
    a.add(q, heads, head_dim, head_dim)
    b.add(gated, heads, head_dim, head_dim)
    c.add(q.reshape(2, 6, heads, head_dim), heads, head_dim, head_dim)
    for key in ("q_mean_real", "q_mean_imag", "q_abs_mean"):
        assert torch.equal(a.means()[key], b.means()[key])
        assert torch.equal(a.means()[key], c.means()[key])
    assert a.count == b.count == c.count == 12


def test_restatement_matches_brute_force_and_accumulates() -> None:
    rng = np.random.default_rng(11)
    heads, head_dim, rotary = 4, 24, 16
    chunks = [rng.standard_normal((n, heads, head_dim)).astype(np.float32) for n in (7, 1, 13)]
    acc = cref.QueryStatsAccumulator()
    for chunk in chunks:
        acc.add(torch.from_numpy(chunk).reshape(chunk.shape[0], -1), heads, head_dim, rotary)
    whole = np.concatenate(chunks)
    brute = cref.query_sums_brute(whole, rotary)
    m = acc.means()
    n = whole.shape[0]
    assert acc.count == n
    np.testing.assert_allclose(m["q_mean_real"].numpy(), brute["real"] / n, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m["q_mean_imag"].numpy(), brute["imag"] / n, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m["q_abs_mean"].numpy(), brute["abs"] / n, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m["q_pass_mean"].numpy(), brute["pass"] / n, rtol=1e-5, atol=1e-6)


def test_rejects_mismatched_width() -> None:
    acc = cref.QueryStatsAccumulator()
    with pytest.raises(RuntimeError):
        acc.add(torch.zeros(3, 10), 2, 4, 4)
