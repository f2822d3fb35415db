"""Pin the oracle's scorer: reference known-answer tests, closed forms and a
float64 brute force (the HIP scorer's parity tests compare against this oracle)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import triattention_ref as ref


def _stats_kat() -> ref.LayerStats:
    # tests/test_scoring.py:13-21 of the reference
    return ref.LayerStats(
        q_mean_real=torch.tensor([[[1.0, 0.5], [0.25, 0.75]]]),
        q_mean_imag=torch.tensor([[[0.0, 0.5], [0.5, 0.25]]]),
        q_abs_mean=torch.ones(1, 2, 2),
        freq_scale_sq=torch.ones(1, 2, 2),
        omega=torch.tensor([1.0, 0.1]),
    )


def _slow_reference(keys, stats, round_start, offsets):
    # Per-offset loop of tests/test_scoring.py:24-50 (phases evaluated per offset).
    kr = keys[..., :2].permute(1, 0, 2).unsqueeze(1)
    ki = keys[..., 2:].permute(1, 0, 2).unsqueeze(1)
    qr, qi = stats.q_mean_real.unsqueeze(2), stats.q_mean_imag.unsqueeze(2)
    pr, pi = qr * kr + qi * ki, qi * kr - qr * ki
    per_offset = []
    for o in offsets:
        phase = (float(round_start) + o) * stats.omega
        per_offset.append((pr * torch.cos(phase) - pi * torch.sin(phase)).sum(dim=-1))
    position = torch.stack(per_offset).mean(dim=0)
    kabs = torch.sqrt(kr.square() + ki.square())
    qabs = torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)
    return position + (kabs * (stats.q_abs_mean - qabs).unsqueeze(2)).sum(dim=-1)


def test_geometric_offsets_closed_form() -> None:
    assert ref.build_geometric_offsets(1).tolist() == [1.0]
    assert ref.build_geometric_offsets(32768).tolist() == [float(2**k) for k in range(16)]
    assert ref.build_geometric_offsets(131072).numel() == 18
    assert ref.build_geometric_offsets(262144).numel() == 19
    with pytest.raises(ValueError):
        ref.build_geometric_offsets(0)


def test_vectorized_mean_matches_per_offset_reference() -> None:
    keys = torch.tensor([[[1.0, 2.0, 3.0, 4.0]], [[0.5, 1.5, 2.5, 3.5]], [[2.0, 1.0, 4.0, 3.0]]])
    offsets = torch.tensor([1.0, 2.0, 4.0])
    got = ref.score_post_rope_keys(keys, _stats_kat(), round_start=3, offsets=offsets)
    torch.testing.assert_close(got, _slow_reference(keys, _stats_kat(), 3, offsets))


def test_one_query_side_scaling_factor_gives_four() -> None:
    # tests/test_scoring.py:85-104: post-RoPE key carries one factor of two.
    stats = ref.LayerStats(
        q_mean_real=torch.ones(1, 1, 1),
        q_mean_imag=torch.zeros(1, 1, 1),
        q_abs_mean=torch.ones(1, 1, 1),
        freq_scale_sq=torch.full((1, 1, 1), 4.0),
        omega=torch.zeros(1),
    )
    got = ref.score_post_rope_keys(torch.tensor([[[2.0, 0.0]]]), stats, round_start=1, offsets=torch.tensor([1.0]))
    torch.testing.assert_close(got, torch.tensor([[[4.0]]]))


def test_partial_rope_content_term() -> None:
    # tests/test_scoring.py:107-133: unrotated dims contribute q_pass . k_pass.
    stats = ref.LayerStats(
        q_mean_real=torch.zeros(1, 1, 1),
        q_mean_imag=torch.zeros(1, 1, 1),
        q_abs_mean=torch.zeros(1, 1, 1),
        freq_scale_sq=torch.ones(1, 1, 1),
        omega=torch.zeros(1),
        rotary_dim=2,
        q_pass_mean=torch.tensor([[[2.0, -1.0]]]),
    )
    keys = torch.tensor([[[0.0, 0.0, 3.0, 4.0]], [[0.0, 0.0, -2.0, 1.0]]])
    got = ref.score_post_rope_keys(keys, stats, round_start=1, offsets=torch.tensor([1.0]))
    torch.testing.assert_close(got, torch.tensor([[[2.0, -5.0]]]))


def test_max_aggregation_shape() -> None:
    got = ref.score_post_rope_keys(
        torch.randn(7, 1, 4), _stats_kat(), round_start=7, offsets=torch.tensor([1.0, 2.0]), aggregation="max"
    )
    assert got.shape == (1, 2, 7)


def test_omega_zero_closed_form() -> None:
    # With omega = 0 every phase is 0: score = sum_f a (qr kr + qi ki) + a*extra*|k|.
    g = torch.Generator().manual_seed(4)
    kv, qpk, freq = 2, 3, 4
    qr, qi = torch.randn(kv, qpk, freq, generator=g), torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + 0.5
    fs = torch.rand(kv, qpk, freq, generator=g) + 0.5
    stats = ref.LayerStats(qr, qi, qa, fs, torch.zeros(freq))
    keys = torch.randn(5, kv, 2 * freq, generator=g)
    got = ref.score_post_rope_keys(keys, stats, round_start=1000, offsets=torch.tensor([1.0, 2.0, 4.0]))
    kr, ki = keys[..., :freq].permute(1, 0, 2), keys[..., freq:].permute(1, 0, 2)
    a = torch.sqrt(fs)
    expected = torch.empty(kv, qpk, 5)
    for h in range(kv):
        for q in range(qpk):
            lin = (a[h, q] * (qr[h, q] * kr[h] + qi[h, q] * ki[h])).sum(-1)
            extra = (a[h, q] * (qa[h, q] - torch.sqrt(qr[h, q] ** 2 + qi[h, q] ** 2 + 1e-8)) * torch.sqrt(kr[h] ** 2 + ki[h] ** 2)).sum(-1)
            expected[h, q] = lin + extra
    torch.testing.assert_close(got, expected, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(
    ("head_dim", "rotary", "style", "round_start"),
    [(16, 16, "half", 300), (16, 16, "interleaved", 4096), (32, 16, "half", 65536), (16, 16, "half", 131072)],
)
def test_oracle_matches_float64_brute_force(head_dim: int, rotary: int, style: str, round_start: int) -> None:
    g = torch.Generator().manual_seed(head_dim + rotary + round_start)
    kv, qpk, tokens = 2, 3, 6
    freq = rotary // 2
    qr, qi = torch.randn(kv, qpk, freq, generator=g), torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + torch.rand(kv, qpk, freq, generator=g)
    fs = torch.rand(kv, qpk, freq, generator=g) + 0.5
    omega = 1.0 / (1e6 ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
    qp = torch.randn(kv, qpk, head_dim - rotary, generator=g) if head_dim > rotary else None
    keys = torch.randn(tokens, kv, head_dim, generator=g).to(torch.bfloat16)
    stats = ref.LayerStats(qr, qi, qa, fs, omega, style, rotary, qp)
    offsets = ref.build_geometric_offsets(32768)
    got = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets).double().numpy()
    # Brute force sees the same float32 phase arguments the torch path forms.
    phase_offsets = [float(o) for o in offsets]
    expected = brute.score_brute(
        keys.float().numpy(), qr.numpy(), qi.numpy(), qa.numpy(), fs.numpy(), omega.numpy(), phase_offsets, round_start,
        rotary_dim=rotary, q_pass=None if qp is None else qp.numpy(), interleaved=style == "interleaved",
    )
    # float32 evaluation of (o + rs) * omega differs from float64 by <= 1 ulp of the
    # argument, i.e. up to ~1e-2 rad at rs = 1.3e5 for the fastest frequency.  The
    # tolerance therefore scales with the argument magnitude.
    scale = np.abs(expected).max() + 1.0
    tol = 1e-5 if round_start < 10000 else 4e-2
    assert np.max(np.abs(got - expected)) <= tol * scale


@pytest.mark.parametrize(
    ("head_dim", "rotary", "style", "n_offsets"),
    [(16, 16, "half", 16), (16, 16, "interleaved", 18), (32, 16, "half", 5), (48, 32, "interleaved", 19)],
)
def test_oracle_max_matches_float64_brute_force(head_dim: int, rotary: int, style: str, n_offsets: int) -> None:
    # tri/scoring.py:84-97: the rotary sum is maximised over the offsets, then
    # the magnitude and pass terms are added.
    g = torch.Generator().manual_seed(7 * head_dim + n_offsets)
    kv, qpk, tokens, rs = 2, 3, 6, 300
    freq = rotary // 2
    qr, qi = torch.randn(kv, qpk, freq, generator=g), torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + torch.rand(kv, qpk, freq, generator=g)
    fs = torch.rand(kv, qpk, freq, generator=g) + 0.5
    omega = 1.0 / (1e4 ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
    qp = torch.randn(kv, qpk, head_dim - rotary, generator=g) if head_dim > rotary else None
    keys = torch.randn(tokens, kv, head_dim, generator=g).to(torch.bfloat16)
    stats = ref.LayerStats(qr, qi, qa, fs, omega, style, rotary, qp)
    offsets = ref.build_geometric_offsets(2 ** (n_offsets - 1))
    assert offsets.numel() == n_offsets
    got = ref.score_post_rope_keys(keys, stats, round_start=rs, offsets=offsets, aggregation="max").double().numpy()
    args = (keys.float().numpy(), qr.numpy(), qi.numpy(), qa.numpy(), fs.numpy(), omega.numpy(), [float(o) for o in offsets], rs)
    kw = dict(rotary_dim=rotary, q_pass=None if qp is None else qp.numpy(), interleaved=style == "interleaved")
    expected = brute.score_brute(*args, aggregation="max", **kw)
    scale = np.abs(expected).max() + 1.0
    assert np.max(np.abs(got - expected)) <= 2e-3 * scale
    # The maximum over offsets is at least their mean, and strictly above it
    # somewhere for random phases.
    mean = brute.score_brute(*args, aggregation="mean", **kw)
    assert np.all(expected >= mean - 1e-9) and np.any(expected > mean + 1e-3)


def test_max_aggregation_reduces_to_mean() -> None:
    # One offset, or omega = 0 (every offset has phase 0): max over offsets = mean.
    g = torch.Generator().manual_seed(12)
    kv, qpk, freq = 1, 2, 8
    qr, qi = torch.randn(kv, qpk, freq, generator=g), torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + 0.25
    fs = torch.rand(kv, qpk, freq, generator=g) + 0.5
    keys = torch.randn(9, kv, 2 * freq, generator=g)
    omega = 1.0 / (1e6 ** (torch.arange(0, 2 * freq, 2, dtype=torch.float32) / (2 * freq)))
    one = torch.tensor([64.0])
    stats = ref.LayerStats(qr, qi, qa, fs, omega)
    torch.testing.assert_close(
        ref.score_post_rope_keys(keys, stats, round_start=999, offsets=one, aggregation="max"),
        ref.score_post_rope_keys(keys, stats, round_start=999, offsets=one, aggregation="mean"),
        rtol=1e-6, atol=1e-6,
    )
    flat = ref.LayerStats(qr, qi, qa, fs, torch.zeros(freq))
    offs = ref.build_geometric_offsets(1 << 17)
    torch.testing.assert_close(
        ref.score_post_rope_keys(keys, flat, round_start=5, offsets=offs, aggregation="max"),
        ref.score_post_rope_keys(keys, flat, round_start=5, offsets=offs, aggregation="mean"),
        rtol=1e-5, atol=1e-5,
    )


def test_oracle_phase_arguments_match_float32_brute_force() -> None:
    # Evaluating the brute force at the float32-rounded phase argument removes
    # the argument rounding: then agreement is to float32 arithmetic precision.
    g = torch.Generator().manual_seed(11)
    kv, qpk, freq, tokens, rs = 1, 2, 8, 5, 131072
    qr, qi = torch.randn(kv, qpk, freq, generator=g), torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + 0.3
    fs = torch.ones(kv, qpk, freq)
    omega = 1.0 / (1e6 ** (torch.arange(0, 2 * freq, 2, dtype=torch.float32) / (2 * freq)))
    keys = torch.randn(tokens, kv, 2 * freq, generator=g)
    offsets = ref.build_geometric_offsets(131072)
    got = ref.score_post_rope_keys(keys, ref.LayerStats(qr, qi, qa, fs, omega), round_start=rs, offsets=offsets)
    phases32 = ((offsets.unsqueeze(1) + float(rs)) * omega.unsqueeze(0)).double()
    c = torch.cos(phases32).mean(0)
    s = torch.sin(phases32).mean(0)
    kr, ki = keys[..., :freq].double().permute(1, 0, 2).unsqueeze(1), keys[..., freq:].double().permute(1, 0, 2).unsqueeze(1)
    qrd, qid = qr.double().unsqueeze(2), qi.double().unsqueeze(2)
    lin = ((qrd * kr + qid * ki) * c - (qid * kr - qrd * ki) * s).sum(-1)
    extra = ((qa.double() - torch.sqrt(qr.double() ** 2 + qi.double() ** 2 + 1e-8)).unsqueeze(2) * torch.sqrt(kr**2 + ki**2)).sum(-1)
    torch.testing.assert_close(got.double(), lin + extra, rtol=2e-5, atol=2e-5)


def test_normalisation_closed_form() -> None:
    # tests/test_selection.py:271-280: (s - mean) * rsqrt(var + 1e-6) with population var;
    # the torch path divides by sqrt(max(var, 1e-6)).
    raw = torch.tensor([[[1.0, 2.0, 3.0, 6.0]], [[0.0, 0.0, 0.0, 4.0]]])
    var, mean = torch.var_mean(raw, dim=-1, correction=0)
    z = ref.normalize_head_scores(raw, mean, var)
    np.testing.assert_allclose(z.amax(dim=(0, 1)).double().numpy(), brute.normalized_layer_max(raw.numpy()), rtol=1e-6)
    const = torch.full((1, 1, 4), 3.0)
    v, m = torch.var_mean(const, dim=-1, correction=0)
    assert torch.equal(ref.normalize_head_scores(const, m, v), torch.zeros(1, 1, 4))
    assert math.isclose(float(ref.normalize_head_scores(torch.tensor([[[0.0, 2.0]]]), torch.tensor([[1.0]]), torch.tensor([[1.0]]))[0, 0, 1]), 1.0)
