"""Shared helpers for the parity tests: oracle adapters and tolerances."""

from __future__ import annotations

import torch

from oracle import stats_ref
from oracle import triattention_ref as ref


def oracle_layer_stats(calibration, model, layers) -> list[ref.LayerStats]:
    """The oracle's statistics of ``layers`` from a loaded calibration, laid out
    by the oracle's restatement of the device layout (oracle.stats_ref), not by
    the product's CalibrationStats.to_device."""
    laid_out = stats_ref.layer_stats_for_device(
        calibration.layers,
        calibration.metadata,
        num_attention_heads=model.num_attention_heads,
        num_kv_heads=model.num_kv_heads,
        head_dim=model.head_dim,
        rotary_dim=model.effective_rotary_dim,
        rope_theta=model.rope_theta,
    )
    return [laid_out[layer] for layer in layers]


def oracle_stats(device_stats) -> ref.LayerStats:
    s = device_stats
    return ref.LayerStats(
        q_mean_real=s.q_mean_real.cpu(),
        q_mean_imag=s.q_mean_imag.cpu(),
        q_abs_mean=s.q_abs_mean.cpu(),
        freq_scale_sq=s.freq_scale_sq.cpu(),
        omega=s.omega.cpu(),
        rope_style=s.rope_style,
        rotary_dim=s.rotary_dim,
        q_pass_mean=None if s.q_pass_mean is None else s.q_pass_mean.cpu(),
    )


def assert_scores_close(got: torch.Tensor, want: torch.Tensor, rel: float = 1e-3) -> float:
    """|got - want| <= rel * (|want| + rms_h(want)), rms over each query head's tokens.

    ``got``/``want`` are [heads, tokens]."""
    got = got.double().cpu()
    want = want.double().cpu()
    rms = want.square().mean(dim=-1, keepdim=True).sqrt()
    bound = rel * (want.abs() + rms)
    err = (got - want).abs()
    worst = float((err / bound).max())
    assert worst <= 1.0, f"scores differ: worst err/bound {worst:.3f}, max abs err {float(err.max()):.3e}"
    return float(err.max())


def assert_agg_close(got: torch.Tensor, want: torch.Tensor, rel: float = 1e-3) -> float:
    """|got - want| <= rel * max(1, |want|), with identical non-finite entries."""
    got = got.double().cpu()
    want = want.double().cpu()
    finite = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), finite)
    assert torch.equal(got[~finite], want[~finite])
    err = (got[finite] - want[finite]).abs()
    bound = rel * want[finite].abs().clamp_min(1.0)
    worst = float((err / bound).max()) if err.numel() else 0.0
    assert worst <= 1.0, f"aggregate differs: worst err/bound {worst:.3f}"
    return float(err.max()) if err.numel() else 0.0


def assert_keep_matches(got: torch.Tensor, want: torch.Tensor, agg: torch.Tensor, budget: int, protected: torch.Tensor | None = None, rel: float = 1e-3) -> int:
    """Keep sets equal except near-ties: every differing index scores within
    rel*max(1,|t|) of the selection threshold t (the lowest kept unprotected
    oracle score).  Returns the number of differing indices."""
    got_set = set(got.cpu().tolist())
    want_set = set(want.cpu().tolist())
    assert len(got_set) == len(got) == budget, "keep indices must be unique and exactly budget"
    assert got.cpu().tolist() == sorted(got_set), "keep indices must be ascending"
    diff = got_set ^ want_set
    if not diff:
        return 0
    agg = agg.double().cpu()
    candidates = [i for i in want_set if protected is None or not bool(protected[i])]
    threshold = min(float(agg[i]) for i in candidates)
    for i in diff:
        assert abs(float(agg[i]) - threshold) <= rel * max(1.0, abs(threshold)), (
            f"index {i} differs from the oracle keep set and is not a near-tie "
            f"(score {float(agg[i])}, threshold {threshold})"
        )
    return len(diff)
