"""Scoring entry points under the reference's names (tri/scoring.py).

``score_post_rope_keys`` scores dense post-RoPE keys on the HIP scorers (the
mean and the max aggregation), for callers of the reference's torch path; the
compression step itself scores paged keys in ``pipeline``.
"""

from __future__ import annotations

import torch

from . import _device as dev
from . import kernels


def build_geometric_offsets(maximum: int, device: torch.device | str) -> torch.Tensor:
    """Future-query offsets 1, 2, 4, ... up to ``maximum`` as float32 (tri/scoring.py:11-20)."""
    if maximum < 1:
        raise ValueError("maximum scoring offset must be positive")
    values = []
    value = 1
    while value <= maximum:
        values.append(float(value))
        value <<= 1
    return torch.tensor(values, dtype=torch.float32, device=device)


def score_post_rope_keys(
    keys: torch.Tensor, stats, *, round_start: int, offsets: torch.Tensor, aggregation: str = "mean"
) -> torch.Tensor:
    """Scores ``[kv_heads, queries_per_kv, tokens]`` of post-RoPE keys
    ``[tokens, kv_heads, head_dim]`` (bf16 or fp16 on a HIP device) against
    one layer's grouped calibration ``stats`` (tri/scoring.py:23-120).  The
    keys are laid into 128-token pages and scored by kvc_score_paged
    (``aggregation="mean"``) or kvc_score_paged_max (``"max"``)."""
    if aggregation not in ("mean", "max"):
        raise ValueError(f"unsupported score aggregation: {aggregation}")
    if keys.ndim != 3:
        raise ValueError("keys must have shape [tokens, kv_heads, head_dim]")
    dev.require_hip(keys, "keys")
    if keys.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("the HIP scorers read bf16 or fp16 keys")
    tokens, kv_heads, head_dim = (int(x) for x in keys.shape)
    qr, qi = stats.q_mean_real, stats.q_mean_imag
    if qr.ndim != 3 or qr.shape[0] != kv_heads:
        raise ValueError("calibration does not match cache keys")
    pages = max(1, -(-tokens // 128))
    paged = torch.zeros((pages, 128, kv_heads, head_dim), dtype=keys.dtype, device=keys.device)
    paged.view(-1, kv_heads, head_dim)[:tokens].copy_(keys)
    blocks = torch.arange(pages, dtype=torch.int64, device=keys.device)
    scale = torch.sqrt(stats.freq_scale_sq.float())
    extra = stats.q_abs_mean.float() - torch.sqrt(qr.float().square() + qi.float().square() + 1e-8)
    rotary = getattr(stats, "rotary_dim", None)
    q_pass = getattr(stats, "q_pass_mean", None)
    style = getattr(stats, "rope_style", "half")
    out = torch.empty((kv_heads, qr.shape[1], tokens), dtype=torch.float32, device=keys.device)
    if tokens == 0:
        return out
    omega = stats.omega.float().contiguous()
    offs = offsets.to(device=keys.device, dtype=torch.float32).contiguous()
    if aggregation == "max":
        kernels.score_paged_keys_max(
            paged, blocks, qr, qi, scale, extra, omega, offs, round_start, tokens, out, 128, style,
            q_pass_mean=q_pass, rotary_dim=rotary,
        )
        return out
    rs = torch.tensor([int(round_start)], dtype=torch.int64, device=keys.device)
    cos, sin = kernels.mean_phase_table(rs, offs, omega.view(1, -1))
    kernels.score_paged_keys_mean_precomputed(
        paged, blocks, qr, qi, scale, extra, cos.view(-1), sin.view(-1), tokens, out, 128, style,
        q_pass_mean=q_pass, rotary_dim=rotary,
    )
    return out


def normalize_head_scores(scores: torch.Tensor, mean: torch.Tensor, variance: torch.Tensor) -> torch.Tensor:
    """(scores - mean) / sqrt(max(variance, 1e-6)) per head (tri/scoring.py:123-128); the
    compression step applies it inside kvc_aggregate."""
    return (scores - mean.unsqueeze(-1)) / torch.sqrt(variance.clamp_min(1e-6)).unsqueeze(-1)
