"""CPU restatement of the calibration -> device layout (oracle).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  Restates
CalibrationStats.to_device and _group_query_stats (tri/stats.py:262-360) and the
bind-time omega default (tri/stats.py:325-331) with explicit index loops, so
that the GPU parity tests build the oracle's per-layer statistics without the
product's own layout code.

Input: per-layer statistics objects with the attributes of
LayerCalibrationStats (tri/stats.py:32-39): q_mean_real, q_mean_imag,
q_abs_mean ([H_q, F] or [H_kv, F]), freq_scale_sq ([1, F], [H_q, F], [H_kv, F]
or None), inv_freq ([F] or None), q_pass_mean ([H_q, P], [H_kv, P] or None);
the artifact metadata mapping; and the model's head counts, head_dim,
rotary_dim and rope_theta.
Output: {layer: triattention_ref.LayerStats} with [kv_local, qpk, width]
float32 tensors for one tensor-parallel shard of the KV heads.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

import torch

from .triattention_ref import LayerStats


def group_rows(rows: torch.Tensor, n_q: int, n_kv: int, width: int) -> torch.Tensor:
    """tri/stats.py:345-360: query-head rows [H_q, w] -> [H_kv, qpk, w] with query
    heads kv*qpk .. kv*qpk+qpk-1 under KV head kv; KV-averaged rows [H_kv, w]
    repeated for every query head of the group."""
    qpk = n_q // n_kv
    shape = tuple(rows.shape)
    if shape not in ((n_q, width), (n_kv, width)):
        raise ValueError(f"calibration tensor shape {shape} cannot be grouped for {n_q} query heads and {n_kv} KV heads")
    source = []
    for kv in range(n_kv):
        for g in range(qpk):
            source.append(kv * qpk + g if shape[0] == n_q else kv)
    return rows[torch.tensor(source, dtype=torch.long)].view(n_kv, qpk, width).clone()


def default_omega(rotary_dim: int, theta: float) -> torch.Tensor:
    """tri/stats.py:329-331: 1 / theta^(i / R) for i = 0, 2, .., R-2, evaluated as
    the reference does (float32 exponents, a float32 power)."""
    exponents = torch.arange(0, rotary_dim, 2, dtype=torch.float32)
    return 1.0 / (theta ** (exponents / float(rotary_dim)))


def _metadata_inv_freq(metadata: Mapping[str, Any], layer: int):
    """tri/stats.py:466-488: per-layer layer_inv_freqs (mapping keyed by int or
    str, or a list), else the shared inv_freq, else None."""
    per_layer = metadata.get("layer_inv_freqs")
    value = None
    if isinstance(per_layer, Mapping):
        value = per_layer.get(layer, per_layer.get(str(layer)))
    elif isinstance(per_layer, (list, tuple)) and layer < len(per_layer):
        value = per_layer[layer]
    if value is None:
        value = metadata.get("inv_freq")
    if isinstance(value, torch.Tensor):
        return value.detach().to("cpu", torch.float32).flatten()
    if isinstance(value, (list, tuple)):
        return torch.tensor(value, dtype=torch.float32).flatten()
    return None


def layer_stats_for_device(
    layers: Mapping[int, Any],
    metadata: Mapping[str, Any],
    *,
    num_attention_heads: int,
    num_kv_heads: int,
    head_dim: int,
    rotary_dim: int,
    rope_theta: float,
    tensor_parallel_rank: int = 0,
    tensor_parallel_size: int = 1,
) -> dict[int, LayerStats]:
    """tri/stats.py:262-342 for one shard of KV heads."""
    if tensor_parallel_size <= 0 or not 0 <= tensor_parallel_rank < tensor_parallel_size:
        raise ValueError("invalid tensor-parallel rank or size")
    if num_kv_heads % tensor_parallel_size:
        raise ValueError("KV heads must divide by the tensor-parallel size")
    freq = rotary_dim // 2
    pass_dim = head_dim - rotary_dim
    local = num_kv_heads // tensor_parallel_size
    first = tensor_parallel_rank * local
    style = str(metadata.get("rope_style", "half"))
    out: dict[int, LayerStats] = {}
    for index, layer in layers.items():

        def shard(rows: torch.Tensor, width: int) -> torch.Tensor:
            full = group_rows(rows.detach().to("cpu", torch.float32), num_attention_heads, num_kv_heads, width)
            return full[first : first + local].clone()

        scale = layer.freq_scale_sq
        if scale is None:
            scale = torch.ones(num_attention_heads, freq)
        elif scale.shape[0] == 1:
            # One row shared by every query head (tri/stats.py:303-304).
            scale = scale.reshape(1, freq).repeat(num_attention_heads, 1)
        inv_freq = layer.inv_freq if layer.inv_freq is not None else _metadata_inv_freq(metadata, index)
        omega = default_omega(rotary_dim, rope_theta) if inv_freq is None else inv_freq.to("cpu", torch.float32)
        out[index] = LayerStats(
            q_mean_real=shard(layer.q_mean_real, freq),
            q_mean_imag=shard(layer.q_mean_imag, freq),
            q_abs_mean=shard(layer.q_abs_mean, freq),
            freq_scale_sq=shard(scale, freq),
            omega=omega.contiguous(),
            rope_style=style,
            rotary_dim=rotary_dim,
            q_pass_mean=None if layer.q_pass_mean is None else shard(layer.q_pass_mean, pass_dim),
        )
    return out
