"""Host-side scoring setup (tri/scoring.py:11-20).

The per-token score itself is computed only by the HIP scorer
(``kernels.score_paged_keys_mean_precomputed`` / ``pipeline``).
"""

from __future__ import annotations

import torch


def build_geometric_offsets(maximum: int, device: torch.device | str) -> torch.Tensor:
    """Future-query offsets 1, 2, 4, ... up to ``maximum`` as float32."""
    if maximum < 1:
        raise ValueError("maximum scoring offset must be positive")
    values = []
    value = 1
    while value <= maximum:
        values.append(float(value))
        value <<= 1
    return torch.tensor(values, dtype=torch.float32, device=device)
