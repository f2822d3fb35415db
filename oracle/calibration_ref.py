"""CPU restatement of the calibration generator's query statistics -- TEST INFRASTRUCTURE ONLY.

Follows the reference's torch path: _LayerAccumulator.add
(pkg/calibration.py:98-131) -- drop an output gate packed after Q, read the
projection as [tokens, heads, head_dim] in float32, sum real / imaginary /
magnitude over tokens per (head, frequency) and the pass dims per (head, dim),
keep float32 running sums across calls -- and the per-layer means of the
finalisation (pkg/calibration.py:351-371).

``query_sums_brute`` is written from the definitions instead (plain loops in
float64 over tokens, heads and dims) and pins the restatement on small inputs;
the GPU kernel is compared with both.
"""

from __future__ import annotations

import math

import numpy as np
import torch


class QueryStatsAccumulator:
    """_LayerAccumulator.add (pkg/calibration.py:98-131), float32 sums on the CPU."""

    def __init__(self) -> None:
        self.real_sum: torch.Tensor | None = None
        self.imag_sum: torch.Tensor | None = None
        self.abs_sum: torch.Tensor | None = None
        self.pass_sum: torch.Tensor | None = None
        self.count = 0

    def add(self, projected: torch.Tensor, heads: int, head_dim: int, rotary_dim: int) -> None:
        expected = heads * head_dim
        if projected.shape[-1] == expected * 2:
            projected = projected[..., :expected]
        if projected.shape[-1] == expected or (projected.shape[-1] == head_dim and projected.numel() % expected == 0):
            values = projected.detach().reshape(-1, heads, head_dim).float()
        else:
            raise RuntimeError(f"query projection width {projected.shape[-1]} does not match {expected}")
        freq = rotary_dim // 2
        real = values[..., :freq]
        imag = values[..., freq:rotary_dim]
        pass_values = values[..., rotary_dim:]
        real_sum = real.sum(dim=0)
        imag_sum = imag.sum(dim=0)
        abs_sum = torch.sqrt(real.square() + imag.square()).sum(dim=0)
        self.real_sum = real_sum if self.real_sum is None else self.real_sum + real_sum
        self.imag_sum = imag_sum if self.imag_sum is None else self.imag_sum + imag_sum
        self.abs_sum = abs_sum if self.abs_sum is None else self.abs_sum + abs_sum
        if pass_values.numel():
            pass_sum = pass_values.sum(dim=0)
            self.pass_sum = pass_sum if self.pass_sum is None else self.pass_sum + pass_sum
        self.count += values.shape[0]

    def means(self) -> dict[str, torch.Tensor]:
        """Per-layer means of pkg/calibration.py:351-371."""
        divisor = float(self.count)
        out = {
            "q_mean_real": self.real_sum / divisor,
            "q_mean_imag": self.imag_sum / divisor,
            "q_abs_mean": self.abs_sum / divisor,
        }
        if self.pass_sum is not None:
            out["q_pass_mean"] = self.pass_sum / divisor
        return out


def query_sums_brute(values: np.ndarray, rotary_dim: int) -> dict[str, np.ndarray]:
    """values [tokens, heads, head_dim] -> float64 sums by explicit loops:
    real[h][f] = sum_t v[t,h,f], imag[h][f] = sum_t v[t,h,F+f],
    abs[h][f] = sum_t |v[t,h,f] + i v[t,h,F+f]|, pass[h][p] = sum_t v[t,h,R+p]."""
    values = np.asarray(values, dtype=np.float64)
    tokens, heads, head_dim = values.shape
    freq = rotary_dim // 2
    width = head_dim - rotary_dim
    real = np.zeros((heads, freq))
    imag = np.zeros((heads, freq))
    mag = np.zeros((heads, freq))
    passed = np.zeros((heads, width))
    for t in range(tokens):
        for h in range(heads):
            for f in range(freq):
                re, im = values[t, h, f], values[t, h, freq + f]
                real[h, f] += re
                imag[h, f] += im
                mag[h, f] += math.hypot(re, im)
            for p in range(width):
                passed[h, p] += values[t, h, rotary_dim + p]
    return {"real": real, "imag": imag, "abs": mag, "pass": passed}
