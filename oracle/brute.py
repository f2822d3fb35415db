"""Float64 brute force used to pin the oracle -- TEST INFRASTRUCTURE ONLY.

Written from the mathematics of the TriAttention score (tri/scoring.py:23-120),
not from the restatement's tensor program: explicit loops over tokens, heads,
frequencies and future offsets in float64.
"""

from __future__ import annotations

import math

import numpy as np


def score_brute(
    keys: np.ndarray,
    q_real: np.ndarray,
    q_imag: np.ndarray,
    q_abs: np.ndarray,
    freq_scale_sq: np.ndarray,
    omega: np.ndarray,
    offsets: list[float],
    round_start: int,
    *,
    rotary_dim: int | None = None,
    q_pass: np.ndarray | None = None,
    interleaved: bool = False,
    aggregation: str = "mean",
) -> np.ndarray:
    """keys [T, kv, D]; stats [kv, qpk, F] (q_pass [kv, qpk, P]) -> [kv, qpk, T].

    The first term is the RoPE attention logit of the mean query rotated to
    the future position p = rs + o against the (already rotated) cached key:
    Re( q_f e^{i p w_f} conj(k_f) ), summed over frequencies and then averaged
    (aggregation "mean") or maximised (aggregation "max") over the offsets o.
    score = agg_o sum_f a_f Re( q_f e^{i (o+rs) w_f} conj(k_f) )
          + sum_f a_f (q_abs_f - |q_f|) |k_f|  + sum_p q_pass_p k_p
    with q_f = qr + i qi, k_f = kr + i ki, a_f = sqrt(freq_scale_sq).
    """
    if aggregation not in ("mean", "max"):
        raise ValueError(aggregation)
    keys = np.asarray(keys, dtype=np.float64)
    tokens, kv_heads, head_dim = keys.shape
    rotary = head_dim if rotary_dim is None else rotary_dim
    freq = rotary // 2
    qpk = q_real.shape[1]
    out = np.zeros((kv_heads, qpk, tokens))
    for h in range(kv_heads):
        for g in range(qpk):
            for t in range(tokens):
                total = 0.0
                per_offset = [0.0] * len(offsets)
                for f in range(freq):
                    if interleaved:
                        kr, ki = keys[t, h, 2 * f], keys[t, h, 2 * f + 1]
                    else:
                        kr, ki = keys[t, h, f], keys[t, h, freq + f]
                    qr, qi = float(q_real[h, g, f]), float(q_imag[h, g, f])
                    a = math.sqrt(float(freq_scale_sq[h, g, f]))
                    k = complex(kr, ki)
                    q = complex(qr, qi)
                    for i, o in enumerate(offsets):
                        phi = (float(o) + round_start) * float(omega[f])
                        per_offset[i] += a * (q * complex(math.cos(phi), math.sin(phi)) * k.conjugate()).real
                    total += a * (float(q_abs[h, g, f]) - math.sqrt(qr * qr + qi * qi + 1e-8)) * abs(k)
                total += sum(per_offset) / len(offsets) if aggregation == "mean" else max(per_offset)
                if rotary < head_dim:
                    total += float(np.dot(np.asarray(q_pass[h, g], dtype=np.float64), keys[t, h, rotary:]))
                out[h, g, t] = total
    return out


def normalized_layer_max(raw: np.ndarray) -> np.ndarray:
    """max over heads of (s - mean)/sqrt(max(var, 1e-6)), population variance."""
    raw = np.asarray(raw, dtype=np.float64).reshape(-1, raw.shape[-1])
    mean = raw.mean(axis=1, keepdims=True)
    var = ((raw - mean) ** 2).mean(axis=1, keepdims=True)
    return ((raw - mean) / np.sqrt(np.maximum(var, 1e-6))).max(axis=0)


def select_stable(scores: np.ndarray, budget: int, prefix: int, recent: int, segments: int, policy: str) -> np.ndarray:
    """Keep set with the deterministic tie rule (higher score first, then lower
    index), protected windows and v3 quotas computed from their definition."""
    scores = np.asarray(scores)
    n = scores.shape[0]
    prefix = min(prefix, n)
    recent = min(recent, n - prefix)
    keep = set(range(prefix)) | set(range(n - recent, n))

    def top(lo: int, hi: int, k: int) -> list[int]:
        idx = sorted(range(lo, hi), key=lambda i: (-order_key(scores[i]), i))
        return idx[:k]

    mc = n - prefix - recent
    if policy == "global":
        keep |= set(top(prefix, n - recent, budget - prefix - recent))
    else:
        evict = n - budget
        for s in range(segments):
            a = prefix + mc * s // segments
            b = prefix + mc * (s + 1) // segments
            if b == a:
                continue
            quota = (b - a) - (evict * (b - prefix) // mc - evict * (a - prefix) // mc)
            keep |= set(top(a, b, max(quota, 0)))
    return np.array(sorted(keep), dtype=np.int64)


def order_key(x: float) -> int:
    """Total order on float32 bit patterns: -NaN < -inf < ... < -0 < +0 < ...
    < +inf < +NaN, so NaN ranks above every number as torch.topk ranks it."""
    bits = int(np.array(x, dtype=np.float32).view(np.uint32))
    return (~bits & 0xFFFFFFFF) if bits & 0x80000000 else (bits | 0x80000000)


def slot_mapping(query_start_loc, positions, request_offsets, block_table, block_size, num_tokens):
    """Slot of every token written at its physical position, by plain loops:
    request r owns tokens [qsl[r], qsl[r+1]); p = position - offset[r];
    slot = table[r][p // bs] * bs + p % bs, or -1 when p < 0, the block index
    is past the table row or the entry is negative; tokens after the last
    request are padding (-1).  Returns (slots, physical positions)."""
    slots = [-1] * num_tokens
    phys = [int(x) for x in positions[:num_tokens]]
    num_reqs = len(query_start_loc) - 1
    for r in range(num_reqs):
        off = 0 if request_offsets is None else int(request_offsets[r])
        for i in range(int(query_start_loc[r]), min(int(query_start_loc[r + 1]), num_tokens)):
            p = int(positions[i]) - off
            phys[i] = p
            if p < 0:
                continue
            blk = p // block_size
            if blk >= len(block_table[r]):
                continue
            page = int(block_table[r][blk])
            if page >= 0:
                slots[i] = page * block_size + p % block_size
    return slots, phys
