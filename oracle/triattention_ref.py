"""Torch-CPU restatement of the reference TriAttention torch path (oracle).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  Each function follows the
cited reference code with the same torch operations in the same order, so it
reproduces what the reference computes on the CPU/generic device path
(tri/kernels.py:99-100 routes every non-NPU device there).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

BLOCK_SIZE = 128


# --------------------------------------------------------------- scoring ----


def build_geometric_offsets(maximum: int) -> torch.Tensor:
    """tri/scoring.py:11-20."""
    if maximum < 1:
        raise ValueError("maximum scoring offset must be positive")
    out = []
    v = 1
    while v <= maximum:
        out.append(float(v))
        v *= 2
    return torch.tensor(out, dtype=torch.float32)


@dataclass(frozen=True)
class LayerStats:
    """Grouped per-layer calibration, [kv_heads, qpk, width] float32
    (DeviceLayerCalibrationStats, tri/stats.py:42-51)."""

    q_mean_real: torch.Tensor
    q_mean_imag: torch.Tensor
    q_abs_mean: torch.Tensor
    freq_scale_sq: torch.Tensor
    omega: torch.Tensor
    rope_style: str = "half"
    rotary_dim: int | None = None
    q_pass_mean: torch.Tensor | None = None


def score_post_rope_keys(
    keys: torch.Tensor, stats: LayerStats, *, round_start: int, offsets: torch.Tensor, aggregation: str = "mean"
) -> torch.Tensor:
    """tri/scoring.py:23-120: keys [T, kv, D] -> scores [kv, qpk, T]."""
    if keys.ndim != 3:
        raise ValueError("keys must have shape [tokens, kv_heads, head_dim]")
    tokens, kv_heads, head_dim = keys.shape
    rotary = head_dim if stats.rotary_dim is None else stats.rotary_dim
    freq = rotary // 2
    if stats.q_mean_real.shape[0] != kv_heads or stats.q_mean_real.shape[-1] != freq:
        raise ValueError("calibration does not match cache keys")
    k = keys.to(dtype=torch.float32).permute(1, 0, 2)
    rot = k[..., :rotary]
    if stats.rope_style == "interleaved":
        kr, ki = rot[..., 0::2], rot[..., 1::2]
    else:
        kr, ki = rot[..., :freq], rot[..., freq:rotary]
    qr = stats.q_mean_real.unsqueeze(2)
    qi = stats.q_mean_imag.unsqueeze(2)
    kr = kr.unsqueeze(1)
    ki = ki.unsqueeze(1)
    prod_re = qr * kr + qi * ki
    prod_im = qi * kr - qr * ki
    fscale = torch.sqrt(stats.freq_scale_sq).unsqueeze(2)
    phases = (offsets.unsqueeze(1) + float(round_start)) * stats.omega.unsqueeze(0)
    if aggregation == "mean":
        c = torch.cos(phases).mean(dim=0).view(1, 1, 1, freq)
        s = torch.sin(phases).mean(dim=0).view(1, 1, 1, freq)
        scores = (fscale * (prod_re * c - prod_im * s)).sum(dim=-1)
    elif aggregation == "max":
        scores = torch.full((kv_heads, stats.q_mean_real.shape[1], tokens), float("-inf"), dtype=torch.float32)
        for phase in phases.unbind(0):
            c = torch.cos(phase).view(1, 1, 1, freq)
            s = torch.sin(phase).view(1, 1, 1, freq)
            scores = torch.maximum(scores, (fscale * (prod_re * c - prod_im * s)).sum(dim=-1))
    else:
        raise ValueError(f"unsupported score aggregation: {aggregation}")
    kabs = torch.sqrt(kr.square() + ki.square())
    qabs_mean = torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)
    extra_coef = (stats.q_abs_mean - qabs_mean).unsqueeze(2)
    scores = scores + (kabs * extra_coef * fscale).sum(dim=-1)
    if rotary < head_dim:
        if stats.q_pass_mean is None or stats.q_pass_mean.shape[-1] != head_dim - rotary:
            raise ValueError("partial-RoPE scoring requires matching q_pass_mean")
        kpass = k[..., rotary:].unsqueeze(1)
        scores = scores + (stats.q_pass_mean.unsqueeze(2) * kpass).sum(dim=-1)
    return scores


def normalize_head_scores(scores: torch.Tensor, mean: torch.Tensor, variance: torch.Tensor) -> torch.Tensor:
    """tri/scoring.py:123-128."""
    return (scores - mean.unsqueeze(-1)) / torch.sqrt(variance.clamp_min(1e-6)).unsqueeze(-1)


# -------------------------------------------------------------- selection ---


def select_keep_indices(
    scores: torch.Tensor, *, budget: int, protected_prefix: int, protected_recent: int, segments: int, policy: str
) -> torch.Tensor:
    """tri/selection.py:108-196 (CPU branch; v3 per-segment loop)."""
    if scores.ndim != 1:
        raise ValueError("scores must be one-dimensional")
    n = int(scores.numel())
    if budget <= 0 or budget > n:
        raise ValueError("budget must be in [1, token_count]")
    if protected_prefix < 0 or protected_recent < 0:
        raise ValueError("protected windows must be non-negative")
    if protected_prefix + protected_recent > budget:
        raise ValueError("protected windows cannot exceed the selection budget")
    if segments <= 0:
        raise ValueError("segments must be positive")
    prefix = min(protected_prefix, n)
    recent = min(protected_recent, n - prefix)
    protected = torch.zeros(n, dtype=torch.bool)
    if prefix:
        protected[:prefix] = True
    if recent:
        protected[n - recent :] = True
    if policy == "global":
        ranked = scores.clone()
        ranked[protected] = float("inf")
        chosen = torch.topk(ranked, k=budget, largest=True, sorted=False).indices
        return torch.sort(chosen).values.contiguous()
    if policy != "v3":
        raise ValueError(f"unsupported position policy: {policy}")
    ms, stop_all = prefix, n - recent
    mc = stop_all - ms
    evict = n - budget
    if evict > mc:
        raise ValueError("selection budget leaves too few slots for protected tokens")
    keep = protected.clone()
    for seg in range(segments):
        a = ms + mc * seg // segments
        b = ms + mc * (seg + 1) // segments
        length = b - a
        if length == 0:
            continue
        quota = length - (evict * (b - ms) // mc - evict * (a - ms) // mc)
        if quota <= 0:
            continue
        if quota == length:
            keep[a:b] = True
            continue
        local = torch.topk(scores[a:b], k=quota, largest=True, sorted=False).indices
        keep[a + local] = True
    chosen = torch.nonzero(keep, as_tuple=False).flatten()
    if int(chosen.numel()) != budget:
        raise RuntimeError(f"V3 selected {chosen.numel()} tokens, expected exactly {budget}")
    return chosen.contiguous()


def v3_batched_plan(n: int, budget: int, prefix: int, recent: int, segments: int):
    """tri/selection.py:24-63: equal-width plan or None."""
    mc = n - prefix - recent
    evict = n - budget
    if mc == 0 or mc % segments:
        return None
    width = mc // segments
    quotas = [width - evict * ((s + 1) * width) // mc + evict * (s * width) // mc for s in range(segments)]
    if min(quotas) <= 0:
        return None
    return width, quotas


def select_v3_batched(scores: torch.Tensor, *, budget: int, prefix: int, recent: int, segments: int):
    """tri/selection.py:66-105: one batched top-k over equal-width segments."""
    n = int(scores.numel())
    plan = v3_batched_plan(n, budget, prefix, recent, segments)
    if plan is None:
        return None
    width, quotas = plan
    max_q = max(quotas)
    sorted_topk = min(quotas) != max_q
    rows = scores[prefix : n - recent if recent else None].reshape(segments, width)
    ranked = torch.topk(rows, k=max_q, dim=1, sorted=sorted_topk).indices
    q = torch.tensor(quotas)[:, None]
    ranks = torch.arange(max_q)[None, :]
    chosen = torch.where(ranks < q, ranked, width)
    chosen = torch.sort(chosen, dim=1).values
    chosen += (torch.arange(segments) * width + prefix)[:, None]
    target_base = torch.tensor([prefix + sum(quotas[:s]) for s in range(segments)])[:, None]
    targets = torch.where(ranks < q, ranks + target_base, 0)
    out = torch.empty(budget, dtype=torch.long)
    out.scatter_(0, targets.flatten(), chosen.flatten())
    if prefix:
        out[:prefix] = torch.arange(prefix)
    else:
        out[0] = chosen[0, 0]
    if recent:
        out[-recent:] = torch.arange(n - recent, n)
    return out.contiguous()


# ------------------------------------------------------------------ cache ---


def token_slots(block_ids: torch.Tensor, token_indices: torch.Tensor, block_size: int) -> torch.Tensor:
    """tri/cache.py:9-15."""
    blocks = torch.div(token_indices, block_size, rounding_mode="floor")
    within = torch.remainder(token_indices, block_size)
    return block_ids.index_select(0, blocks) * block_size + within


def gather_slots(cache: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
    """tri/cache.py:18-33 (both the flat and the strided form)."""
    bs = cache.shape[1]
    if cache.is_contiguous():
        return cache.view(-1, cache.shape[2], cache.shape[3]).index_select(0, slots)
    return cache[torch.div(slots, bs, rounding_mode="floor"), torch.remainder(slots, bs)]


def write_slots(cache: torch.Tensor, slots: torch.Tensor, values: torch.Tensor) -> None:
    """tri/cache.py:36-45."""
    bs = cache.shape[1]
    if cache.is_contiguous():
        cache.view(-1, cache.shape[2], cache.shape[3]).index_copy_(0, slots, values)
        return
    cache[torch.div(slots, bs, rounding_mode="floor"), torch.remainder(slots, bs)] = values


def gather_paged_tokens(cache: torch.Tensor, block_ids: torch.Tensor, token_indices: torch.Tensor, block_size: int) -> torch.Tensor:
    """tri/cache.py:48-58."""
    if cache.ndim != 4 or cache.shape[1] != block_size:
        raise ValueError("cache must use [blocks, block, heads, dim] layout")
    return gather_slots(cache, token_slots(block_ids, token_indices, block_size))


def gather_paged_range(cache: torch.Tensor, block_ids: torch.Tensor, *, start: int, count: int, block_size: int) -> torch.Tensor:
    """tri/cache.py:61-76."""
    return gather_paged_tokens(cache, block_ids, torch.arange(start, start + count, dtype=torch.long), block_size)


def materialize_token_slots(k_cache, v_cache, source_slots, destination_slots) -> None:
    """tri/cache.py:100-112: gather into workspaces, then scatter."""
    k_ws = gather_slots(k_cache, source_slots).clone()
    v_ws = gather_slots(v_cache, source_slots).clone()
    write_slots(k_cache, destination_slots, k_ws)
    write_slots(v_cache, destination_slots, v_ws)


def materialize_selected_tokens(k_cache, v_cache, source_block_ids, destination_block_ids, keep, block_size) -> None:
    """tri/cache.py:79-97."""
    src = token_slots(source_block_ids, keep, block_size)
    dst = token_slots(destination_block_ids, torch.arange(keep.shape[0], dtype=torch.long), block_size)
    materialize_token_slots(k_cache, v_cache, src, dst)


# ------------------------------------------------------------- the method ---


@dataclass
class MethodConfig:
    budget: int
    recent: int = 128
    prefix: int = 0
    segments: int = 8
    policy: str = "global"
    score_aggregation: str = "mean"
    layer_aggregation: str = "mean"
    score_chunk_size: int = 512
    score_layer_stride: int = 8


def score_layers(
    scoring_k_caches: list[torch.Tensor],
    layer_stats: list[LayerStats],
    block_ids: torch.Tensor,
    n_tokens: int,
    round_start: int,
    offsets: torch.Tensor,
    cfg: MethodConfig,
) -> tuple[list[torch.Tensor], list[tuple[torch.Tensor, torch.Tensor]]]:
    """Raw scores [kv, qpk, N] and (var, mean) per scoring layer
    (tri/method.py:405-423: chunked gather + score, then var_mean)."""
    raws, stats = [], []
    for cache, st in zip(scoring_k_caches, layer_stats):
        kv, qpk = st.q_mean_real.shape[:2]
        raw = torch.empty((kv, qpk, n_tokens), dtype=torch.float32)
        for start in range(0, n_tokens, cfg.score_chunk_size):
            count = min(cfg.score_chunk_size, n_tokens - start)
            keys = gather_paged_range(cache, block_ids, start=start, count=count, block_size=BLOCK_SIZE)
            raw[:, :, start : start + count].copy_(
                score_post_rope_keys(keys, st, round_start=round_start, offsets=offsets, aggregation=cfg.score_aggregation)
            )
        var, mean = torch.var_mean(raw, dim=-1, correction=0)
        raws.append(raw)
        stats.append((var, mean))
    return raws, stats


def aggregate_layers(raws, stats, cfg: MethodConfig) -> torch.Tensor:
    """_aggregate_torch per layer then layer mean + nan_to_num (tri/method.py:423-467,477-503)."""
    agg = None
    for index, (raw, (var, mean)) in enumerate(zip(raws, stats)):
        layer = normalize_head_scores(raw, mean, var).amax(dim=(0, 1))
        if index == 0:
            agg = layer.clone()
        elif cfg.layer_aggregation == "mean":
            agg.add_(layer)
        else:
            torch.maximum(agg, layer, out=agg)
    if cfg.layer_aggregation == "mean":
        agg.div_(float(len(raws)))
    agg.nan_to_num_(nan=float("-inf"), posinf=1e30, neginf=float("-inf"))
    return agg


def method_select(
    scoring_k_caches, layer_stats, block_ids, n_tokens, round_start, offsets, cfg: MethodConfig
) -> dict[str, object]:
    """TriAttentionMethod._select_keep_indices, CPU branch (tri/method.py:297-475)."""
    raws, stats = score_layers(scoring_k_caches, layer_stats, block_ids, n_tokens, round_start, offsets, cfg)
    agg = aggregate_layers(raws, stats, cfg)
    keep = select_keep_indices(
        agg,
        budget=cfg.budget,
        protected_prefix=cfg.prefix,
        protected_recent=cfg.recent,
        segments=cfg.segments,
        policy=cfg.policy,
    )
    return {"raw": raws, "stats": stats, "agg": agg, "keep": keep}


def method_compress(k_caches, v_caches, source_block_ids, destination_block_ids, keep, budget) -> None:
    """compress materialisation over every bound layer (tri/method.py:272-288)."""
    src = token_slots(source_block_ids, keep, BLOCK_SIZE)
    dst = token_slots(destination_block_ids, torch.arange(budget, dtype=torch.long), BLOCK_SIZE)
    for k, v in zip(k_caches, v_caches):
        materialize_token_slots(k, v, src, dst)


def rewrite_block_table(source_ids: list[int], destination_ids: list[int] | None, budget: int) -> tuple[list[int], list[int]]:
    """New table and released pages after commit (pkg/provider.py:596-601,
    pkg/stateful.py:327-338).  Private destinations: the table becomes the
    destination pages and every source page is released in reverse order.
    In place: the first ceil(budget/128) source pages are kept."""
    nb = -(-budget // BLOCK_SIZE)
    if destination_ids is None:
        return list(source_ids[:nb]), list(reversed(source_ids[nb:]))
    return list(destination_ids[:nb]), list(reversed(source_ids))


# ------------------------------------------------- decode after compaction --


def shift_positions(positions: torch.Tensor, request_indices: torch.Tensor, request_offsets: torch.Tensor) -> torch.Tensor:
    """tri/kernels.py:35-47: positions - request_offsets[request_indices]."""
    return torch.sub(positions, request_offsets.index_select(0, request_indices.to(torch.long)))


def physical_seq_lens(seq_lens: torch.Tensor, request_offsets: torch.Tensor, num_reqs: int) -> torch.Tensor:
    """pkg/provider.py:707-728 (device half): seq_lens[:num_reqs] - offsets[:num_reqs]."""
    out = seq_lens.clone()
    out[:num_reqs].sub_(request_offsets[:num_reqs].to(out.dtype))
    return out
