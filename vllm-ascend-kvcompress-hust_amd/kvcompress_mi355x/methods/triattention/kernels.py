"""HIP entry points under the reference's kernel-wrapper names (tri/kernels.py).

Each function keeps the reference signature and argument meaning.  Where the
reference returns ``False`` for "not my device" so its caller can fall back to
torch, these wrappers raise instead: the MI355X path has no host fallback.
All work is enqueued on the current stream of the tensors' device.
"""

from __future__ import annotations

import torch

from ... import _native
from . import _device as dev


def prepare_mean_phase_coefficients(
    omega: torch.Tensor,
    offset_cos_mean: torch.Tensor,
    offset_sin_mean: torch.Tensor,
    round_start: int,
    phase_cos: torch.Tensor,
    phase_sin: torch.Tensor,
) -> bool:
    """Angle-addition phase table for every (layer, frequency) (tri/kernels.py:85-122)."""
    for name, t in (
        ("omega", omega),
        ("offset_cos_mean", offset_cos_mean),
        ("offset_sin_mean", offset_sin_mean),
        ("phase_cos", phase_cos),
        ("phase_sin", phase_sin),
    ):
        dev.require_hip(t, name)
        dev.require_dtype(t, name, torch.float32)
        dev.require_contiguous(t, name)
    if not (omega.shape == offset_cos_mean.shape == offset_sin_mean.shape == phase_cos.shape == phase_sin.shape):
        raise ValueError("phase coefficient tensors must have matching shapes")
    _native.call(
        "kvc_shift_mean_phases",
        dev.stream_handle(omega.device),
        int(omega.numel()),
        int(round_start),
        dev.ptr(omega),
        dev.ptr(offset_cos_mean),
        dev.ptr(offset_sin_mean),
        dev.ptr(phase_cos),
        dev.ptr(phase_sin),
    )
    return True


def mean_phase_table(
    round_starts: torch.Tensor, offsets: torch.Tensor, omega: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Directly evaluated phase means, as the torch scoring path forms them
    (tri/scoring.py:77-80): [n_seq, layers, F] for int64 round_starts [n_seq]
    and omega [layers, F]."""
    for name, t in (("round_starts", round_starts), ("offsets", offsets), ("omega", omega)):
        dev.require_hip(t, name)
        dev.require_contiguous(t, name)
    dev.require_dtype(round_starts, "round_starts", torch.int64)
    dev.require_dtype(offsets, "offsets", torch.float32)
    dev.require_dtype(omega, "omega", torch.float32)
    if omega.ndim != 2 or round_starts.ndim != 1 or offsets.ndim != 1:
        raise ValueError("expected round_starts [n], offsets [o], omega [layers, F]")
    n_seq, (layers, freq) = int(round_starts.numel()), omega.shape
    cos = torch.empty((n_seq, layers, freq), dtype=torch.float32, device=omega.device)
    sin = torch.empty_like(cos)
    _native.call(
        "kvc_mean_phases",
        dev.stream_handle(omega.device),
        n_seq,
        int(layers),
        int(freq),
        dev.ptr(round_starts),
        dev.ptr(offsets),
        int(offsets.numel()),
        dev.ptr(omega),
        dev.ptr(cos),
        dev.ptr(sin),
    )
    return cos, sin


def _single_layer_scoring(
    k_cache: torch.Tensor,
    source_block_ids: torch.Tensor,
    q_real: torch.Tensor,
    q_imag: torch.Tensor,
    frequency_scale: torch.Tensor,
    extra_coefficient: torch.Tensor,
    num_tokens: int,
    output: torch.Tensor,
    block_size: int,
    q_pass_mean: torch.Tensor | None,
    rotary_dim: int | None,
) -> dict:
    """Checks shared by the one-layer scorers; returns the launch arguments
    that do not depend on the offset aggregation."""
    if block_size != 128:
        raise ValueError("the HIP scorer addresses 128-token cache blocks")
    dev.validate_cache(k_cache, "k_cache", block_size)
    kv_heads, qpk, freq = q_real.shape
    rotary = 2 * freq if rotary_dim is None else int(rotary_dim)
    head_dim = int(k_cache.shape[-1])
    if rotary != 2 * freq or not 0 < rotary <= head_dim:
        raise ValueError("rotary_dim must match the calibrated frequency count")
    pass_dim = head_dim - rotary
    if pass_dim:
        if q_pass_mean is None or tuple(q_pass_mean.shape) != (kv_heads, qpk, pass_dim):
            raise ValueError("partial-RoPE scoring requires matching q_pass_mean")
        if not q_pass_mean.is_contiguous():
            raise ValueError("q_pass_mean must be contiguous")
    elif q_pass_mean is not None:
        raise ValueError("full-RoPE scoring must not pass q_pass_mean")
    if int(k_cache.shape[2]) != kv_heads:
        raise ValueError("calibration KV-head count does not match cache keys")
    dev.require_16_byte_pages(k_cache, "k_cache")
    for name, t in (
        ("q_real", q_real),
        ("q_imag", q_imag),
        ("frequency_scale", frequency_scale),
        ("extra_coefficient", extra_coefficient),
    ):
        dev.require_hip(t, name)
        if tuple(t.shape) != (kv_heads, qpk, freq):
            raise ValueError(f"{name} must have shape {(kv_heads, qpk, freq)}")
    dev.require_hip(output, "output")
    dev.require_dtype(output, "output", torch.float32)
    if output.ndim != 3 or tuple(output.shape[:2]) != (kv_heads, qpk) or output.shape[2] < num_tokens:
        raise ValueError("output must be [kv_heads, queries_per_kv, >= num_tokens]")
    if output.stride(2) != 1 or output.stride(0) != qpk * output.stride(1):
        raise ValueError("output query rows must be contiguous and evenly strided")
    num_tokens = int(num_tokens)
    blocks = source_block_ids.to(dtype=torch.int64).contiguous()
    dev.require_hip(blocks, "source_block_ids")
    if blocks.numel() * block_size < num_tokens:
        raise ValueError("source block table does not cover num_tokens")
    device = k_cache.device

    def f32(t: torch.Tensor) -> torch.Tensor:
        return t.to(dtype=torch.float32).contiguous()

    return dict(
        device=device,
        kv_heads=kv_heads,
        qpk=qpk,
        freq=freq,
        rotary=rotary,
        head_dim=head_dim,
        num_tokens=num_tokens,
        blocks=blocks,
        desc=dev.one_sequence_descriptor(k_cache, num_tokens, blocks.numel()),
        calib=(f32(q_real), f32(q_imag), f32(frequency_scale), f32(extra_coefficient)),
        q_pass=f32(q_pass_mean) if q_pass_mean is not None else None,
    )


def _launch_single_layer(entry: str, a: dict, k_cache, rope_style, phase_args: tuple, output, ws_bytes: int) -> None:
    if ws_bytes == 0:
        raise ValueError("unsupported scoring shape for the MI355X kernel")
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=a["device"])
    qr, qi, sc, ex = a["calib"]
    _native.call(
        entry,
        dev.stream_handle(a["device"]),
        dev.cache_dtype_code(k_cache.dtype),
        1,
        a["desc"]["layer_ptrs"],
        int(k_cache.shape[0]),
        int(k_cache.stride(0)),
        a["kv_heads"],
        a["head_dim"],
        a["rotary"],
        a["qpk"],
        dev.rope_style_code(rope_style),
        1,
        a["num_tokens"],
        a["desc"]["seq_lens"],
        a["desc"]["token_offsets"],
        a["desc"]["block_offsets"],
        dev.ptr(a["blocks"]),
        dev.ptr(qr),
        dev.ptr(qi),
        dev.ptr(sc),
        dev.ptr(ex),
        dev.ptr(a["q_pass"]),
        *phase_args,
        dev.ptr(output),
        0,
        1,
        int(output.stride(1)),
        dev.ptr(workspace),
        ws_bytes,
    )


def score_paged_keys_mean_precomputed(
    k_cache: torch.Tensor,
    source_block_ids: torch.Tensor,
    q_real: torch.Tensor,
    q_imag: torch.Tensor,
    frequency_scale: torch.Tensor,
    extra_coefficient: torch.Tensor,
    phase_cos: torch.Tensor,
    phase_sin: torch.Tensor,
    num_tokens: int,
    output: torch.Tensor,
    block_size: int,
    rope_style: str,
    *,
    q_pass_mean: torch.Tensor | None = None,
    rotary_dim: int | None = None,
) -> bool:
    """Score one layer's paged keys with precomputed phases (tri/kernels.py:247-317).

    ``output`` is [kv_heads, queries_per_kv, >= num_tokens] float32 with
    contiguous query rows, as in the reference workspace layout."""
    a = _single_layer_scoring(
        k_cache, source_block_ids, q_real, q_imag, frequency_scale, extra_coefficient, num_tokens, output, block_size,
        q_pass_mean, rotary_dim,
    )
    for name, t in (("phase_cos", phase_cos), ("phase_sin", phase_sin)):
        dev.require_hip(t, name)
        if t.numel() != a["freq"]:
            raise ValueError(f"{name} must hold {a['freq']} values")
    pc = phase_cos.reshape(-1).to(dtype=torch.float32).contiguous()
    ps = phase_sin.reshape(-1).to(dtype=torch.float32).contiguous()
    ws_bytes = _native.load().kvc_score_workspace_bytes(
        1, a["kv_heads"], a["head_dim"], a["rotary"], a["qpk"], 1, max(a["num_tokens"], 1)
    )
    _launch_single_layer("kvc_score_paged", a, k_cache, rope_style, (dev.ptr(pc), dev.ptr(ps), 0), output, ws_bytes)
    return True


def score_paged_keys_max(
    k_cache: torch.Tensor,
    source_block_ids: torch.Tensor,
    q_real: torch.Tensor,
    q_imag: torch.Tensor,
    frequency_scale: torch.Tensor,
    extra_coefficient: torch.Tensor,
    omega: torch.Tensor,
    offsets: torch.Tensor,
    round_start: int,
    num_tokens: int,
    output: torch.Tensor,
    block_size: int,
    rope_style: str,
    *,
    q_pass_mean: torch.Tensor | None = None,
    rotary_dim: int | None = None,
) -> bool:
    """One layer's scores with the rotary term maximised over the offsets,
    score_post_rope_keys(aggregation="max") (tri/scoring.py:84-97), which the
    reference runs on the torch path only (tri/method.py:348-431).  Arguments
    as score_paged_keys_mean_precomputed plus omega [F], offsets [O] and the
    round start the phases are formed at."""
    a = _single_layer_scoring(
        k_cache, source_block_ids, q_real, q_imag, frequency_scale, extra_coefficient, num_tokens, output, block_size,
        q_pass_mean, rotary_dim,
    )
    for name, t in (("omega", omega), ("offsets", offsets)):
        dev.require_hip(t, name)
    if omega.numel() != a["freq"]:
        raise ValueError(f"omega must hold {a['freq']} values")
    n_off = int(offsets.numel())
    if n_off == 0:
        raise ValueError("at least one offset is required")
    device = a["device"]
    om = omega.reshape(-1).to(dtype=torch.float32).contiguous()
    off = offsets.reshape(-1).to(dtype=torch.float32).contiguous()
    rs = torch.tensor([int(round_start)], dtype=torch.int64, device=device)
    pc = torch.empty((n_off, a["freq"]), dtype=torch.float32, device=device)
    ps = torch.empty_like(pc)
    _native.call(
        "kvc_offset_phases", dev.stream_handle(device), 1, 1, a["freq"], dev.ptr(rs), dev.ptr(off), n_off, dev.ptr(om),
        dev.ptr(pc), dev.ptr(ps),
    )
    ws_bytes = _native.load().kvc_score_max_workspace_bytes(
        1, a["kv_heads"], a["head_dim"], a["rotary"], a["qpk"], 1, max(a["num_tokens"], 1), n_off
    )
    _launch_single_layer(
        "kvc_score_paged_max", a, k_cache, rope_style, (dev.ptr(pc), dev.ptr(ps), n_off, 0), output, ws_bytes
    )
    return True


def score_paged_keys_mean(
    k_cache: torch.Tensor,
    source_block_ids: torch.Tensor,
    q_real: torch.Tensor,
    q_imag: torch.Tensor,
    frequency_scale: torch.Tensor,
    extra_coefficient: torch.Tensor,
    omega: torch.Tensor,
    offset_cos_mean: torch.Tensor,
    offset_sin_mean: torch.Tensor,
    round_start: int,
    num_tokens: int,
    output: torch.Tensor,
    block_size: int,
    rope_style: str,
    *,
    q_pass_mean: torch.Tensor | None = None,
    rotary_dim: int | None = None,
) -> bool:
    """Compatibility form that prepares one layer's phases (tri/kernels.py:320-362)."""
    phase_cos = torch.empty_like(omega, dtype=torch.float32)
    phase_sin = torch.empty_like(phase_cos)
    prepare_mean_phase_coefficients(
        omega.float().contiguous(),
        offset_cos_mean.float().contiguous(),
        offset_sin_mean.float().contiguous(),
        round_start,
        phase_cos,
        phase_sin,
    )
    return score_paged_keys_mean_precomputed(
        k_cache,
        source_block_ids,
        q_real,
        q_imag,
        frequency_scale,
        extra_coefficient,
        phase_cos,
        phase_sin,
        num_tokens,
        output,
        block_size,
        rope_style,
        q_pass_mean=q_pass_mean,
        rotary_dim=rotary_dim,
    )


def aggregate_normalized_scores(
    scores: torch.Tensor,
    mean: torch.Tensor,
    variance: torch.Tensor,
    aggregate: torch.Tensor,
    num_tokens: int,
    *,
    layer_aggregation: str,
    first_layer: bool,
) -> bool:
    """Normalise, max over query heads, accumulate one layer (tri/kernels.py:407-437).

    Uses the reference device kernel's rsqrt form; ``scores`` is
    [kv_heads, queries_per_kv, >= num_tokens] with evenly strided query rows."""
    for name, t in (("scores", scores), ("mean", mean), ("variance", variance), ("aggregate", aggregate)):
        dev.require_hip(t, name)
        dev.require_dtype(t, name, torch.float32)
    if layer_aggregation not in ("mean", "max"):
        raise ValueError(f"unsupported layer aggregation {layer_aggregation!r}")
    heads = int(mean.numel())
    if scores.stride(-1) != 1:
        raise ValueError("score rows must be contiguous")
    flat_scores = scores.reshape(heads, scores.shape[-1]) if scores.ndim == 3 else scores
    if flat_scores.shape[0] != heads or variance.numel() != heads:
        raise ValueError("mean/variance must hold one value per query head")
    num_tokens = int(num_tokens)
    device = scores.device
    m = mean.reshape(-1).contiguous()
    v = variance.reshape(-1).contiguous()
    # One-sequence descriptor words (token offsets, sequence length), kept on
    # the device per value: nothing is copied to the device per call, so the
    # call can be captured into a graph.
    desc = dev.one_sequence_descriptor(aggregate, num_tokens, 0)
    flags = _native.AGG_RSQRT | (0 if first_layer else _native.AGG_ACCUMULATE)
    _native.call(
        "kvc_aggregate",
        dev.stream_handle(device),
        1,
        heads,
        1,
        num_tokens,
        desc["seq_lens"],
        desc["token_offsets"],
        dev.ptr(flat_scores),
        0,
        1,
        int(flat_scores.stride(0)),
        dev.ptr(m),
        dev.ptr(v),
        0,
        0,
        _native.LAYER_MEAN if layer_aggregation == "mean" else _native.LAYER_MAX,
        flags,
        dev.ptr(aggregate),
    )
    return True


# ------------------------------------------------------- decode after compaction --


def shift_positions(
    positions: torch.Tensor,
    request_indices: torch.Tensor,
    request_offsets: torch.Tensor,
    output: torch.Tensor,
) -> torch.Tensor:
    """Physical positions of a step's tokens (tri/kernels.py:35-47):
    ``output = positions - request_offsets[request_indices]``.

    positions, request_offsets and output are int64; request_indices int32 or
    int64 (the reference converts them to int64 before indexing)."""
    for name, t in (("positions", positions), ("request_indices", request_indices),
                    ("request_offsets", request_offsets), ("output", output)):
        dev.require_hip(t, name)
        dev.require_contiguous(t, name)
    for name, t in (("positions", positions), ("request_offsets", request_offsets), ("output", output)):
        dev.require_dtype(t, name, torch.int64)
    if request_indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("request_indices must be int32 or int64")
    n = int(positions.numel())
    if int(request_indices.numel()) != n or int(output.numel()) != n:
        raise ValueError("positions, request_indices and output must have the same length")
    _native.call(
        "kvc_shift_positions",
        dev.stream_handle(positions.device),
        dev.ptr(positions),
        dev.ptr(request_indices),
        request_indices.element_size(),
        dev.ptr(request_offsets),
        n,
        dev.ptr(output),
    )
    return output


def compute_physical_slot_mapping(
    query_start_loc: torch.Tensor,
    positions: torch.Tensor,
    request_offsets: torch.Tensor | None,
    block_table: torch.Tensor,
    block_size: int,
    slot_mapping: torch.Tensor,
    physical_positions: torch.Tensor | None = None,
) -> torch.Tensor:
    """Slot mapping of a step's tokens written at their physical positions:
    the slot-mapping hook of the reference (pkg/plugin.py:487-506 ->
    pkg/provider.py:687-705) and the host's compute_slot_mapping in one launch.

    query_start_loc: int32 [num_reqs + 1]; positions, slot_mapping (and
    physical_positions): int64 [num_tokens]; block_table: int32
    [>= num_reqs, max_blocks] with unit inner stride.  Padding tokens and
    positions outside the table map to -1."""
    for name, t in (("query_start_loc", query_start_loc), ("positions", positions),
                    ("block_table", block_table), ("slot_mapping", slot_mapping)):
        dev.require_hip(t, name)
    dev.require_dtype(query_start_loc, "query_start_loc", torch.int32)
    dev.require_dtype(positions, "positions", torch.int64)
    dev.require_dtype(block_table, "block_table", torch.int32)
    dev.require_dtype(slot_mapping, "slot_mapping", torch.int64)
    if block_table.ndim != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be [num_reqs, max_blocks] with contiguous rows")
    num_reqs = int(query_start_loc.numel()) - 1
    if num_reqs < 0 or int(block_table.shape[0]) < num_reqs:
        raise ValueError("block_table must have a row for every request")
    num_tokens = int(positions.numel())
    if int(slot_mapping.numel()) != num_tokens:
        raise ValueError("slot_mapping must have one entry per token")
    if request_offsets is not None:
        dev.require_hip(request_offsets, "request_offsets")
        dev.require_dtype(request_offsets, "request_offsets", torch.int64)
        if int(request_offsets.numel()) < num_reqs:
            raise ValueError("request_offsets must have an entry for every request")
    if physical_positions is not None:
        dev.require_hip(physical_positions, "physical_positions")
        dev.require_dtype(physical_positions, "physical_positions", torch.int64)
        if int(physical_positions.numel()) != num_tokens:
            raise ValueError("physical_positions must have one entry per token")
    _native.call(
        "kvc_physical_slot_mapping",
        dev.stream_handle(positions.device),
        num_reqs,
        dev.ptr(query_start_loc),
        dev.ptr(positions),
        dev.ptr(request_offsets),
        dev.ptr(block_table),
        int(block_table.stride(0)),
        int(block_table.shape[1]),
        int(block_size),
        num_tokens,
        dev.ptr(slot_mapping),
        dev.ptr(physical_positions),
    )
    return slot_mapping


def shift_seq_lens(seq_lens: torch.Tensor, request_offsets: torch.Tensor, num_reqs: int) -> torch.Tensor:
    """``seq_lens[:num_reqs] -= request_offsets[:num_reqs]`` in place, the
    device half of apply_physical_attention_lengths (pkg/provider.py:707-728)."""
    dev.require_hip(seq_lens, "seq_lens")
    dev.require_hip(request_offsets, "request_offsets")
    dev.require_contiguous(seq_lens, "seq_lens")
    dev.require_dtype(request_offsets, "request_offsets", torch.int64)
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise ValueError("seq_lens must be int32 or int64")
    if num_reqs > int(seq_lens.numel()) or num_reqs > int(request_offsets.numel()):
        raise ValueError("num_reqs exceeds the length or offset buffers")
    _native.call(
        "kvc_shift_lengths",
        dev.stream_handle(seq_lens.device),
        dev.ptr(seq_lens),
        seq_lens.element_size(),
        dev.ptr(request_offsets),
        int(num_reqs),
    )
    return seq_lens
