"""Kernel-level parity of the HIP path against the CPU oracle (needs a GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_agg_close, assert_scores_close
from oracle import brute
from oracle import triattention_ref as ref

pytestmark = pytest.mark.gpu


def _kvc():
    from kvcompress_mi355x.methods.triattention import cache, kernels, selection

    return kernels, selection, cache


def _random_stats(g, kv, qpk, freq, pass_dim, rotary, theta=1e6, style="half"):
    qr = torch.randn(kv, qpk, freq, generator=g)
    qi = torch.randn(kv, qpk, freq, generator=g)
    qa = torch.sqrt(qr.square() + qi.square()) + torch.rand(kv, qpk, freq, generator=g)
    fs = 0.5 + torch.rand(kv, qpk, freq, generator=g)
    omega = 1.0 / (theta ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
    qp = torch.randn(kv, qpk, pass_dim, generator=g) if pass_dim else None
    return ref.LayerStats(qr, qi, qa, fs, omega, style, rotary, qp)


@pytest.mark.parametrize("round_start", [300, 16384, 131072])
def test_mean_phase_table_matches_torch(hip_device, round_start: int) -> None:
    kernels, _, _ = _kvc()
    offsets = ref.build_geometric_offsets(32768)
    omega = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    omega2 = torch.stack([omega, omega * 0.5])
    rs = torch.tensor([round_start, round_start + 1], dtype=torch.int64)
    cos, sin = kernels.mean_phase_table(rs.to(hip_device), offsets.to(hip_device), omega2.to(hip_device))
    for b in range(2):
        for layer in range(2):
            phases = (offsets.unsqueeze(1) + float(rs[b])) * omega2[layer].unsqueeze(0)
            torch.testing.assert_close(cos[b, layer].cpu(), torch.cos(phases).mean(0), rtol=0, atol=2e-6)
            torch.testing.assert_close(sin[b, layer].cpu(), torch.sin(phases).mean(0), rtol=0, atol=2e-6)


def test_shift_phase_coefficients_formula(hip_device) -> None:
    kernels, _, _ = _kvc()
    omega = torch.tensor([[1.0, 0.1, 0.01, 0.001]] * 3)
    offsets = torch.tensor([1.0, 2.0, 4.0])
    oc = torch.cos(offsets.unsqueeze(1) * omega[0]).mean(0).expand(3, -1).contiguous()
    os_ = torch.sin(offsets.unsqueeze(1) * omega[0]).mean(0).expand(3, -1).contiguous()
    pc = torch.empty(3, 4, device=hip_device)
    ps = torch.empty_like(pc)
    assert kernels.prepare_mean_phase_coefficients(omega.to(hip_device), oc.to(hip_device), os_.to(hip_device), 300, pc, ps)
    rc, rsn = torch.cos(300 * omega.double()), torch.sin(300 * omega.double())
    torch.testing.assert_close(pc.cpu().double(), rc * oc.double() - rsn * os_.double(), rtol=0, atol=1e-6)
    torch.testing.assert_close(ps.cpu().double(), rsn * oc.double() + rc * os_.double(), rtol=0, atol=1e-6)
    # The angle-addition table agrees with direct evaluation within the
    # reference smoke tolerance (tests/run_npu_kernel_smoke.py:136-138).
    direct = torch.cos((offsets.unsqueeze(1) + 300.0) * omega[0]).mean(0)
    torch.testing.assert_close(pc[0].cpu(), direct, rtol=2e-3, atol=2e-3)


SCORE_CASES = [
    # (kv, qpk, head_dim, rotary, style, dtype, tokens)
    (2, 4, 128, 128, "half", torch.bfloat16, 4096),
    (8, 5, 128, 128, "half", torch.bfloat16, 1000),
    (2, 8, 256, 64, "half", torch.bfloat16, 700),
    (8, 5, 128, 128, "half", torch.float16, 333),
    (2, 4, 64, 64, "interleaved", torch.bfloat16, 257),
    (1, 8, 256, 64, "half", torch.bfloat16, 130),
    (4, 1, 128, 128, "half", torch.bfloat16, 129),
    (16, 2, 64, 64, "half", torch.bfloat16, 300),
    # interleaved RoPE on the matrix cores (bf16, fp16, partial rotary)
    (8, 5, 128, 128, "interleaved", torch.bfloat16, 700),
    (8, 5, 128, 128, "interleaved", torch.float16, 513),
    (2, 8, 256, 64, "interleaved", torch.bfloat16, 300),
    # VALU scorer: frequency counts that are not a multiple of 32
    (4, 4, 128, 32, "half", torch.bfloat16, 400),
    (2, 6, 96, 96, "interleaved", torch.float16, 350),
]


FP16_RANGE_CASES = [
    # (key scale, per-query-head weight scales): fp16 keys whose |k| exceeds 65504, tiny
    # weights, and query heads whose weights differ by 10^8 (one scale per head is needed).
    (2.0e4, (1.0, 1.0, 1.0, 1.0, 1.0)),
    (1.0, (1e-6, 1e-6, 1e-6, 1e-6, 1e-6)),
    (1.0, (1e-4, 1.0, 1e4, 3e-3, 250.0)),
    (300.0, (1e3, 1e-3, 1.0, 1.0, 1e-5)),
]


@pytest.mark.parametrize("case", FP16_RANGE_CASES, ids=[f"k{c[0]:g}w{min(c[1]):g}-{max(c[1]):g}" for c in FP16_RANGE_CASES])
def test_score_paged_fp16_ranges(hip_device, case) -> None:
    kernels, _, _ = _kvc()
    key_scale, head_scales = case
    kv, qpk, head_dim, tokens = 8, 5, 128, 700
    g = torch.Generator().manual_seed(len(FP16_RANGE_CASES) + tokens)
    stats = _random_stats(g, kv, qpk, head_dim // 2, 0, head_dim)
    w = torch.tensor(head_scales, dtype=torch.float32).view(1, qpk, 1)
    stats = ref.LayerStats(stats.q_mean_real, stats.q_mean_imag, stats.q_abs_mean, stats.freq_scale_sq * w.square(), stats.omega,
                           stats.rope_style, stats.rotary_dim, stats.q_pass_mean)
    n_blocks = -(-tokens // 128)
    pool = n_blocks + 3
    # Keys up to +-65000 (finite fp16) put |k| up to ~92000, past fp16's largest value.
    cache = (torch.randn(pool, 128, kv, head_dim, generator=g) * key_scale).clamp(-65000.0, 65000.0).to(torch.float16)
    assert torch.isfinite(cache).all()
    blocks = torch.randperm(pool, generator=g)[:n_blocks]
    offsets = ref.build_geometric_offsets(32768)
    round_start = tokens + 5
    keys = ref.gather_paged_range(cache, blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets)
    cos, sin = kernels.mean_phase_table(
        torch.tensor([round_start], dtype=torch.int64, device=hip_device), offsets.to(hip_device), stats.omega.view(1, -1).to(hip_device)
    )
    out = torch.full((kv, qpk, tokens), float("nan"), device=hip_device)
    d = lambda t: None if t is None else t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_mean_precomputed(
        cache.to(hip_device), blocks.to(hip_device), d(stats.q_mean_real), d(stats.q_mean_imag),
        d(torch.sqrt(stats.freq_scale_sq)),
        d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)),
        cos.view(-1), sin.view(-1), tokens, out, 128, "half",
    )
    assert_scores_close(out.cpu().reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))


@pytest.mark.parametrize("case", SCORE_CASES, ids=[f"kv{c[0]}q{c[1]}d{c[2]}r{c[3]}{c[4][0]}{str(c[5]).split('.')[-1]}t{c[6]}" for c in SCORE_CASES])
def test_score_paged_matches_oracle(hip_device, case) -> None:
    kernels, _, _ = _kvc()
    kv, qpk, head_dim, rotary, style, dtype, tokens = case
    g = torch.Generator().manual_seed(sum(case[:4]) + tokens)
    freq = rotary // 2
    stats = _random_stats(g, kv, qpk, freq, head_dim - rotary, rotary, style=style)
    n_blocks = -(-tokens // 128)
    pool = n_blocks + 5
    cache = torch.randn(pool, 128, kv, head_dim, generator=g).to(dtype)
    blocks = torch.randperm(pool, generator=g)[:n_blocks]
    offsets = ref.build_geometric_offsets(32768)
    round_start = tokens + 17
    keys = ref.gather_paged_range(cache, blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets)

    # Direct phase table (torch-path semantics) through the batched entry point.
    cos, sin = kernels.mean_phase_table(
        torch.tensor([round_start], dtype=torch.int64, device=hip_device), offsets.to(hip_device), stats.omega.view(1, -1).to(hip_device)
    )
    out = torch.full((kv, qpk, tokens + 3), float("nan"), device=hip_device)
    d = lambda t: None if t is None else t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_mean_precomputed(
        cache.to(hip_device),
        blocks.to(hip_device),
        d(stats.q_mean_real),
        d(stats.q_mean_imag),
        d(torch.sqrt(stats.freq_scale_sq)),
        d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)),
        cos.view(-1),
        sin.view(-1),
        tokens,
        out,
        128,
        style,
        q_pass_mean=d(stats.q_pass_mean),
        rotary_dim=rotary if rotary != head_dim else None,
    )
    got = out.cpu()
    assert torch.isnan(got[..., tokens:]).all(), "scorer wrote past num_tokens"
    assert_scores_close(got[..., :tokens].reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))


MAX_CASES = [
    # (kv, qpk, head_dim, rotary, style, dtype, tokens, max_model_len -> offsets)
    (8, 5, 128, 128, "half", torch.bfloat16, 1000, 32768),        # 16 offsets, one chunk
    (8, 5, 128, 128, "half", torch.bfloat16, 700, 131072),        # 18: a chunk per head + one tail chunk (two quads)
    (4, 8, 128, 128, "half", torch.bfloat16, 700, 131072),        # 18: two chunks per head, two head groups
    (4, 5, 128, 128, "half", torch.bfloat16, 900, 65536),         # 17: tail rows of one offset, two quads a chunk
    (2, 3, 128, 64, "half", torch.bfloat16, 800, 1 << 23),        # 24: two chunks per head (no tail past 20)
    (2, 1, 128, 128, "half", torch.bfloat16, 400, 1 << 20),       # 21: one query head, two chunks
    (2, 5, 128, 64, "interleaved", torch.bfloat16, 500, 1 << 23),  # 24: two chunks per head, partial RoPE
    (2, 8, 128, 64, "half", torch.bfloat16, 300, 1 << 23),        # 24: two chunks per head, eight heads
    (2, 4, 128, 128, "half", torch.bfloat16, 5000, 32768),        # several spans per workgroup
    (2, 8, 256, 64, "half", torch.bfloat16, 700, 262144),         # partial RoPE, 19 offsets (one quad a tail chunk: two)
    (8, 5, 128, 128, "half", torch.float16, 513, 32768),
    (8, 5, 128, 128, "interleaved", torch.bfloat16, 600, 131072),
    (2, 8, 256, 64, "interleaved", torch.float16, 300, 32768),
    (2, 4, 64, 64, "half", torch.bfloat16, 257, 8),               # 4 offsets
    (1, 8, 256, 256, "half", torch.bfloat16, 130, 65536),         # F = 128: one query head per workgroup
    (8, 5, 128, 128, "half", torch.bfloat16, 600, 1 << 19),       # 20: one quad a tail chunk, two tail chunks
    (2, 8, 128, 64, "half", torch.bfloat16, 500, 65536),          # 17: two full quads share one tail chunk
    (2, 3, 128, 128, "half", torch.bfloat16, 450, 65536),         # 17: one partly filled quad
    (2, 1, 128, 128, "half", torch.bfloat16, 333, 65536),         # 17: one query head, three empty quad slots
    (2, 7, 128, 64, "half", torch.bfloat16, 610, 262144),         # 19: second tail chunk holds a 3-head quad
    (4, 4, 128, 64, "interleaved", torch.bfloat16, 700, 32768),   # 16: one tile per pass, partial RoPE
    # vector-ALU path: F not a multiple of 32 or head_dim not 64/128/256
    (4, 4, 128, 32, "half", torch.bfloat16, 400, 32768),          # F = 16, partial RoPE
    (2, 6, 96, 96, "interleaved", torch.float16, 350, 131072),    # F = 48, 18 offsets
    (2, 2, 80, 80, "half", torch.bfloat16, 300, 16384),           # head_dim 80
    (2, 3, 192, 64, "interleaved", torch.bfloat16, 600, 262144),  # head_dim 192, partial RoPE, 19 offsets
]


@pytest.mark.parametrize("case", MAX_CASES, ids=[f"kv{c[0]}q{c[1]}d{c[2]}r{c[3]}{c[4][0]}{str(c[5]).split('.')[-1]}t{c[6]}o{c[7]}" for c in MAX_CASES])
def test_score_paged_max_matches_oracle(hip_device, case) -> None:
    # score_aggregation="max" (tri/scoring.py:84-97) against the oracle's torch program.
    kernels, _, _ = _kvc()
    kv, qpk, head_dim, rotary, style, dtype, tokens, max_len = case
    g = torch.Generator().manual_seed(sum(case[:4]) + tokens + max_len)
    freq = rotary // 2
    stats = _random_stats(g, kv, qpk, freq, head_dim - rotary, rotary, style=style)
    n_blocks = -(-tokens // 128)
    pool = n_blocks + 5
    cache = torch.randn(pool, 128, kv, head_dim, generator=g).to(dtype)
    blocks = torch.randperm(pool, generator=g)[:n_blocks]
    offsets = ref.build_geometric_offsets(max_len)
    round_start = tokens + 17
    keys = ref.gather_paged_range(cache, blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets, aggregation="max")
    out = torch.full((kv, qpk, tokens + 3), float("nan"), device=hip_device)
    d = lambda t: None if t is None else t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_max(
        cache.to(hip_device), blocks.to(hip_device), d(stats.q_mean_real), d(stats.q_mean_imag),
        d(torch.sqrt(stats.freq_scale_sq)),
        d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)),
        d(stats.omega), d(offsets), round_start, tokens, out, 128, style,
        q_pass_mean=d(stats.q_pass_mean), rotary_dim=rotary if rotary != head_dim else None,
    )
    got = out.cpu()
    assert torch.isnan(got[..., tokens:]).all(), "scorer wrote past num_tokens"
    assert_scores_close(got[..., :tokens].reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))
    # The maximum is not the mean: the two aggregations differ on these inputs.
    mean = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets)
    assert float((want - mean).abs().max()) > 1e-2


@pytest.mark.parametrize("case", FP16_RANGE_CASES, ids=[f"k{c[0]:g}w{min(c[1]):g}-{max(c[1]):g}" for c in FP16_RANGE_CASES])
def test_score_paged_max_fp16_ranges(hip_device, case) -> None:
    # fp16 keys up to +-65000 (|k| past fp16's range) and query heads whose
    # weights differ by 10^8: one power-of-two scale per query head for the
    # per-offset weights, as for the mean scorer.
    kernels, _, _ = _kvc()
    key_scale, head_scales = case
    kv, qpk, head_dim, tokens = 8, 5, 128, 600
    g = torch.Generator().manual_seed(len(FP16_RANGE_CASES) + tokens + 1)
    stats = _random_stats(g, kv, qpk, head_dim // 2, 0, head_dim)
    w = torch.tensor(head_scales, dtype=torch.float32).view(1, qpk, 1)
    stats = ref.LayerStats(stats.q_mean_real, stats.q_mean_imag, stats.q_abs_mean, stats.freq_scale_sq * w.square(), stats.omega,
                           stats.rope_style, stats.rotary_dim, stats.q_pass_mean)
    n_blocks = -(-tokens // 128)
    pool = n_blocks + 3
    cache = (torch.randn(pool, 128, kv, head_dim, generator=g) * key_scale).clamp(-65000.0, 65000.0).to(torch.float16)
    blocks = torch.randperm(pool, generator=g)[:n_blocks]
    offsets = ref.build_geometric_offsets(131072)
    round_start = tokens + 5
    keys = ref.gather_paged_range(cache, blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets, aggregation="max")
    out = torch.full((kv, qpk, tokens), float("nan"), device=hip_device)
    d = lambda t: t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_max(
        d(cache), d(blocks), d(stats.q_mean_real), d(stats.q_mean_imag), d(torch.sqrt(stats.freq_scale_sq)),
        d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)),
        d(stats.omega), d(offsets), round_start, tokens, out, 128, "half",
    )
    assert_scores_close(out.cpu().reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))


def test_score_paged_max_nan_key(hip_device) -> None:
    # A NaN key gives NaN for every offset, so its max-aggregated score is NaN
    # (torch.maximum propagates it); other tokens and KV heads are unaffected.
    kernels, _, _ = _kvc()
    kv, qpk, head_dim, tokens = 2, 4, 128, 300
    g = torch.Generator().manual_seed(99)
    stats = _random_stats(g, kv, qpk, head_dim // 2, 0, head_dim)
    cache = torch.randn(4, 128, kv, head_dim, generator=g).to(torch.bfloat16)
    cache[1, 5, 0, 17] = float("nan")  # token 128 + 5 of KV head 0
    blocks = torch.tensor([0, 1, 2])
    offsets = ref.build_geometric_offsets(32768)
    keys = ref.gather_paged_range(cache, blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=tokens, offsets=offsets, aggregation="max")
    out = torch.empty((kv, qpk, tokens), device=hip_device)
    d = lambda t: t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_max(
        d(cache), d(blocks), d(stats.q_mean_real), d(stats.q_mean_imag), d(torch.sqrt(stats.freq_scale_sq)),
        d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)),
        d(stats.omega), d(offsets), tokens, tokens, out, 128, "half",
    )
    got = out.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert int(torch.isnan(got).sum()) == qpk
    keep = ~torch.isnan(want)
    assert_scores_close(torch.where(keep, got, 0.0).reshape(kv * qpk, tokens), torch.where(keep, want, 0.0).reshape(kv * qpk, tokens))


def test_offset_phase_table_matches_torch(hip_device) -> None:
    from kvcompress_mi355x import _native
    from kvcompress_mi355x.methods.triattention import _device as dev

    offsets = ref.build_geometric_offsets(131072)
    omega = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    omega2 = torch.stack([omega, omega * 0.5]).to(hip_device)
    rs = torch.tensor([300, 131072], dtype=torch.int64, device=hip_device)
    n_off, freq = offsets.numel(), omega.numel()
    cos = torch.empty(2, 2, n_off, freq, device=hip_device)
    sin = torch.empty_like(cos)
    _native.call("kvc_offset_phases", dev.stream_handle(cos.device), 2, 2, freq, dev.ptr(rs), dev.ptr(offsets.to(hip_device)),
                 n_off, dev.ptr(omega2), dev.ptr(cos), dev.ptr(sin))
    for b in range(2):
        for layer in range(2):
            phases = (offsets.unsqueeze(1) + float(rs[b])) * omega2[layer].cpu().unsqueeze(0)
            torch.testing.assert_close(cos[b, layer].cpu(), torch.cos(phases), rtol=0, atol=2e-6)
            torch.testing.assert_close(sin[b, layer].cpu(), torch.sin(phases), rtol=0, atol=2e-6)


def test_reference_smoke_inputs_with_shifted_phases(hip_device) -> None:
    # The reference device smoke (tests/run_npu_kernel_smoke.py:83-138) widened to
    # a 16-dim head: linspace keys and statistics, angle-addition phases at
    # round_start 300, compared with the torch path at rtol = atol = 2e-3.
    kernels, _, _ = _kvc()
    kv, qpk, freq = 2, 2, 8
    cache = torch.linspace(-1.0, 1.0, 3 * 128 * kv * 2 * freq).view(3, 128, kv, 2 * freq).to(torch.bfloat16)
    blocks = torch.tensor([2, 0])
    qr = torch.linspace(0.1, 0.8, kv * qpk * freq).view(kv, qpk, freq)
    qi = torch.linspace(-0.4, 0.3, kv * qpk * freq).view(kv, qpk, freq)
    qa = torch.sqrt(qr.square() + qi.square()) + 0.2
    fscale = torch.linspace(0.8, 1.2, kv * qpk * freq).view(kv, qpk, freq)
    omega = torch.logspace(0, -3, freq)
    offsets = torch.tensor([1.0, 2.0, 4.0])
    extra = qa - torch.sqrt(qr.square() + qi.square() + 1e-8)
    out = torch.empty(kv, qpk, 256, device=hip_device)
    d = lambda t: t.to(hip_device)  # noqa: E731
    assert kernels.score_paged_keys_mean(
        d(cache), d(blocks), d(qr), d(qi), d(fscale), d(extra), d(omega),
        d(torch.cos(offsets.unsqueeze(1) * omega).mean(0)), d(torch.sin(offsets.unsqueeze(1) * omega).mean(0)),
        300, 256, out, 128, "half",
    )
    keys = ref.gather_paged_range(cache, blocks, start=0, count=256, block_size=128)
    want = ref.score_post_rope_keys(keys, ref.LayerStats(qr, qi, qa, fscale.square(), omega), round_start=300, offsets=offsets)
    torch.testing.assert_close(out.cpu(), want, rtol=2e-3, atol=2e-3)


def test_aggregate_single_layer_rsqrt_form(hip_device) -> None:
    kernels, _, _ = _kvc()
    g = torch.Generator().manual_seed(9)
    scores = torch.randn(2, 2, 256, generator=g) * 3 + 1
    var, mean = torch.var_mean(scores, dim=-1, correction=0)
    agg = torch.empty(256, device=hip_device)
    assert kernels.aggregate_normalized_scores(
        scores.to(hip_device), mean.to(hip_device), var.to(hip_device), agg, 256, layer_aggregation="mean", first_layer=True
    )
    want = ((scores - mean.unsqueeze(-1)) * torch.rsqrt(var.unsqueeze(-1) + 1e-6)).amax(dim=(0, 1))
    torch.testing.assert_close(agg.cpu(), want, rtol=2e-3, atol=2e-3)
    second = torch.randn(2, 2, 256, generator=g)
    v2, m2 = torch.var_mean(second, dim=-1, correction=0)
    assert kernels.aggregate_normalized_scores(
        second.to(hip_device), m2.to(hip_device), v2.to(hip_device), agg, 256, layer_aggregation="max", first_layer=False
    )
    want2 = torch.maximum(want, ((second - m2.unsqueeze(-1)) * torch.rsqrt(torch.clamp(v2, min=1e-6).unsqueeze(-1))).amax(dim=(0, 1)))
    torch.testing.assert_close(agg.cpu(), want2, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("layer_mode", ["mean", "max"])
def test_aggregate_row_stride_invariance(hip_device, layer_mode) -> None:
    # kvc_aggregate on head-major scores with ragged, unaligned sequence starts
    # gives the same bits whatever the row stride, NaN and +-inf included.
    from kvcompress_mi355x import _native
    from kvcompress_mi355x.methods.triattention import _device as dev

    g = torch.Generator().manual_seed(21)
    lens = [1, 3, 5, 1000, 4097, 2]
    total = sum(lens)
    layers, heads = 3, 7
    offs = [0]
    for n in lens:
        offs.append(offs[-1] + n)
    base = torch.randn(layers, heads, total, generator=g) * 2
    base[1, 3, 7] = float("nan")
    base[0, 0, 1500] = float("inf")
    base[2, 5, 9] = float("-inf")
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=hip_device)
    tok_off = torch.tensor(offs[:-1], dtype=torch.int64, device=hip_device)
    mean = torch.randn(layers, len(lens), heads, generator=g).to(hip_device)
    var = (torch.rand(layers, len(lens), heads, generator=g) + 0.1).to(hip_device)
    mode = _native.LAYER_MEAN if layer_mode == "mean" else _native.LAYER_MAX
    outs = []
    for row in (total + (-total) % 4 + 64, total + 1 + ((total + 1) % 4 == 0)):
        raw = torch.full((layers, heads, row), float("nan"), device=hip_device)
        raw[:, :, :total] = base.to(hip_device)
        agg = torch.full((total,), 123.0, device=hip_device)
        _native.call(
            "kvc_aggregate", dev.stream_handle(hip_device), layers, heads, len(lens), max(lens), dev.ptr(seq_lens),
            dev.ptr(tok_off), dev.ptr(raw), heads * row, 1, row, dev.ptr(mean), dev.ptr(var), len(lens) * heads, heads,
            mode, _native.AGG_FINALIZE, dev.ptr(agg),
        )
        outs.append(agg.cpu())
    assert outs[0].view(torch.int32).equal(outs[1].view(torch.int32))
    assert not torch.isnan(outs[0]).any() and bool((outs[0] != 123.0).all())


@pytest.mark.parametrize("layer_mode", ["mean", "max"])
def test_aggregate_finalize_non_finite_matches_oracle(hip_device, layer_mode) -> None:
    # Normalise, head max, layer mean/max and nan_to_num(nan=-inf, posinf=1e30)
    # (tri/method.py:423-467) against the oracle's torch program, per sequence of
    # a ragged batch, with NaN and +-inf planted in the raw scores.
    from kvcompress_mi355x import _native
    from kvcompress_mi355x.methods.triattention import _device as dev

    g = torch.Generator().manual_seed(33)
    lens = [700, 45, 1301]
    total, layers, heads = sum(lens), 3, 6
    offs = [0, lens[0], lens[0] + lens[1]]
    raw = torch.randn(layers, heads, total, generator=g) * 2 + 0.5
    raw[1, 3, 7] = float("nan")                    # NaN head score -> NaN layer -> -inf
    raw[0, 0, 500] = float("inf")                  # +inf -> 1e30
    raw[2, 5, 9] = float("-inf")                   # one head -inf: the others' maximum
    raw[0, :, 20] = float("-inf")                  # every head -inf: -inf
    raw[0, 2, 730] = float("inf")                  # +inf in layer 0 ...
    raw[1, :, 730] = float("-inf")                 # ... -inf in layer 1: NaN (mean) / +inf (max)
    raw[2, 4, 800] = float("nan")
    mean = torch.randn(layers, len(lens), heads, generator=g)
    var = torch.rand(layers, len(lens), heads, generator=g) + 0.1
    cfg = ref.MethodConfig(budget=1, recent=0, prefix=0, segments=1, policy="global", layer_aggregation=layer_mode)
    want = []
    for b, n in enumerate(lens):
        part = raw[:, :, offs[b] : offs[b] + n].reshape(layers, 2, 3, n)  # [kv, qpk, tokens] per layer
        stats = [(var[l, b].view(2, 3), mean[l, b].view(2, 3)) for l in range(layers)]
        want.append(ref.aggregate_layers(list(part), stats, cfg))
    want = torch.cat(want)
    assert int(torch.isneginf(want).sum()) >= 2 and int((want == 1e30).sum()) >= 1
    d = hip_device
    agg = torch.full((total,), 123.0, device=d)
    raw_d, mean_d, var_d = raw.to(d), mean.to(d), var.to(d)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=d)
    tok_off = torch.tensor(offs, dtype=torch.int64, device=d)
    _native.call(
        "kvc_aggregate", dev.stream_handle(d), layers, heads, len(lens), max(lens), dev.ptr(seq_lens), dev.ptr(tok_off),
        dev.ptr(raw_d), heads * total, 1, total, dev.ptr(mean_d), dev.ptr(var_d), len(lens) * heads, heads,
        _native.LAYER_MEAN if layer_mode == "mean" else _native.LAYER_MAX, _native.AGG_FINALIZE, dev.ptr(agg),
    )
    got = agg.cpu()
    finite = torch.isfinite(want) & (want != 1e30)
    assert torch.equal(torch.isneginf(got), torch.isneginf(want)), "-inf positions differ"
    assert torch.equal(got[want == 1e30], want[want == 1e30]), "+inf must finalise to 1e30"
    assert not torch.isnan(got).any()
    torch.testing.assert_close(got[finite], want[finite], rtol=1e-3, atol=1e-3)


# ----------------------------------------------------------------- select --


def test_select_reference_kats(hip_device) -> None:
    _, selection, _ = _kvc()
    keep = selection.select_keep_indices(
        torch.tensor([10.0, 9.0, 8.0, 7.0, -5.0, -6.0], device=hip_device),
        budget=4, protected_prefix=0, protected_recent=2, segments=8, policy="global",
    )
    assert keep.cpu().tolist() == [0, 1, 4, 5]
    keep = selection.select_keep_indices(
        torch.arange(16, dtype=torch.float32, device=hip_device), budget=12, protected_prefix=2, protected_recent=2, segments=4, policy="v3"
    )
    assert set(range(16)) - set(keep.cpu().tolist()) == {2, 5, 8, 11}
    keep = selection.select_keep_indices(torch.zeros(19, device=hip_device), budget=13, protected_prefix=2, protected_recent=2, segments=8, policy="v3")
    assert keep.numel() == 13 and {0, 1, 17, 18} <= set(keep.cpu().tolist())


SELECT_CASES = [
    # (n, budget, prefix, recent, segments, policy, ties)
    (4096, 2048, 0, 128, 8, "global", False),
    (16384, 4096, 0, 128, 8, "global", False),
    (36001, 4608, 128, 512, 8, "v3", False),
    (5000, 4608, 128, 512, 8, "v3", True),
    (3000, 1000, 7, 33, 3, "global", True),
    (131072, 4608, 0, 256, 8, "global", False),
    (1000, 1000, 0, 128, 8, "global", False),
    (300, 128, 0, 0, 8, "v3", True),
    (19, 13, 2, 2, 8, "v3", False),
    # The single-workgroup selector keeps a segment's 16-byte words in
    # registers up to 4096 words (16384 scores); around that edge, with an
    # aligned start (prefix 0) and a start three scores past a 16-byte
    # boundary (prefix 3: one head scalar before the first word).
    (16512, 4096, 0, 128, 8, "global", False),  # exactly 4096 words
    (16513, 4096, 0, 128, 8, "global", True),   # 4096 words + 1 tail scalar
    (16515, 4096, 0, 128, 8, "global", False),  # 4096 words + 3 tail scalars
    (16516, 4096, 0, 128, 8, "global", True),   # 4097 words: the uncached walk
    (16516, 4096, 3, 128, 8, "global", False),  # head scalar + 4096 words
    (16519, 4096, 3, 128, 8, "global", True),   # head + 4096 words + 3 tail scalars
    (16520, 4096, 3, 128, 8, "global", False),  # head + 4097 words: uncached
    (131712, 4608, 128, 512, 8, "v3", True),    # eight v3 segments of exactly 16384 scores
]


@pytest.mark.parametrize("case", SELECT_CASES)
def test_select_matches_stable_brute_force(hip_device, case) -> None:
    _, selection, _ = _kvc()
    n, budget, prefix, recent, segments, policy, ties = case
    g = torch.Generator().manual_seed(n + budget)
    scores = torch.randn(n, generator=g)
    if ties:
        scores = torch.round(scores * 4) / 4  # heavy ties
    keep = selection.select_keep_indices(
        scores.to(hip_device), budget=budget, protected_prefix=prefix, protected_recent=recent, segments=segments, policy=policy
    ).cpu()
    want = brute.select_stable(scores.numpy(), budget, prefix, recent, segments, policy)
    np.testing.assert_array_equal(keep.numpy(), want)
    if not ties:
        oracle = ref.select_keep_indices(
            scores, budget=budget, protected_prefix=prefix, protected_recent=recent, segments=segments, policy=policy
        )
        assert torch.equal(keep, oracle)


def _stable_keep_np(scores: np.ndarray, budget: int, prefix: int, recent: int, segments: int, policy: str) -> np.ndarray:
    """brute.select_stable's rule (higher order key first, then lower index),
    vectorised for long inputs: the same protected windows and v3 quotas."""
    bits = scores.astype(np.float32).view(np.uint32).astype(np.int64)
    keys = np.where(bits & 0x80000000, (~bits) & 0xFFFFFFFF, bits | 0x80000000)
    n = scores.shape[0]
    prefix = min(prefix, n)
    recent = min(recent, n - prefix)
    keep = [np.arange(prefix), np.arange(n - recent, n)]

    def top(lo: int, hi: int, k: int) -> np.ndarray:
        idx = np.arange(lo, hi)
        order = np.lexsort((idx, -keys[lo:hi]))
        return idx[order[:k]]

    mc = n - prefix - recent
    if policy == "global":
        keep.append(top(prefix, n - recent, budget - prefix - recent))
    else:
        evict = n - budget
        for s in range(segments):
            a = prefix + mc * s // segments
            b = prefix + mc * (s + 1) // segments
            if b > a:
                quota = (b - a) - (evict * (b - prefix) // mc - evict * (a - prefix) // mc)
                keep.append(top(a, b, max(quota, 0)))
    return np.sort(np.concatenate(keep)).astype(np.int64)


SPLIT_BATCHES = [
    # (lengths, budget, prefix, recent, segments, policy)
    ((300001, 70000, 4097, 40000, 131072), 4096, 0, 128, 8, "global"),
    ((600003, 300000), 4608, 128, 512, 8, "v3"),
    ((4224, 8191), 4096, 0, 128, 8, "global"),
]


@pytest.mark.parametrize("case", SPLIT_BATCHES, ids=["global-ragged", "v3-long", "global-short"])
@pytest.mark.parametrize("ties", [False, True])
def test_select_split_matches_single_and_brute_force(hip_device, case, ties) -> None:
    _, selection, _ = _kvc()
    lens, budget, prefix, recent, segments, policy = case
    g = torch.Generator().manual_seed(sum(lens) + ties)
    scores = torch.randn(sum(lens), generator=g)
    if ties:
        scores = torch.round(scores * 4) / 4
        specials = torch.randint(0, sum(lens), (64,), generator=g)
        scores[specials[:16]] = float("nan")
        scores[specials[16:32]] = float("inf")
        scores[specials[32:48]] = float("-inf")
        scores[specials[48:]] = -0.0
    offsets = [0]
    for n in lens:
        offsets.append(offsets[-1] + n)
    d_scores = scores.to(hip_device)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=hip_device)
    token_offsets = torch.tensor(offsets, dtype=torch.int64, device=hip_device)
    kw = dict(budget=budget, protected_prefix=prefix, protected_recent=recent, segments=segments, policy=policy)
    single = torch.full((len(lens), budget + 3), -7, dtype=torch.int64, device=hip_device)
    split = torch.full_like(single, -7)
    selection.select_keep_indices_batched(d_scores, seq_lens, token_offsets, list(lens), single, shape="single", **kw)
    ws = selection.select_workspace(len(lens), segments, policy, hip_device)
    ws.fill_(0xAB)  # any contents: the first launch resets the scratch
    for _ in range(2):  # the second call reuses the workspace left by the first
        selection.select_keep_indices_batched(d_scores, seq_lens, token_offsets, list(lens), split, shape="split", workspace=ws, **kw)
    torch.cuda.synchronize()
    assert torch.equal(split, single)
    assert bool((split[:, budget:] == -7).all()), "entries past the budget must stay untouched"
    for b, n in enumerate(lens):
        want = _stable_keep_np(scores[offsets[b] : offsets[b + 1]].numpy(), budget, prefix, recent, segments, policy)
        np.testing.assert_array_equal(split[b, :budget].cpu().numpy(), want)


def test_select_split_rejects_a_small_workspace(hip_device) -> None:
    _, selection, _ = _kvc()
    scores = torch.randn(50000, device=hip_device)
    lens = torch.tensor([50000], dtype=torch.int32, device=hip_device)
    offs = torch.tensor([0, 50000], dtype=torch.int64, device=hip_device)
    keep = torch.empty((1, 4096), dtype=torch.int64, device=hip_device)
    small = torch.empty(64, dtype=torch.uint8, device=hip_device)
    with pytest.raises(ValueError, match="workspace"):
        selection.select_keep_indices_batched(scores, lens, offs, [50000], keep, budget=4096, protected_prefix=0,
                                              protected_recent=128, segments=8, policy="global", shape="split",
                                              workspace=small)


def test_select_special_values(hip_device) -> None:
    _, selection, _ = _kvc()
    scores = torch.tensor([0.0, -0.0, float("nan"), float("inf"), 1.0, 1.0, float("-inf"), -3.0])
    for budget in range(1, 9):
        keep = selection.select_keep_indices(
            scores.to(hip_device), budget=budget, protected_prefix=0, protected_recent=0, segments=1, policy="global"
        ).cpu()
        np.testing.assert_array_equal(keep.numpy(), brute.select_stable(scores.numpy(), budget, 0, 0, 1, "global"))


def test_select_rejects_invalid_arguments(hip_device) -> None:
    _, selection, _ = _kvc()
    s = torch.zeros(10, device=hip_device)
    with pytest.raises(ValueError):
        selection.select_keep_indices(s, budget=11, protected_prefix=0, protected_recent=0, segments=1, policy="global")
    with pytest.raises(ValueError):
        selection.select_keep_indices(s, budget=4, protected_prefix=3, protected_recent=2, segments=1, policy="global")
    with pytest.raises(ValueError):
        selection.select_keep_indices(s.cpu(), budget=4, protected_prefix=0, protected_recent=0, segments=1, policy="global")


# ---------------------------------------------------------------- compact --


def _layers(g, n_layers, pages, kv, dim, dtype):
    ks = [torch.randn(pages, 128, kv, dim, generator=g).to(dtype) for _ in range(n_layers)]
    vs = [torch.randn(pages, 128, kv, dim, generator=g).to(dtype) for _ in range(n_layers)]
    return ks, vs


@pytest.mark.parametrize("path", ["walk", "plan", "plan-interleaved"])
@pytest.mark.parametrize("mode", ["private", "inplace"])
@pytest.mark.parametrize("pattern", ["random", "front", "tail", "strided", "split", "shift"])
def test_compact_bit_exact(hip_device, mode: str, pattern: str, path: str) -> None:
    """Every form (rows resolved per workgroup and every layer walked, or rows
    planned once into the workspace and moved one layer per workgroup, layer
    after layer or with the layers interleaved), after the ordered in-place
    walk where the mode has one, against the reference materialisation."""
    _, _, cache = _kvc()
    from kvcompress_mi355x.methods.triattention import _device as dev

    g = torch.Generator().manual_seed(len(mode) * 7 + len(pattern))
    kv, dim, n_layers, budget = 4, 128, 3, 640
    lens = [2000, 1500, 641]
    src_tables, dst_tables = [], []
    pool = sum(-(-n // 128) for n in lens) + (0 if mode == "inplace" else 5 * len(lens)) + 3
    perm = torch.randperm(pool, generator=g).tolist()
    cur = 0
    for n in lens:
        nb = -(-n // 128)
        src_tables.append(perm[cur : cur + nb])
        cur += nb
    if mode == "private":
        for _ in lens:
            dst_tables.append(perm[cur : cur + 5])
            cur += 5
    keeps = []
    for n in lens:
        if pattern == "random":
            k = torch.sort(torch.randperm(n, generator=g)[:budget]).values
        elif pattern == "front" or (pattern == "split" and n < 2 * budget):
            k = torch.arange(budget)
        elif pattern == "split":
            # In place, the first half reads rows 1, 3, 5, ... below the budget,
            # which the second half (sources at or past the budget) overwrites.
            half = budget // 2
            k = torch.cat([2 * torch.arange(half) + 1, torch.arange(budget, 2 * budget - half)])
        elif pattern == "tail":
            k = torch.arange(n - budget, n)
        elif pattern == "shift":
            # In place, every row but the last is a hazard row reading the row
            # after it, which the next row overwrites: a chain through three
            # walk tiles of 256 rows.
            k = torch.arange(1, budget + 1)
        else:
            k = torch.linspace(0, n - 1, budget).round().long().unique()
            while k.numel() < budget:
                k = torch.unique(torch.cat([k, torch.randint(0, n, (budget,), generator=g)]))[:budget]
            k = torch.sort(k[:budget]).values
        keeps.append(k)
    ks, vs = _layers(g, n_layers, pool, kv, dim, torch.bfloat16)
    ks_d = [k.to(hip_device) for k in ks]
    vs_d = [v.to(hip_device) for v in vs]
    # Oracle: reference materialisation per sequence and layer.
    for b, n in enumerate(lens):
        dst = torch.tensor(dst_tables[b] if mode == "private" else src_tables[b][: -(-budget // 128)])
        ref.method_compress(ks, vs, torch.tensor(src_tables[b]), dst, keeps[b], budget)
    so, si, slen = dev.ragged(src_tables, hip_device)
    do = di = None
    if mode == "private":
        do, di, _ = dev.ragged(dst_tables, hip_device)
    keep = torch.stack(keeps).to(hip_device)
    cache.compact_layers(
        dev.pointer_table(ks_d, hip_device),
        dev.pointer_table(vs_d, hip_device),
        num_pages=pool,
        page_stride=int(ks_d[0].stride(0)),
        row_elems=kv * dim,
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=hip_device),
        src_block_offsets=so,
        src_block_ids=si,
        dst_block_offsets=do,
        dst_block_ids=di,
        keep=keep,
        budget=budget,
        workspace=None
        if path == "walk"
        else torch.full((cache.compact_workspace_bytes(len(lens), budget),), 0xAB, dtype=torch.uint8, device=hip_device),
        layer_order="interleaved" if path == "plan-interleaved" else "layer_major",
    )
    torch.cuda.synchronize()
    for layer in range(n_layers):
        assert torch.equal(ks_d[layer].cpu(), ks[layer]), f"K layer {layer} differs"
        assert torch.equal(vs_d[layer].cpu(), vs[layer]), f"V layer {layer} differs"
    tables, freed = cache.rewrite_block_tables(
        budget=budget, src_block_offsets=so, src_block_ids=si, src_lengths=slen, dst_block_offsets=do, dst_block_ids=di
    )
    for b in range(len(lens)):
        want_table, want_freed = ref.rewrite_block_table(src_tables[b], dst_tables[b] if mode == "private" else None, budget)
        assert tables[b].cpu().tolist() == want_table
        assert freed[b].cpu().tolist() == want_freed


@pytest.mark.parametrize("mode", ["private", "inplace"])
def test_compact_layer_extent_past_32_bit_offsets(hip_device, mode: str) -> None:
    """A layer pool of 16400 pages of 256 KB (4.30 GB each for K and V): the
    layer-major planned copy stores through 32-bit buffer offsets only for
    pools below 4 GiB, so this one takes the global stores.  The sequences'
    pages sit at the end of the pool, half of them past byte 2^32, and every
    row lands bit-exact against the oracle run on those pages alone."""
    _, _, cache = _kvc()
    from kvcompress_mi355x.methods.triattention import _device as dev

    kv, dim, budget = 8, 128, 512
    page_bytes = 128 * kv * dim * 2
    pool = (1 << 32) // page_bytes + 16
    assert pool * page_bytes > (1 << 32)
    g = torch.Generator().manual_seed(11)
    lens = [1000, 700]
    far = list(range(pool - 24, pool))  # pages 16376 .. 16399; 16384 starts at byte 2^32
    order = [far[i] for i in torch.randperm(len(far), generator=g).tolist()]
    src_tables, dst_tables, cur = [], [], 0
    for n in lens:
        nb = -(-n // 128)
        src_tables.append(order[cur : cur + nb])
        cur += nb
    if mode == "private":
        for _ in lens:
            dst_tables.append(order[cur : cur + budget // 128])
            cur += budget // 128
    keeps = [torch.sort(torch.randperm(n, generator=g)[:budget]).values for n in lens]
    used = sorted({p for t in src_tables + dst_tables for p in t})
    # Only the pages the sequences use are filled; the rest is never read.
    k = torch.empty((pool, 128, kv, dim), dtype=torch.bfloat16, device=hip_device)
    v = torch.empty_like(k)
    mini_k = torch.randn(len(used), 128, kv, dim, generator=g).to(torch.bfloat16)
    mini_v = torch.randn(len(used), 128, kv, dim, generator=g).to(torch.bfloat16)
    idx = torch.tensor(used, dtype=torch.int64, device=hip_device)
    k.index_copy_(0, idx, mini_k.to(hip_device))
    v.index_copy_(0, idx, mini_v.to(hip_device))
    # Oracle over the used pages, renumbered 0 .. len(used) - 1.
    remap = {p: i for i, p in enumerate(used)}
    for b in range(len(lens)):
        dst = dst_tables[b] if mode == "private" else src_tables[b][: -(-budget // 128)]
        ref.method_compress([mini_k], [mini_v], torch.tensor([remap[p] for p in src_tables[b]]),
                            torch.tensor([remap[p] for p in dst]), keeps[b], budget)
    so, si, _ = dev.ragged(src_tables, hip_device)
    do = di = None
    if mode == "private":
        do, di, _ = dev.ragged(dst_tables, hip_device)
    cache.compact_layers(
        dev.pointer_table([k], hip_device),
        dev.pointer_table([v], hip_device),
        num_pages=pool,
        page_stride=int(k.stride(0)),
        row_elems=kv * dim,
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=hip_device),
        src_block_offsets=so,
        src_block_ids=si,
        dst_block_offsets=do,
        dst_block_ids=di,
        keep=torch.stack(keeps).to(hip_device),
        budget=budget,
        workspace=torch.empty((cache.compact_workspace_bytes(len(lens), budget),), dtype=torch.uint8, device=hip_device),
        layer_order="layer_major",
    )
    torch.cuda.synchronize()
    assert torch.equal(k.index_select(0, idx).cpu(), mini_k)
    assert torch.equal(v.index_select(0, idx).cpu(), mini_v)
    del k, v
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kv,dim", [(1, 128), (4, 128), (8, 128), (10, 128)], ids=["256B", "1KB", "2KB", "2560B"])
def test_compact_planned_row_widths(hip_device, kv: int, dim: int) -> None:
    """The planned private form (both layer orders) for row widths that give
    1, 2 or 8 rows per 128-thread workgroup and rows split into two column
    slices (2560 B), with an unmapped destination page, bit-exact against the
    walked form and the reference materialisation."""
    _, _, cache = _kvc()
    from kvcompress_mi355x.methods.triattention import _device as dev

    g = torch.Generator().manual_seed(kv * 100 + dim)
    n_layers, budget = 2, 384
    lens = [1000, 700, 385, 900]
    pool = sum(-(-n // 128) for n in lens) + 3 * len(lens) + 2
    perm = torch.randperm(pool, generator=g).tolist()
    cur, src_tables, dst_tables = 0, [], []
    for n in lens:
        src_tables.append(perm[cur : cur + -(-n // 128)])
        cur += -(-n // 128)
    for _ in lens:
        dst_tables.append(perm[cur : cur + 3])
        cur += 3
    dst_tables[2][1] = -1  # an unmapped destination page: its rows move nowhere
    keeps = [torch.sort(torch.randperm(n, generator=g)[:budget]).values for n in lens]
    ks, vs = _layers(g, n_layers, pool, kv, dim, torch.bfloat16)
    results = {}
    paths = ("walk", "plan", "plan-interleaved")
    for path in paths:
        ks_d = [k.to(hip_device) for k in ks]
        vs_d = [v.to(hip_device) for v in vs]
        so, si, _ = dev.ragged(src_tables, hip_device)
        do, di, _ = dev.ragged(dst_tables, hip_device)
        cache.compact_layers(
            dev.pointer_table(ks_d, hip_device),
            dev.pointer_table(vs_d, hip_device),
            num_pages=pool,
            page_stride=int(ks_d[0].stride(0)),
            row_elems=kv * dim,
            seq_lens=torch.tensor(lens, dtype=torch.int32, device=hip_device),
            src_block_offsets=so,
            src_block_ids=si,
            dst_block_offsets=do,
            dst_block_ids=di,
            keep=torch.stack(keeps).to(hip_device),
            budget=budget,
            workspace=None
            if path == "walk"
            else torch.empty(cache.compact_workspace_bytes(len(lens), budget), dtype=torch.uint8, device=hip_device),
            layer_order="interleaved" if path == "plan-interleaved" else "layer_major",
        )
        torch.cuda.synchronize()
        results[path] = ([k.cpu() for k in ks_d], [v.cpu() for v in vs_d])
    for b in range(len(lens)):
        dst = [p for p in dst_tables[b]]
        rows = [i for i in range(budget) if dst[i // 128] >= 0]
        keep_b = keeps[b][rows]
        for layer in range(n_layers):
            for kind, src_cache in ((0, ks), (1, vs)):
                want = ref.gather_paged_tokens(src_cache[layer], torch.tensor(src_tables[b]), keep_b, 128)
                for path in paths:
                    got_cache = results[path][kind][layer].view(-1, kv, dim)
                    slots = torch.tensor([dst[i // 128] * 128 + i % 128 for i in rows])
                    assert torch.equal(got_cache[slots], want), (path, b, layer, kind)
    for kind in range(2):
        for layer in range(n_layers):
            for path in paths[1:]:
                assert torch.equal(results["walk"][kind][layer], results[path][kind][layer])


def _shared_kv_buffers(g, n_layers, pages, kv, dim, dtype, pad, device):
    """Per layer one buffer [pages][K page | V page | pad elements], the
    padding filled with NaN; returns (buffers, K views, V views)."""
    page = 128 * kv * dim
    stride = 2 * page + pad
    shape, strides = (pages, 128, kv, dim), (stride, kv * dim, dim, 1)
    bufs, ks, vs = [], [], []
    for _ in range(n_layers):
        buf = torch.full((pages * stride,), float("nan"), dtype=dtype)
        k = torch.as_strided(buf, shape, strides, 0)
        v = torch.as_strided(buf, shape, strides, page)
        k.copy_(torch.randn(shape, generator=g))
        v.copy_(torch.randn(shape, generator=g))
        buf = buf.to(device)
        bufs.append(buf)
        ks.append(torch.as_strided(buf, shape, strides, 0))
        vs.append(torch.as_strided(buf, shape, strides, page))
    return bufs, ks, vs


def _padding_bits(buf, pages, kv, dim, pad):
    page = 128 * kv * dim
    return buf.view(pages, 2 * page + pad)[:, 2 * page :].cpu().view(torch.int16)


@pytest.mark.parametrize("path", ["walk", "plan", "plan-interleaved"])
@pytest.mark.parametrize("mode", ["private", "inplace"])
@pytest.mark.parametrize("pad", [0, 8, 4], ids=["pad0", "pad8", "pad4-8B-words"])
def test_compact_shared_kv_buffer(hip_device, mode: str, path: str, pad: int) -> None:
    """Every compaction form on K and V as interleaved views of one buffer per
    layer with padded pages (tests/test_cache.py:50-94 at 128-token blocks;
    pkg/provider.py:1201-1230): rows bit-exact against the reference's
    materialisation and every padding element untouched.  Padding of 4
    elements (the reference KAT's) moves the rows in 8-byte words."""
    _, _, cache = _kvc()
    from kvcompress_mi355x.methods.triattention import _device as dev

    g = torch.Generator().manual_seed(pad * 13 + len(mode) + len(path))
    kv, dim, n_layers, budget = 4, 128, 3, 640
    lens = [2000, 1500, 641]
    pool = sum(-(-n // 128) for n in lens) + (0 if mode == "inplace" else 5 * len(lens)) + 3
    perm = torch.randperm(pool, generator=g).tolist()
    cur, src_tables, dst_tables = 0, [], []
    for n in lens:
        src_tables.append(perm[cur : cur + -(-n // 128)])
        cur += -(-n // 128)
    if mode == "private":
        for _ in lens:
            dst_tables.append(perm[cur : cur + 5])
            cur += 5
    keeps = [torch.sort(torch.randperm(n, generator=g)[:budget]).values for n in lens]
    if mode == "inplace":
        # One sequence whose hazard rows read rows the safe rows overwrite.
        half = budget // 2
        keeps[0] = torch.cat([2 * torch.arange(half) + 1, torch.arange(budget, 2 * budget - half)])
    bufs, ks_d, vs_d = _shared_kv_buffers(g, n_layers, pool, kv, dim, torch.bfloat16, pad, hip_device)
    ks = [k.cpu() for k in ks_d]
    vs = [v.cpu() for v in vs_d]
    pad_before = [_padding_bits(b, pool, kv, dim, pad) for b in bufs] if pad else None
    for b, n in enumerate(lens):
        dst = torch.tensor(dst_tables[b] if mode == "private" else src_tables[b][: -(-budget // 128)])
        ref.method_compress(ks, vs, torch.tensor(src_tables[b]), dst, keeps[b], budget)
    so, si, _ = dev.ragged(src_tables, hip_device)
    do = di = None
    if mode == "private":
        do, di, _ = dev.ragged(dst_tables, hip_device)
    cache.compact_layers(
        dev.pointer_table(ks_d, hip_device),
        dev.pointer_table(vs_d, hip_device),
        num_pages=pool,
        page_stride=int(ks_d[0].stride(0)),
        row_elems=kv * dim,
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=hip_device),
        src_block_offsets=so,
        src_block_ids=si,
        dst_block_offsets=do,
        dst_block_ids=di,
        keep=torch.stack(keeps).to(hip_device),
        budget=budget,
        workspace=None
        if path == "walk"
        else torch.empty(cache.compact_workspace_bytes(len(lens), budget), dtype=torch.uint8, device=hip_device),
        layer_order="interleaved" if path == "plan-interleaved" else "layer_major",
    )
    torch.cuda.synchronize()
    for layer in range(n_layers):
        assert torch.equal(ks_d[layer].cpu(), ks[layer]), f"K layer {layer} differs"
        assert torch.equal(vs_d[layer].cpu(), vs[layer]), f"V layer {layer} differs"
        if pad:
            assert torch.equal(_padding_bits(bufs[layer], pool, kv, dim, pad), pad_before[layer]), f"layer {layer} padding written"


SHARED_SCORE_CASES = [
    # (kv, qpk, head_dim, rotary, dtype, tokens, pad, aggregation)
    (8, 5, 128, 128, torch.bfloat16, 1500, 8, "mean"),
    (8, 5, 128, 128, torch.float16, 1300, 64, "mean"),
    (2, 8, 256, 64, torch.bfloat16, 900, 0, "mean"),
    (8, 5, 128, 128, torch.bfloat16, 1100, 8, "max"),
    (2, 8, 256, 64, torch.float16, 700, 16, "max"),
]


@pytest.mark.parametrize("case", SHARED_SCORE_CASES, ids=[f"kv{c[0]}d{c[2]}r{c[3]}{str(c[4]).split('.')[-1]}pad{c[6]}-{c[7]}" for c in SHARED_SCORE_CASES])
def test_score_paged_shared_kv_buffer(hip_device, case) -> None:
    """Both scorers reading K as a view of a shared K/V buffer with padded
    pages (the padding is NaN: a stray read would poison the scores), against
    the oracle."""
    kernels, _, _ = _kvc()
    kv, qpk, head_dim, rotary, dtype, tokens, pad, aggregation = case
    g = torch.Generator().manual_seed(tokens + pad)
    stats = _random_stats(g, kv, qpk, rotary // 2, head_dim - rotary, rotary)
    n_blocks = -(-tokens // 128)
    pool = n_blocks + 4
    _, ks_d, _ = _shared_kv_buffers(g, 1, pool, kv, head_dim, dtype, pad, hip_device)
    k_d = ks_d[0]
    blocks = torch.randperm(pool, generator=g)[:n_blocks]
    max_len = 32768 if aggregation == "mean" else 131072
    offsets = ref.build_geometric_offsets(max_len)
    round_start = tokens + 9
    keys = ref.gather_paged_range(k_d.cpu(), blocks, start=0, count=tokens, block_size=128)
    want = ref.score_post_rope_keys(keys, stats, round_start=round_start, offsets=offsets, aggregation=aggregation)
    out = torch.full((kv, qpk, tokens), float("nan"), device=hip_device)
    d = lambda t: None if t is None else t.to(hip_device)  # noqa: E731
    common = (d(stats.q_mean_real), d(stats.q_mean_imag), d(torch.sqrt(stats.freq_scale_sq)),
              d(stats.q_abs_mean - torch.sqrt(stats.q_mean_real.square() + stats.q_mean_imag.square() + 1e-8)))
    extra = dict(q_pass_mean=d(stats.q_pass_mean), rotary_dim=rotary if rotary != head_dim else None)
    if aggregation == "mean":
        cos, sin = kernels.mean_phase_table(
            torch.tensor([round_start], dtype=torch.int64, device=hip_device), offsets.to(hip_device), stats.omega.view(1, -1).to(hip_device)
        )
        assert kernels.score_paged_keys_mean_precomputed(k_d, blocks.to(hip_device), *common, cos.view(-1), sin.view(-1),
                                                         tokens, out, 128, "half", **extra)
    else:
        assert kernels.score_paged_keys_max(k_d, blocks.to(hip_device), *common, d(stats.omega), d(offsets), round_start,
                                            tokens, out, 128, "half", **extra)
    assert_scores_close(out.cpu().reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))


def test_score_rejects_pages_off_16_byte_boundaries(hip_device) -> None:
    # A page stride padded by 4 bf16 elements puts odd pages 8 bytes off a
    # 16-byte boundary: the scorers refuse it (the compaction moves such rows
    # in 8-byte words, test_compact_shared_kv_buffer).
    kernels, _, _ = _kvc()
    g = torch.Generator().manual_seed(5)
    stats = _random_stats(g, 2, 4, 64, 0, 128)
    _, ks_d, _ = _shared_kv_buffers(g, 1, 4, 2, 128, torch.bfloat16, 4, hip_device)
    out = torch.empty((2, 4, 256), device=hip_device)
    d = lambda t: t.to(hip_device)  # noqa: E731
    cos = torch.zeros(64, device=hip_device)
    with pytest.raises(ValueError, match="16 bytes"):
        kernels.score_paged_keys_mean_precomputed(
            ks_d[0], torch.arange(2, device=hip_device), d(stats.q_mean_real), d(stats.q_mean_imag),
            d(torch.sqrt(stats.freq_scale_sq)), d(stats.q_abs_mean), cos, cos, 256, out, 128, "half",
        )


def test_materialize_token_slots_padded_pages(hip_device) -> None:
    # tests/test_cache.py:50-94 with 128-token blocks: K and V interleaved in one
    # padded buffer; the padding must stay untouched.
    _, _, cache = _kvc()
    bs, pages, heads, dim = 128, 4, 1, 8
    logical = bs * heads * dim
    stride = 2 * logical + 4
    raw = torch.full((pages * stride,), -1, dtype=torch.float16, device=hip_device)
    shape, strides = (pages, bs, heads, dim), (stride, heads * dim, dim, 1)
    k = torch.as_strided(raw, shape, strides)
    v = torch.as_strided(raw, shape, strides, storage_offset=logical)
    k.copy_(torch.arange(pages * logical, device=hip_device).view(shape))
    v.copy_((torch.arange(pages * logical, device=hip_device) % 1000 + 100).view(shape))
    src = torch.tensor([2, 0, 3], device=hip_device)
    keep = torch.sort(torch.randperm(384, generator=torch.Generator().manual_seed(3))[:128]).values.to(hip_device)
    kh, vh = k.cpu(), v.cpu()
    want_k = ref.gather_paged_tokens(kh, src.cpu(), keep.cpu(), bs)
    want_v = ref.gather_paged_tokens(vh, src.cpu(), keep.cpu(), bs)
    cache.materialize_selected_tokens(k, v, src, torch.tensor([2], device=hip_device), keep, bs)
    torch.cuda.synchronize()
    assert torch.equal(k[2].cpu(), want_k) and torch.equal(v[2].cpu(), want_v)
    assert torch.equal(raw.view(pages, stride)[:, -4:].cpu(), torch.full((pages, 4), -1, dtype=torch.float16))


def test_token_slots_and_expand(hip_device) -> None:
    _, _, cache = _kvc()
    blocks = torch.tensor([2, 0], device=hip_device)
    got = cache.token_slots(blocks, torch.tensor([0, 3, 4, 7, 130, 255], device=hip_device), 128)
    assert got.cpu().tolist() == [256, 259, 260, 263, 2, 127]
    ids = torch.tensor([3, 1], device=hip_device)
    assert cache.expand_scheduler_block_ids(ids, 16).cpu().tolist() == [48 + j for j in range(16)] + [16 + j for j in range(16)]
    assert cache.expand_scheduler_block_ids(ids, 1).cpu().tolist() == [3, 1]


# ------------------------------------------------- decode after compaction --


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_shift_positions_matches_oracle(hip_device, index_dtype) -> None:
    kernels, _, _ = _kvc()
    # Reference smoke case (tests/run_npu_kernel_smoke.py:29-36).
    pos = torch.tensor([300, 20, 301], dtype=torch.int64)
    idx = torch.tensor([0, 1, 0], dtype=index_dtype)
    off = torch.tensor([172, 0], dtype=torch.int64)
    out = torch.empty(3, dtype=torch.int64, device=hip_device)
    kernels.shift_positions(pos.to(hip_device), idx.to(hip_device), off.to(hip_device), out)
    assert out.cpu().tolist() == [128, 20, 129]
    # A batch of 256 requests, one decode token each plus chunked prefills.
    g = torch.Generator().manual_seed(11)
    n_req = 256
    off = torch.randint(0, 30000, (n_req,), generator=g, dtype=torch.int64)
    idx = torch.randint(0, n_req, (5000,), generator=g).to(index_dtype)
    pos = off[idx.long()] + torch.randint(0, 4096, (5000,), generator=g, dtype=torch.int64)
    out = torch.empty(5000, dtype=torch.int64, device=hip_device)
    kernels.shift_positions(pos.to(hip_device), idx.to(hip_device), off.to(hip_device), out)
    assert torch.equal(out.cpu(), ref.shift_positions(pos, idx, off))


@pytest.mark.parametrize("with_offsets", [True, False])
def test_physical_slot_mapping_matches_brute_force(hip_device, with_offsets: bool) -> None:
    kernels, _, _ = _kvc()
    g = torch.Generator().manual_seed(12)
    n_req, max_blocks, bs = 64, 48, 128
    q_lens = torch.randint(0, 40, (n_req,), generator=g)
    q_lens[::3] = 1  # decode rows
    qsl = torch.zeros(n_req + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(q_lens, 0).to(torch.int32)
    n_real = int(qsl[-1])
    num_tokens = n_real + 9  # graph padding after the last request
    table = torch.randint(0, 5000, (n_req, max_blocks), generator=g, dtype=torch.int32)
    table[:, 40:] = -1
    offsets = torch.randint(0, 3000, (n_req,), generator=g, dtype=torch.int64) if with_offsets else None
    positions = torch.empty(num_tokens, dtype=torch.int64)
    for r in range(n_req):
        start = int(torch.randint(0, 6000, (1,), generator=g))
        base = (int(offsets[r]) if offsets is not None else 0) + start
        positions[int(qsl[r]) : int(qsl[r + 1])] = torch.arange(base, base + int(q_lens[r]))
    positions[n_real:] = torch.arange(9)
    positions[0] = -5 if not with_offsets else positions[0]  # below zero -> -1
    slots = torch.empty(num_tokens, dtype=torch.int64, device=hip_device)
    phys = torch.empty(num_tokens, dtype=torch.int64, device=hip_device)
    kernels.compute_physical_slot_mapping(
        qsl.to(hip_device),
        positions.to(hip_device),
        None if offsets is None else offsets.to(hip_device),
        table.to(hip_device),
        bs,
        slots,
        phys,
    )
    want_slots, want_phys = brute.slot_mapping(
        qsl.tolist(), positions.tolist(), None if offsets is None else offsets.tolist(), table.tolist(), bs, num_tokens
    )
    assert slots.cpu().tolist() == want_slots
    assert phys.cpu().tolist() == want_phys
    assert -1 in want_slots  # padding and out-of-table cases were exercised


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_shift_seq_lens_matches_oracle(hip_device, dtype) -> None:
    kernels, _, _ = _kvc()
    lens = torch.tensor([301, 21, 50], dtype=dtype)
    off = torch.tensor([172, 0, 7], dtype=torch.int64)
    dev_lens = lens.to(hip_device)
    kernels.shift_seq_lens(dev_lens, off.to(hip_device), 2)
    assert dev_lens.cpu().tolist() == ref.physical_seq_lens(lens, off, 2).tolist() == [129, 21, 50]


@pytest.mark.parametrize("aggregation", ["mean", "max"])
@pytest.mark.parametrize(
    ("kv", "qpk", "head_dim", "rotary", "style", "tokens"),
    [(2, 4, 128, 128, "half", 1000), (2, 8, 256, 64, "interleaved", 300), (2, 3, 96, 96, "half", 77)],
)
def test_score_post_rope_keys_matches_oracle(hip_device, aggregation, kv, qpk, head_dim, rotary, style, tokens) -> None:
    # The reference's dense-key scoring function (tri/scoring.py:23-120) under
    # its own name, on the HIP scorers.
    from kvcompress_mi355x.methods.triattention import scoring
    from kvcompress_mi355x.methods.triattention.stats import DeviceLayerCalibrationStats

    g = torch.Generator().manual_seed(kv * 100 + head_dim + tokens)
    stats = _random_stats(g, kv, qpk, rotary // 2, head_dim - rotary, rotary, style=style)
    keys = torch.randn(tokens, kv, head_dim, generator=g).to(torch.bfloat16)
    offsets = ref.build_geometric_offsets(65536)
    want = ref.score_post_rope_keys(keys, stats, round_start=tokens + 9, offsets=offsets, aggregation=aggregation)
    d = lambda t: None if t is None else t.to(hip_device)  # noqa: E731
    dstats = DeviceLayerCalibrationStats(
        d(stats.q_mean_real), d(stats.q_mean_imag), d(stats.q_abs_mean), d(stats.freq_scale_sq), d(stats.omega),
        style, None if rotary == head_dim else rotary, d(stats.q_pass_mean),
    )
    got = scoring.score_post_rope_keys(d(keys), dstats, round_start=tokens + 9, offsets=d(offsets), aggregation=aggregation)
    assert got.shape == want.shape
    assert_scores_close(got.cpu().reshape(kv * qpk, tokens), want.reshape(kv * qpk, tokens))
    with pytest.raises(ValueError, match="unsupported score aggregation"):
        scoring.score_post_rope_keys(d(keys), dstats, round_start=1, offsets=d(offsets), aggregation="median")


def test_gather_paged_range_matches_oracle(hip_device) -> None:
    from kvcompress_mi355x.methods.triattention import cache as kcache

    g = torch.Generator().manual_seed(8)
    pool = torch.randn(6, 128, 2, 64, generator=g).to(torch.bfloat16)
    blocks = torch.tensor([4, 1, 5])
    want = ref.gather_paged_range(pool, blocks, start=100, count=200, block_size=128)
    got = kcache.gather_paged_range(pool.to(hip_device), blocks.to(hip_device), start=100, count=200, block_size=128)
    assert torch.equal(got.cpu(), want)
    # Padded pages (page stride past the page's elements), as the reference's
    # interleaved K/V storage has (tests/test_cache.py:50-94).
    padded = torch.zeros(6, 2, 128, 2, 64, dtype=torch.bfloat16)
    padded[:, 0] = pool
    k_view = padded.to(hip_device)[:, 0]
    got = kcache.gather_paged_range(k_view, blocks.to(hip_device), start=0, count=384, block_size=128)
    assert torch.equal(got.cpu(), ref.gather_paged_range(pool, blocks, start=0, count=384, block_size=128))
