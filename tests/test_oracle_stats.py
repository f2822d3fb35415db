"""Pin the oracle's calibration -> device layout (oracle.stats_ref) and check the
product's CalibrationStats.to_device against it; load the reference's real
calibration artifacts through the product loader.

Pins of the oracle, each independent of its code:
  - the reference's known-answer cases (tests/test_stats.py:38-316: KV-averaged
    rows expanded across the GQA group, freq_scale_sq 4.0 kept, Qwen3.5 partial
    RoPE shapes, KV-head tensor-parallel shards that differ);
  - closed-form index maps: row value 1000*h + w must land at [kv, g, w] with
    h = kv*qpk + g (consecutive query heads per KV head; a strided grouping
    h = g*H_kv + kv fails), and shard r of a TP group holds KV heads
    r*local .. r*local + local - 1;
  - omega = 1/theta^(2i/R) against float64 math, and the precedence layer
    inv_freq > metadata layer_inv_freqs > metadata inv_freq > theta default
    (tri/stats.py:325-331,466-488).
"""

from __future__ import annotations

import math
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from kvcompress_mi355x.methods.base import ModelShape
from kvcompress_mi355x.methods.triattention.stats import CalibrationStats, LayerCalibrationStats
from oracle import stats_ref


def _oracle(cal: CalibrationStats, model: ModelShape, rank: int = 0, size: int = 1):
    return stats_ref.layer_stats_for_device(
        cal.layers,
        cal.metadata,
        num_attention_heads=model.num_attention_heads,
        num_kv_heads=model.num_kv_heads,
        head_dim=model.head_dim,
        rotary_dim=model.effective_rotary_dim,
        rope_theta=model.rope_theta,
        tensor_parallel_rank=rank,
        tensor_parallel_size=size,
    )


def _model(n_q=4, n_kv=2, head_dim=8, rotary=None, theta=10000.0, layers=1, indices=None, model_type="qwen3"):
    return ModelShape(
        model_type=model_type,
        num_layers=layers,
        num_attention_heads=n_q,
        num_kv_heads=n_kv,
        head_dim=head_dim,
        rope_theta=theta,
        has_rope_scaling=False,
        rotary_dim=rotary,
        attention_layer_indices=indices,
    )


def _indexed(rows: int, width: int) -> torch.Tensor:
    return torch.tensor([[1000.0 * h + w for w in range(width)] for h in range(rows)])


def test_reference_kat_kv_rows_expand_across_the_group():
    # tests/test_stats.py:138-167
    layer = SimpleNamespace(
        q_mean_real=torch.tensor([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]]),
        q_mean_imag=torch.zeros(2, 4),
        q_abs_mean=torch.ones(2, 4),
        freq_scale_sq=torch.full((2, 4), 4.0),
        inv_freq=None,
        q_pass_mean=None,
    )
    got = stats_ref.layer_stats_for_device(
        {0: layer}, {}, num_attention_heads=4, num_kv_heads=2, head_dim=8, rotary_dim=8, rope_theta=10000.0
    )[0]
    assert got.q_mean_real.shape == (2, 2, 4)
    assert torch.equal(got.q_mean_real[0, 0], got.q_mean_real[0, 1])
    assert torch.equal(got.q_mean_real[1, 0], torch.tensor([5.0, 6.0, 7.0, 8.0]))
    assert torch.equal(got.freq_scale_sq, torch.full((2, 2, 4), 4.0))
    assert got.omega.shape == (4,)


def test_closed_form_grouping_of_query_head_rows():
    n_q, n_kv, width = 40, 8, 64
    layer = SimpleNamespace(
        q_mean_real=_indexed(n_q, width),
        q_mean_imag=-_indexed(n_q, width),
        q_abs_mean=_indexed(n_q, width) + 0.5,
        freq_scale_sq=None,
        inv_freq=None,
        q_pass_mean=None,
    )
    got = stats_ref.layer_stats_for_device(
        {5: layer}, {}, num_attention_heads=n_q, num_kv_heads=n_kv, head_dim=128, rotary_dim=128, rope_theta=1e6
    )[5]
    qpk = n_q // n_kv
    for kv in range(n_kv):
        for g in range(qpk):
            h = kv * qpk + g
            assert got.q_mean_real[kv, g, 7].item() == 1000.0 * h + 7
            assert got.q_mean_imag[kv, g, 63].item() == -(1000.0 * h + 63)
            assert got.q_abs_mean[kv, g, 0].item() == 1000.0 * h + 0.5
    assert torch.equal(got.freq_scale_sq, torch.ones(n_kv, qpk, width))


def test_closed_form_tensor_parallel_shards():
    # tests/test_stats.py:282-316 (Qwen3.5, two ranks) plus the exact rows each rank holds.
    n_q, n_kv, freq, pass_dim = 16, 2, 32, 192
    layer = SimpleNamespace(
        q_mean_real=_indexed(n_q, freq),
        q_mean_imag=torch.zeros(n_q, freq),
        q_abs_mean=torch.ones(n_q, freq),
        freq_scale_sq=None,
        inv_freq=None,
        q_pass_mean=_indexed(n_q, pass_dim),
    )
    shards = [
        stats_ref.layer_stats_for_device(
            {3: layer}, {"rope_style": "half"}, num_attention_heads=n_q, num_kv_heads=n_kv, head_dim=256,
            rotary_dim=64, rope_theta=1e7, tensor_parallel_rank=r, tensor_parallel_size=2,
        )[3]
        for r in range(2)
    ]
    for r, s in enumerate(shards):
        assert s.q_mean_real.shape == (1, 8, 32)
        assert s.q_pass_mean.shape == (1, 8, 192)
        for g in range(8):
            assert s.q_mean_real[0, g, 31].item() == 1000.0 * (r * 8 + g) + 31
            assert s.q_pass_mean[0, g, 191].item() == 1000.0 * (r * 8 + g) + 191
    assert not torch.equal(shards[0].q_mean_real, shards[1].q_mean_real)
    with pytest.raises(ValueError):
        stats_ref.layer_stats_for_device({3: layer}, {}, num_attention_heads=16, num_kv_heads=2, head_dim=256,
                                         rotary_dim=64, rope_theta=1e7, tensor_parallel_rank=0, tensor_parallel_size=4)


def test_omega_default_and_precedence():
    rotary, theta = 128, 1e6
    omega = stats_ref.default_omega(rotary, theta)
    want = torch.tensor([1.0 / math.pow(theta, 2 * i / rotary) for i in range(rotary // 2)], dtype=torch.float64)
    torch.testing.assert_close(omega.double(), want, rtol=1e-6, atol=0.0)

    def layer(inv):
        return SimpleNamespace(q_mean_real=torch.ones(2, 4), q_mean_imag=torch.zeros(2, 4), q_abs_mean=torch.ones(2, 4),
                               freq_scale_sq=torch.ones(1, 4), inv_freq=inv, q_pass_mean=None)

    kw = dict(num_attention_heads=2, num_kv_heads=1, head_dim=8, rotary_dim=8, rope_theta=10000.0)
    own = torch.tensor([4.0, 3.0, 2.0, 1.0])
    md = {"layer_inv_freqs": {"1": [9.0, 8.0, 7.0, 6.0]}, "inv_freq": [0.5, 0.25, 0.125, 0.0625]}
    got = stats_ref.layer_stats_for_device({0: layer(own), 1: layer(None), 2: layer(None)}, md, **kw)
    assert got[0].omega.tolist() == [4.0, 3.0, 2.0, 1.0]
    assert got[1].omega.tolist() == [9.0, 8.0, 7.0, 6.0]  # str-keyed per-layer entry
    assert got[2].omega.tolist() == [0.5, 0.25, 0.125, 0.0625]
    got = stats_ref.layer_stats_for_device({0: layer(None)}, {}, **kw)
    torch.testing.assert_close(got[0].omega.double(), torch.tensor([1.0 / 10000.0 ** (i / 8) for i in (0, 2, 4, 6)], dtype=torch.float64), rtol=1e-6, atol=0.0)
    # A [1, F] frequency scale is shared by every query head.
    scaled = layer(own)
    scaled.freq_scale_sq = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    got = stats_ref.layer_stats_for_device({0: scaled}, {}, **kw)
    assert got[0].freq_scale_sq.tolist() == [[[1.0, 2.0, 3.0, 4.0], [1.0, 2.0, 3.0, 4.0]]]


def _random_calibration(model: ModelShape, *, kv_rows: bool, scale_rows: int | None, seed: int) -> CalibrationStats:
    g = torch.Generator().manual_seed(seed)
    rows = model.num_kv_heads if kv_rows else model.num_attention_heads
    freq = model.effective_rotary_dim // 2
    pass_dim = model.head_dim - model.effective_rotary_dim
    layers = {}
    for index in model.full_attention_layer_indices:
        layers[index] = LayerCalibrationStats(
            q_mean_real=torch.randn(rows, freq, generator=g),
            q_mean_imag=torch.randn(rows, freq, generator=g),
            q_abs_mean=torch.rand(rows, freq, generator=g) + 1.0,
            freq_scale_sq=None if scale_rows is None else torch.rand(scale_rows, freq, generator=g) + 0.5,
            q_pass_mean=torch.randn(rows, pass_dim, generator=g) if pass_dim else None,
        )
    return CalibrationStats(metadata={"rope_style": "half"}, layers=layers)


@pytest.mark.parametrize(
    "model,kv_rows,scale_rows,size",
    [
        (_model(40, 8, 128, None, 1e6, 4), False, None, 1),
        (_model(40, 8, 128, None, 1e6, 4), True, 1, 2),
        (_model(16, 2, 256, 64, 1e7, 8, (3, 7), "qwen3_5_moe_text"), False, 16, 2),
        (_model(8, 2, 128, None, 1e6, 1), True, 2, 1),
    ],
    ids=["qwen2.5-q-rows", "kv-rows-tp2", "qwen3.5-partial-tp2", "tiny-kv-scale"],
)
def test_product_to_device_matches_oracle(model, kv_rows, scale_rows, size):
    cal = _random_calibration(model, kv_rows=kv_rows, scale_rows=scale_rows, seed=7)
    for rank in range(size):
        got = cal.to_device(model, torch.device("cpu"), tensor_parallel_rank=rank, tensor_parallel_size=size)
        want = _oracle(cal, model, rank, size)
        assert set(got) == set(want)
        for index in want:
            a, b = got[index], want[index]
            for name in ("q_mean_real", "q_mean_imag", "q_abs_mean", "freq_scale_sq", "omega"):
                assert torch.equal(getattr(a, name), getattr(b, name)), (index, name)
            assert (a.q_pass_mean is None) == (b.q_pass_mean is None)
            if b.q_pass_mean is not None:
                assert torch.equal(a.q_pass_mean, b.q_pass_mean)
            assert a.rotary_dim == b.rotary_dim and a.rope_style == b.rope_style


ARTIFACTS = Path("/root/reference/artifacts")
QWEN25 = _model(40, 8, 128, None, 1e6, 48, None, "qwen2")
QWEN35 = _model(16, 2, 256, 64, 1e7, 40, tuple(range(3, 40, 4)), "qwen3_5_moe_text")


@pytest.mark.parametrize(
    "name,model,schema",
    [
        ("qwen2.5-14b-instruct-stats-v3.pt", QWEN25, "layer_stats"),
        ("qwen2.5-coder-14b-stats.pt", QWEN25, "stats"),
        ("qwen2.5-coder-14b-stats-smoke.pt", QWEN25, "stats"),
        ("qwen3.5-35b-a3b-stats-v3.pt", QWEN35, "layer_stats"),
    ],
)
def test_reference_artifacts_load_and_lay_out(name, model, schema):
    """The reference's shipped calibration artifacts (schema-3 layer_stats and
    legacy flat layerLL_headHH) read weights-only in place, validated against
    the model they were made for, and laid out as the oracle lays them out."""
    path = ARTIFACTS / name
    if not path.is_file():
        pytest.skip("reference artifacts are not present on this host")
    payload = torch.load(path, map_location="cpu", weights_only=True)
    assert schema in payload
    cal = CalibrationStats.load(path)
    assert sorted(cal.layers) == list(model.full_attention_layer_indices)
    assert cal.validate(model) == ()
    freq = model.effective_rotary_dim // 2
    for layer in cal.layers.values():
        assert tuple(layer.q_mean_real.shape) == (model.num_attention_heads, freq)
        assert bool(torch.isfinite(layer.q_abs_mean).all()) and bool((layer.q_abs_mean >= 0).all())
    got = cal.to_device(model, torch.device("cpu"))
    want = _oracle(cal, model)
    for index in want:
        for field in ("q_mean_real", "q_mean_imag", "q_abs_mean", "freq_scale_sq", "omega"):
            assert torch.equal(getattr(got[index], field), getattr(want[index], field))
        if want[index].q_pass_mean is not None:
            assert tuple(want[index].q_pass_mean.shape) == (model.num_kv_heads, model.num_attention_heads // model.num_kv_heads, model.head_dim - model.effective_rotary_dim)
            assert torch.equal(got[index].q_pass_mean, want[index].q_pass_mean)
    if schema == "layer_stats":
        # Exact inverse frequencies ship with the schema-3 artifacts; they are the
        # default 1/theta^(2i/R) of the model to float32 rounding.
        first = want[model.full_attention_layer_indices[0]]
        torch.testing.assert_close(first.omega, stats_ref.default_omega(model.effective_rotary_dim, model.rope_theta), rtol=1e-5, atol=0.0)
