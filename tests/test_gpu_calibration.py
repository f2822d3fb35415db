"""GPU parity of the calibration statistics (kvc_qstats_accumulate) and the
generator end to end.

The kernel's float64 sums are compared with the float64 brute force of the
definitions (oracle/calibration_ref.py) on the same float32-widened values:
real, imaginary and pass sums to 1e-12 relative (only the summation order
differs), magnitude sums to 1e-6 (each term is the reference's float32
magnitude, the brute force keeps it in float64); and with the reference's
float32 torch path (the restatement) to 1e-4.  Generator scenarios follow the
reference's tests/test_calibration.py; the end-to-end case runs a small
random-weight Qwen2 model saved to and loaded from a local directory (no
network), and compares every layer's artifact statistics with the restatement
hooked into the same model on the CPU.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import calibration_ref as cref

pytestmark = pytest.mark.gpu


def _calib():
    from kvcompress_mi355x import calibration

    return calibration


def _check_sums(acc, values: np.ndarray, rotary: int) -> None:
    """acc: LayerAccumulator after adding `values` [T, H, D] (float32-representable)."""
    want = cref.query_sums_brute(values, rotary) if values.size <= 20000 else _sums_numpy(values, rotary)
    scale = np.abs(values).sum(axis=0).max() + 1.0
    pairs = (("real", acc.real_sum, 1e-12), ("imag", acc.imag_sum, 1e-12), ("abs", acc.abs_sum, 1e-6))
    for key, got, rtol in pairs:
        np.testing.assert_allclose(got.cpu().numpy(), want[key], rtol=rtol, atol=rtol * scale, err_msg=key)
    if want["pass"].size:
        np.testing.assert_allclose(acc.pass_sum.cpu().numpy(), want["pass"], rtol=1e-12, atol=1e-12 * scale)
    else:
        assert acc.pass_sum is None
    assert acc.count == values.shape[0]


def _sums_numpy(values: np.ndarray, rotary: int) -> dict[str, np.ndarray]:
    v = values.astype(np.float64)
    f = rotary // 2
    return {
        "real": v[..., :f].sum(0),
        "imag": v[..., f:rotary].sum(0),
        "abs": np.hypot(v[..., :f], v[..., f:rotary]).sum(0),
        "pass": v[..., rotary:].sum(0),
    }


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("heads, head_dim, rotary, tokens", [(5, 128, 128, 37), (4, 256, 64, 300), (3, 64, 32, 1)])
def test_qstats_matches_brute_force(hip_device, dtype, heads, head_dim, rotary, tokens) -> None:
    calibration = _calib()
    g = torch.Generator().manual_seed(heads * 131 + tokens)
    q = (torch.randn(tokens, heads * head_dim, generator=g) * 3).to(dtype)
    acc = calibration.LayerAccumulator()
    acc.add(q.to(hip_device), heads, head_dim, rotary)
    torch.cuda.synchronize()
    _check_sums(acc, q.float().reshape(tokens, heads, head_dim).numpy(), rotary)


def test_qstats_gate_strides_head_shape_and_repeated_adds(hip_device) -> None:
    calibration = _calib()
    heads, head_dim, rotary = 6, 128, 96
    g = torch.Generator().manual_seed(5)
    chunks = [torch.randn(2, n, heads * head_dim, generator=g).to(torch.bfloat16) for n in (17, 64, 3)]
    acc = calibration.LayerAccumulator()
    for i, chunk in enumerate(chunks):
        dev = chunk.to(hip_device)
        if i == 0:
            # q_proj with an output gate after Q: the gate half must not count.
            gate = torch.full_like(dev, float("nan"))
            acc.add(torch.cat([dev, gate], dim=-1), heads, head_dim, rotary)
        elif i == 1:
            # q_norm output, [..., heads, head_dim].
            acc.add(dev.reshape(2, -1, heads, head_dim), heads, head_dim, rotary)
        else:
            acc.add(dev, heads, head_dim, rotary)
    torch.cuda.synchronize()
    values = torch.cat([c.reshape(-1, heads, head_dim) for c in chunks]).float().numpy()
    _check_sums(acc, values, rotary)


def test_qstats_large_input_matches_reference_path_and_is_deterministic(hip_device) -> None:
    calibration = _calib()
    heads, head_dim, rotary, tokens = 40, 128, 128, 6000
    g = torch.Generator().manual_seed(9)
    q = (torch.randn(tokens, heads * head_dim, generator=g) + 0.5).to(torch.bfloat16)
    runs = []
    for _ in range(2):
        acc = calibration.LayerAccumulator()
        acc.add(q.to(hip_device), heads, head_dim, rotary)
        runs.append(acc)
    torch.cuda.synchronize()
    for name in ("real_sum", "imag_sum", "abs_sum"):
        assert torch.equal(getattr(runs[0], name), getattr(runs[1], name)), f"{name} not deterministic"
    _check_sums(runs[0], q.float().reshape(tokens, heads, head_dim).numpy(), rotary)
    ref = cref.QueryStatsAccumulator()
    ref.add(q, heads, head_dim, rotary)
    got, want = runs[0].means(), ref.means()
    for key in ("q_mean_real", "q_mean_imag", "q_abs_mean"):
        np.testing.assert_allclose(got[key].numpy(), want[key].numpy(), rtol=1e-4, atol=1e-6, err_msg=key)


def test_qstats_rejects_invalid_arguments(hip_device) -> None:
    calibration = _calib()
    from kvcompress_mi355x import _native

    acc = calibration.LayerAccumulator()
    with pytest.raises(RuntimeError, match="values per row"):
        acc.add(torch.zeros(4, 10, device=hip_device), 2, 4, 4)
    out = torch.zeros(8, dtype=torch.float64, device=hip_device)
    q = torch.zeros(4, 16, device=hip_device)
    stream = int(torch.cuda.current_stream().cuda_stream)
    lib = _native.load()
    state = torch.zeros(int(lib.kvc_qstats_state_bytes(2, 8, 8)), dtype=torch.uint8, device=hip_device)
    args = (_native.DTYPE_FP32, q.data_ptr(), 4)
    with pytest.raises(ValueError, match="token_stride"):
        _native.call("kvc_qstats_accumulate", stream, *args, 8, 2, 8, 8, state.data_ptr(), state.numel())
    with pytest.raises(ValueError, match="rotary_dim"):
        _native.call("kvc_qstats_accumulate", stream, *args, 16, 2, 8, 7, state.data_ptr(), state.numel())
    with pytest.raises(ValueError, match="state"):
        _native.call("kvc_qstats_accumulate", stream, *args, 16, 2, 8, 8, state.data_ptr(), 8)
    with pytest.raises(ValueError, match="null pointer"):
        _native.call("kvc_qstats_finish", stream, 2, 8, 4, state.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(), None)
    assert lib.kvc_qstats_state_bytes(2, 8, 9) == 0


# ---------------------------------------------------------------- generator --


class _FakeAttention(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.q_proj = torch.nn.Linear(8, 8, bias=False)


class _FakeLayer(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.self_attn = _FakeAttention()


class _FakeModel(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList([_FakeLayer(), _FakeLayer()])

    def forward(self, input_ids, attention_mask=None, use_cache=False):
        del attention_mask, use_cache
        hidden = torch.nn.functional.one_hot(input_ids % 8, num_classes=8).float()
        for layer in self.layers:
            hidden = layer.self_attn.q_proj(hidden)
        return (hidden,)


class _FakeConfig:
    model_type = "qwen2"
    num_hidden_layers = 2
    num_attention_heads = 2
    num_key_value_heads = 1
    hidden_size = 8
    head_dim = 4
    rope_theta = 10000.0
    rope_scaling = None
    rope_parameters = None

    def to_dict(self):
        return {"model_type": self.model_type, "num_hidden_layers": 2, "num_attention_heads": 2, "head_dim": 4}


class _FakeTokenizer:
    def __init__(self, count: int = 32, vocab: int = 8) -> None:
        self.count, self.vocab = count, vocab

    def __call__(self, text, **kwargs):
        del text, kwargs
        ids = (torch.arange(self.count) * 7 % self.vocab).reshape(1, -1)
        return {"input_ids": ids, "attention_mask": torch.ones_like(ids)}


def test_generator_creates_safe_model_matched_artifact(hip_device, tmp_path: Path, monkeypatch) -> None:
    calibration = _calib()
    import transformers

    from kvcompress_mi355x.methods.base import ModelShape
    from kvcompress_mi355x.methods.triattention.stats import CalibrationStats

    monkeypatch.setattr(transformers.AutoConfig, "from_pretrained", lambda *a, **k: _FakeConfig())
    monkeypatch.setattr(transformers.AutoTokenizer, "from_pretrained", lambda *a, **k: _FakeTokenizer())
    models = []

    def load_model(*args, **kwargs):
        torch.manual_seed(0)
        models.append(_FakeModel())
        return models[-1]

    monkeypatch.setattr(transformers.AutoModel, "from_pretrained", load_model)
    output = tmp_path / "stats.pt"
    request = calibration.CalibrationRequest(model="fake/model", output=output, device="cpu", dtype="float32", max_length=128)
    assert calibration.generate_calibration_artifact(request)
    assert not calibration.generate_calibration_artifact(request)
    assert len(models) == 1
    assert not list(tmp_path.glob("*.tmp"))
    artifact = CalibrationStats.load(output)
    assert artifact.validate(ModelShape("qwen2", 2, 2, 1, 4, 10000.0, False)) == ()
    # The reference's generator name (its loader checks provenance under that
    # name only); this package is recorded as the producer.
    assert artifact.metadata["generator"] == calibration.REFERENCE_GENERATOR == "vllm-ascend-kvcompress-hust"
    assert artifact.metadata["producer"] == calibration.GENERATOR == "kvcompress-mi355x"
    assert artifact.metadata["token_count"] == 32
    assert artifact.metadata["input_source"] == calibration.BUILTIN_INPUT_SOURCE
    assert artifact.layers[0].q_mean_real.shape == (2, 2)
    assert artifact.layers[0].inv_freq is not None
    # Same statistics from the restatement hooked into the same model.
    model = models[0]
    accs = [cref.QueryStatsAccumulator() for _ in range(2)]
    hooks = [
        layer.self_attn.q_proj.register_forward_hook(lambda m, i, o, a=acc: a.add(o, 2, 4, 4))
        for layer, acc in zip(model.layers, accs)
    ]
    with torch.inference_mode():
        model(_FakeTokenizer()("x")["input_ids"])
    for h in hooks:
        h.remove()
    for index, acc in enumerate(accs):
        want = acc.means()
        got = artifact.layers[index]
        for key in ("q_mean_real", "q_mean_imag", "q_abs_mean"):
            torch.testing.assert_close(getattr(got, key), want[key], rtol=1e-5, atol=1e-6)


def test_generator_loads_only_qwen35_text_model(hip_device, tmp_path: Path, monkeypatch) -> None:
    calibration = _calib()
    import transformers

    config = _FakeConfig()
    config.model_type = "qwen3_5_moe"
    config.text_config = _FakeConfig()
    monkeypatch.setattr(transformers.AutoConfig, "from_pretrained", lambda *a, **k: config)
    monkeypatch.setattr(transformers.AutoTokenizer, "from_pretrained", lambda *a, **k: _FakeTokenizer())
    captured = []

    def load_model(*args, **kwargs):
        captured.append(kwargs)
        return _FakeModel()

    monkeypatch.setattr(transformers.AutoModel, "from_pretrained", lambda *a, **k: pytest.fail("multimodal AutoModel"))
    monkeypatch.setattr(transformers.AutoModelForCausalLM, "from_pretrained", load_model)
    request = calibration.CalibrationRequest(model="fake/model", output=tmp_path / "stats.pt", max_length=128, device="cpu")
    assert calibration.generate_calibration_artifact(request)
    assert captured[0]["config"] is config.text_config
    assert captured[0]["key_mapping"] == {r"^model\.language_model\.(.+)$": r"model.\1"}


@pytest.mark.parametrize("device_name", ["cpu", "cuda:0"])
def test_generator_end_to_end_on_a_local_qwen2_checkpoint(hip_device, tmp_path: Path, monkeypatch, device_name) -> None:
    calibration = _calib()
    import transformers
    from transformers import Qwen2Config, Qwen2Model

    from kvcompress_mi355x.methods.triattention.stats import CalibrationStats

    torch.manual_seed(1)
    cfg = Qwen2Config(
        vocab_size=96,
        hidden_size=128,
        intermediate_size=256,
        num_hidden_layers=3,
        num_attention_heads=4,
        num_key_value_heads=2,
        max_position_embeddings=512,
        rope_theta=1e6,
    )
    model_dir = tmp_path / "tiny-qwen2"
    Qwen2Model(cfg).save_pretrained(model_dir)
    tokenizer = _FakeTokenizer(count=200, vocab=96)
    monkeypatch.setattr(transformers.AutoTokenizer, "from_pretrained", lambda *a, **k: tokenizer)
    output = tmp_path / "stats.pt"
    request = calibration.CalibrationRequest(
        model=str(model_dir), output=output, device=device_name, dtype="float32", local_files_only=True, max_length=256
    )
    assert calibration.generate_calibration_artifact(request)
    artifact = CalibrationStats.load(output)
    shape = calibration.shape_from_hf_config(cfg)
    assert artifact.validate(shape) == ()
    assert artifact.metadata["model_source_fingerprint"].startswith("local-manifest:")
    calibration.validate_artifact(output, shape, type("M", (), {"model": str(model_dir), "revision": None})())

    # The restatement hooked into the same checkpoint on the CPU.
    reference = transformers.AutoModel.from_pretrained(model_dir, local_files_only=True, dtype=torch.float32,
                                                       attn_implementation="eager").eval()
    accs = {i: cref.QueryStatsAccumulator() for i in range(cfg.num_hidden_layers)}
    hooks = [
        layer.self_attn.q_proj.register_forward_hook(lambda m, i, o, a=accs[idx]: a.add(o, 4, 32, 32))
        for idx, layer in enumerate(reference.layers)
    ]
    with torch.inference_mode():
        reference(input_ids=tokenizer("x")["input_ids"], use_cache=False)
    for h in hooks:
        h.remove()
    inv_freq = reference.rotary_emb.inv_freq.float()
    for index, acc in accs.items():
        want, got = acc.means(), artifact.layers[index]
        assert got.q_mean_real.shape == (4, 16)
        for key in ("q_mean_real", "q_mean_imag", "q_abs_mean"):
            torch.testing.assert_close(getattr(got, key), want[key], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(got.inv_freq, inv_freq)
        assert torch.equal(got.freq_scale_sq, torch.ones(1, 16))
