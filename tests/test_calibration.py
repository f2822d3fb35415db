"""Host logic of the calibration generator (no GPU): model shape, inputs,
fingerprints, artifact validation, locking, runner settings and the CLI.

Scenarios follow the reference's tests/test_calibration.py; the accumulation
itself needs a HIP device and is covered by tests/test_gpu_calibration.py.
"""

from __future__ import annotations

import concurrent.futures
import time
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from kvcompress_mi355x import calibration
from kvcompress_mi355x.calibration import CalibrationRequest, generate_calibration_artifact
from kvcompress_mi355x.methods.base import ModelShape
from kvcompress_mi355x.model import model_shape_from_config


class _Config(SimpleNamespace):
    def to_dict(self):
        return dict(vars(self))


def _qwen2_config(**overrides):
    values = dict(
        model_type="qwen2",
        num_hidden_layers=2,
        num_attention_heads=2,
        num_key_value_heads=1,
        hidden_size=8,
        head_dim=4,
        rope_theta=10000.0,
        rope_scaling=None,
        rope_parameters=None,
    )
    values.update(overrides)
    return _Config(**values)


def _layer_stats(layers=2, heads=2, freq=2, with_rope=True):
    out = {}
    for index in range(layers):
        entry = {
            "q_mean_real": torch.zeros(heads, freq),
            "q_mean_imag": torch.zeros(heads, freq),
            "q_abs_mean": torch.ones(heads, freq),
        }
        if with_rope:
            entry["inv_freq"] = torch.ones(freq)
            entry["freq_scale_sq"] = torch.ones(1, freq)
        out[str(index)] = entry
    return out


# ------------------------------------------------------------- model shape --


def test_model_shape_from_config_defaults_and_head_dim() -> None:
    shape = model_shape_from_config(SimpleNamespace(hf_text_config=_qwen2_config(head_dim=None, hidden_size=16)))
    assert shape == ModelShape("qwen2", 2, 2, 1, 8, 10000.0, False, 8, (0, 1))
    assert shape.effective_rotary_dim == 8


def test_model_shape_hybrid_partial_rope_and_scaling() -> None:
    text = _qwen2_config(
        model_type="qwen3_5_moe_text",
        num_hidden_layers=4,
        num_attention_heads=16,
        num_key_value_heads=2,
        head_dim=256,
        rope_theta=None,
        rope_parameters={"rope_theta": 1e7, "partial_rotary_factor": 0.25, "rope_type": "default"},
        layer_types=["linear_attention", "linear_attention", "linear_attention", "full_attention"],
    )
    shape = model_shape_from_config(SimpleNamespace(hf_config=text))
    assert shape.rotary_dim == 64 and shape.rope_theta == 1e7
    assert shape.full_attention_layer_indices == (3,)
    # Any rope_parameters key beyond theta and type counts as scaling (pkg/model.py:97-109).
    assert shape.has_rope_scaling
    plain = _qwen2_config(rope_parameters={"rope_theta": 1e6, "rope_type": "default"})
    assert not model_shape_from_config(SimpleNamespace(hf_text_config=plain)).has_rope_scaling
    scaled = model_shape_from_config(SimpleNamespace(hf_text_config=_qwen2_config(rope_scaling={"rope_type": "yarn", "factor": 4.0})))
    assert scaled.has_rope_scaling


@pytest.mark.parametrize(
    "overrides, message",
    [
        ({"num_hidden_layers": 0}, "layer count"),
        ({"num_key_value_heads": 3, "num_attention_heads": 4}, "divisible"),
        ({"head_dim": 5}, "even"),
        ({"rotary_dim": 6}, "rotary"),
        ({"layer_types": ["full_attention"]}, "length"),
        ({"layer_types": ["full_attention", "sliding"]}, "unsupported"),
        ({"layer_types": ["linear_attention", "linear_attention"]}, "no full-attention"),
    ],
)
def test_model_shape_rejects(overrides, message) -> None:
    with pytest.raises(ValueError, match=message):
        model_shape_from_config(SimpleNamespace(hf_text_config=_qwen2_config(**overrides)))


# ------------------------------------------------------------------ inputs --


def test_builtin_text_and_explicit_input(tmp_path: Path) -> None:
    text, source = calibration.calibration_text(CalibrationRequest(model="m", output=tmp_path / "s.pt", max_length=200))
    assert source == calibration.BUILTIN_INPUT_SOURCE
    assert len(text) >= 200 * 6
    path = tmp_path / "input.txt"
    path.write_text("hello calibration", encoding="utf-8")
    text, source = calibration.calibration_text(CalibrationRequest(model="m", output=tmp_path / "s.pt", input_path=path))
    assert text == "hello calibration" and source == str(path.resolve())


def test_generator_rejects_empty_or_missing_input(tmp_path: Path) -> None:
    empty = tmp_path / "empty.txt"
    empty.write_text("  \n", encoding="utf-8")
    with pytest.raises(ValueError, match="empty"):
        calibration.calibration_text(CalibrationRequest(model="m", output=tmp_path / "s.pt", input_path=empty))
    with pytest.raises(ValueError, match="does not exist"):
        calibration.calibration_text(
            CalibrationRequest(model="m", output=tmp_path / "s.pt", input_path=tmp_path / "missing.txt")
        )


def test_generator_rejects_short_max_length(tmp_path: Path) -> None:
    with pytest.raises(ValueError, match="at least 128"):
        generate_calibration_artifact(CalibrationRequest(model="m", output=tmp_path / "s.pt", max_length=64))


def test_dtype_names() -> None:
    assert calibration.dtype_name(torch.float16) == "float16"
    assert calibration.dtype_name("half") == "float16"
    assert calibration.dtype_name("auto") == "bfloat16"
    assert calibration.torch_dtype("float") == torch.float32
    with pytest.raises(ValueError, match="unsupported"):
        calibration.torch_dtype("int8")


def test_distributed_calibration_reports_missing_accelerate(tmp_path: Path, monkeypatch) -> None:
    request = CalibrationRequest(model="fake/model", output=tmp_path / "stats.pt", device_map="auto")
    monkeypatch.setattr(calibration.importlib.util, "find_spec", lambda name: None)
    with pytest.raises(RuntimeError, match="accelerate"):
        calibration._artifact(request)


# ------------------------------------------------------------ fingerprints --


def test_model_source_fingerprint(tmp_path: Path) -> None:
    a = calibration.model_source_fingerprint("org/model", None)
    assert a.startswith("identifier:")
    assert a == calibration.model_source_fingerprint("org/model", "default")
    assert a != calibration.model_source_fingerprint("org/model", "v2")
    with pytest.raises(ValueError, match="no checkpoint files"):
        calibration.model_source_fingerprint(str(tmp_path), None)
    (tmp_path / "config.json").write_text("{}", encoding="utf-8")
    local = calibration.model_source_fingerprint(str(tmp_path), None)
    assert local.startswith("local-manifest:")
    (tmp_path / "model.safetensors").write_bytes(b"0123")
    assert calibration.model_source_fingerprint(str(tmp_path), None) != local


def test_plugin_generated_artifact_rejects_a_different_model_source(tmp_path: Path) -> None:
    output = tmp_path / "stats.pt"
    torch.save(
        {
            "metadata": {
                "generator": calibration.GENERATOR,
                "model": "model/a",
                "model_revision": "default",
                "model_source_fingerprint": calibration.model_source_fingerprint("model/a", None),
                "model_type": "qwen2",
                "num_layers": 2,
                "num_attention_heads": 2,
                "num_kv_heads": 1,
                "head_dim": 4,
                "rope_theta": 10000.0,
            },
            "layer_stats": _layer_stats(),
        },
        output,
    )
    shape = ModelShape("qwen2", 2, 2, 1, 4, 10000.0, False)
    calibration.validate_artifact(output, shape, SimpleNamespace(model="model/a", revision=None))
    with pytest.raises(ValueError, match="model_source_fingerprint"):
        calibration.validate_artifact(output, shape, SimpleNamespace(model="model/b", revision=None))


@pytest.mark.parametrize("generator, checked", [("kvcompress-mi355x", True), ("vllm-ascend-kvcompress-hust", True), (None, False)])
def test_provenance_is_checked_for_both_generators(tmp_path: Path, generator, checked) -> None:
    # Artifacts of this build and of the reference record their model source and
    # are held to it; an artifact without a generator (e.g. a hand-made or legacy
    # one) is checked for shape only.
    output = tmp_path / "stats.pt"
    metadata = {
        "model": "model/a",
        "model_revision": "default",
        "model_source_fingerprint": calibration.model_source_fingerprint("model/a", None),
        "model_type": "qwen2",
    }
    if generator is not None:
        metadata["generator"] = generator
    torch.save({"metadata": metadata, "layer_stats": _layer_stats()}, output)
    shape = ModelShape("qwen2", 2, 2, 1, 4, 10000.0, False)
    calibration.validate_artifact(output, shape, SimpleNamespace(model="model/a", revision=None))
    if checked:
        with pytest.raises(ValueError, match="calibration model 'model/a' does not match 'model/b'"):
            calibration.validate_artifact(output, shape, SimpleNamespace(model="model/b", revision=None))
        with pytest.raises(ValueError, match="model_revision"):
            calibration.validate_artifact(output, shape, SimpleNamespace(model="model/a", revision="v2"))
    else:
        calibration.validate_artifact(output, shape, SimpleNamespace(model="model/b", revision=None))


def test_fingerprint_format_is_the_reference_one(tmp_path: Path) -> None:
    # "identifier:" + sha256("<id>@<revision>") and "local-manifest:" + sha256 of the
    # compact sorted-key JSON list of [name, size, mtime_ns] (pkg/calibration.py:530-552),
    # so artifacts validate on either side; computed here from the definition.
    import hashlib
    import json
    import os

    assert calibration.model_source_fingerprint("org/m", "r1") == "identifier:" + hashlib.sha256(b"org/m@r1").hexdigest()
    for name, data in (("config.json", b"{}"), ("b.safetensors", b"12"), ("a.bin", b"3"), ("notes.txt", b"x")):
        (tmp_path / name).write_bytes(data)
    (tmp_path / "sub.bin").mkdir()
    entries = []
    for name in sorted(["a.bin", "b.safetensors", "config.json"]):
        st = os.stat(tmp_path / name)
        entries.append([name, st.st_size, st.st_mtime_ns])
    want = "local-manifest:" + hashlib.sha256(json.dumps(entries, sort_keys=True, separators=(",", ":")).encode()).hexdigest()
    assert calibration.model_source_fingerprint(str(tmp_path), None) == want


# ------------------------------------------------------- publish and runner --


def test_concurrent_generation_publishes_one_atomic_artifact(tmp_path: Path, monkeypatch) -> None:
    output = tmp_path / "stats.pt"
    request = CalibrationRequest(model="fake/model", output=output, max_length=128)
    calls = []
    payload = {"metadata": {}, "layer_stats": _layer_stats(layers=1, heads=1, with_rope=False)}

    def generate(_request):
        calls.append(1)
        time.sleep(0.1)
        return payload

    monkeypatch.setattr(calibration, "_artifact", generate)
    monkeypatch.setattr(calibration, "_validate_for_request", lambda path, request: None)
    with concurrent.futures.ThreadPoolExecutor(max_workers=2) as pool:
        results = list(pool.map(generate_calibration_artifact, (request, request)))
    assert sorted(results) == [False, True]
    assert len(calls) == 1
    assert output.is_file()
    assert not list(tmp_path.glob("*.tmp"))


def _runner_selection(output: Path, **options):
    return SimpleNamespace(method="triattention", method_config={"stats_path": str(output), **options})


def _write_generated(output: Path):
    torch.save(
        {
            "metadata": {
                "model_type": "qwen2",
                "num_layers": 2,
                "num_attention_heads": 2,
                "num_kv_heads": 1,
                "head_dim": 4,
                "rope_theta": 10000.0,
            },
            "layer_stats": _layer_stats(),
        },
        output,
    )


def test_runner_uses_model_settings_for_missing_artifact(tmp_path: Path, monkeypatch) -> None:
    output = tmp_path / "stats.pt"
    selection = _runner_selection(output, calibration_max_length=1024, calibration_local_files_only=True)
    model_config = SimpleNamespace(
        model="fake/model",
        tokenizer=None,
        revision="model-revision",
        tokenizer_revision=None,
        trust_remote_code=True,
        dtype=torch.float16,
        hf_text_config=_qwen2_config(),
    )
    runner = SimpleNamespace(model_config=model_config, device=torch.device("cuda:0"))
    captured = []

    def generate(request):
        captured.append(request)
        _write_generated(output)
        return True

    monkeypatch.setattr(calibration, "generate_calibration_artifact", generate)
    assert calibration.ensure_calibration_for_runner(runner, selection)
    request = captured[0]
    assert request.model == "fake/model" and request.revision == "model-revision"
    assert request.device == "cuda:0" and request.device_map is None
    assert request.dtype == "float16" and request.max_length == 1024 and request.local_files_only
    # An existing artifact is validated, not regenerated.
    monkeypatch.setattr(calibration, "generate_calibration_artifact", lambda request: pytest.fail("regenerated"))
    assert not calibration.ensure_calibration_for_runner(runner, selection)


def test_tensor_parallel_runner_uses_auto_device_map(tmp_path: Path, monkeypatch) -> None:
    output = tmp_path / "stats.pt"
    runner = SimpleNamespace(
        model_config=SimpleNamespace(
            model="fake/model",
            tokenizer=None,
            revision=None,
            tokenizer_revision=None,
            trust_remote_code=False,
            dtype=torch.bfloat16,
            hf_text_config=_qwen2_config(),
        ),
        device=torch.device("cuda:0"),
        vllm_config=SimpleNamespace(parallel_config=SimpleNamespace(tensor_parallel_size=2)),
    )
    captured = []

    def generate(request):
        captured.append(request)
        _write_generated(output)
        return True

    monkeypatch.setattr(calibration, "generate_calibration_artifact", generate)
    assert calibration.ensure_calibration_for_runner(runner, _runner_selection(output))
    assert captured[0].device_map == "auto"


def test_runner_does_not_generate_when_disabled_or_other_method(tmp_path: Path, monkeypatch) -> None:
    monkeypatch.setattr(calibration, "generate_calibration_artifact", lambda request: pytest.fail("generated"))
    runner = SimpleNamespace(model_config=SimpleNamespace(hf_text_config=_qwen2_config()))
    selection = _runner_selection(tmp_path / "missing.pt", auto_calibrate=False)
    assert not calibration.ensure_calibration_for_runner(runner, selection)
    assert not calibration.ensure_calibration_for_runner(runner, SimpleNamespace(method="other", method_config={}))


def test_cli_builds_the_request(tmp_path: Path, monkeypatch) -> None:
    captured = []
    monkeypatch.setattr(calibration, "generate_calibration_artifact", lambda request: captured.append(request) or True)
    rc = calibration.main(
        ["--model", "org/m", "--output", str(tmp_path / "s.pt"), "--max-length", "512", "--dtype", "float16",
         "--local-files-only", "--device", "cuda:0"]
    )
    assert rc == 0
    request = captured[0]
    assert request.model == "org/m" and request.max_length == 512 and request.dtype == "float16"
    assert request.local_files_only and request.device == "cuda:0" and not request.force
