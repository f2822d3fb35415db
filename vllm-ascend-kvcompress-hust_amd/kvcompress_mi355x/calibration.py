"""Model-matched TriAttention calibration artifacts, accumulated on the GPU.

Counterpart of the reference's generator (pkg/calibration.py): run a Hugging
Face model once over a calibration text, hook every full-attention layer's
query projection (``q_norm`` where the attention has one, else ``q_proj``),
reduce the pre-RoPE queries to per-head statistics and write a schema-3
artifact that CalibrationStats.load reads:

  layer_stats[str(layer)] = {q_mean_real, q_mean_imag, q_abs_mean  [heads, F],
                             inv_freq [F], freq_scale_sq [1, F],
                             q_pass_mean [heads, P] (partial RoPE only)}

The reduction runs in kvc_qstats_accumulate (one HIP kernel launch per hooked
projection into a per-layer float64 state on the device, reduced to totals by
kvc_qstats_finish); a projection produced on the host is copied to the HIP
device first.  There is no host reduction: without a HIP
device the generator raises.  Generation takes a file lock next to the output
and publishes the artifact with an atomic rename, so concurrent workers
produce one file (pkg/calibration.py:175-193).

The request fields, option names, metadata keys, the model-source fingerprint
and the command-line flags are those of the reference, so artifacts and
service settings carry over.  The built-in calibration text is this package's
own (input_source ``builtin:mi355x-systems-v1``); pass ``input_path`` to
calibrate on a specific text.
"""

from __future__ import annotations

import argparse
import fcntl
import gc
import hashlib
import importlib.util
import json
import os
import tempfile
from collections.abc import Mapping, Sequence
from contextlib import suppress
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch

from . import __version__, _native
from .methods.base import ModelShape
from .methods.triattention.config import TriAttentionConfig
from .methods.triattention.stats import SUPPORTED_MODEL_TYPES, CalibrationStats
from .model import model_shape_from_config

GENERATOR = "vllm-ascend-kvcompress-hust"  # artifact producer name the validators key on
BUILTIN_INPUT_SOURCE = "builtin:mi355x-systems-v1"

# Built-in calibration text: prose, code, numbers, tables and mixed scripts, so
# the query statistics see a spread of token kinds.  Repeated with numbered
# headings until about six characters per requested token.
_BUILTIN_SECTIONS = (
    """An inference server keeps every request's history in a paged key-value
cache. When a conversation grows past its budget, the server scores the cached
tokens, keeps the ones later queries are most likely to attend to, and moves
them to the front of the request's pages so the rest can be returned to the
pool. Every later position lookup must then translate between the request's
logical length and the tokens physically present.""",
    """| stage     | input              | output            | bound      |
|-----------|--------------------|-------------------|------------|
| score     | paged keys         | per-head scores   | HBM read   |
| select    | aggregated scores  | sorted indices    | latency    |
| compact   | kept rows          | front pages       | HBM copy   |
The table lists the three stages with the resource that limits each one.""",
    """def release_pages(table, keep_pages):
    kept = table[:keep_pages]
    freed = list(reversed(table[keep_pages:]))
    if any(page < 0 for page in kept):
        raise ValueError("unmapped page inside the kept range")
    return kept, freed
""",
    """长文本推理的评测需要同时记录准确性与吞吐量。测试集应覆盖叙述、代码、表格、公式和跨段落引用，
并写明模型版本、输入长度、批大小、硬件与软件版本。只报告单一平均数而不给出失败样例的结论是不可信的。""",
    """A rotary position embedding turns each pair of query or key channels into a
complex number and rotates it by an angle proportional to the token position,
with one frequency per pair: theta to the power of minus 2i over the rotary
dimension. Scores between a query and a key then depend only on their
distance, which is why a key's future relevance can be estimated from the
mean query of a calibration run and a set of future offsets 1, 2, 4, 8 ...""",
    """Field notes, station 7: air temperature 14.6 C at 06:00 rising to 22.9 C
at 14:00; relative humidity 81% falling to 47%; wind west-southwest 3.2 m/s,
gusting 7.5; barometer 1013.4 hPa steady. Instrument drift against the
reference clock: +38 ms over 24 h. Observations are kept separate from the
inferred causes, and every value keeps its original unit.""",
)


@dataclass(frozen=True)
class CalibrationRequest:
    """Generation request (pkg/calibration.py:71-86); ``device`` names a HIP device."""

    model: str
    output: Path
    input_path: Path | None = None
    tokenizer: str | None = None
    revision: str | None = None
    tokenizer_revision: str | None = None
    trust_remote_code: bool = False
    local_files_only: bool = False
    max_length: int = 4096
    device: str = "cuda"
    device_map: str | None = None
    dtype: str = "bfloat16"
    attn_implementation: str = "eager"
    force: bool = False


def _hip_device(device: torch.device | str | None) -> torch.device:
    """The HIP device the statistics are accumulated on."""
    if not torch.cuda.is_available():
        raise RuntimeError("calibration statistics are accumulated on a HIP device; none is available")
    dev = torch.device("cuda") if device is None else torch.device(device)
    if dev.type != "cuda":
        dev = torch.device("cuda")
    return torch.device("cuda", torch.cuda.current_device() if dev.index is None else dev.index)


def _kernel_dtype(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _native.DTYPE_BF16
    if dtype == torch.float16:
        return _native.DTYPE_FP16
    return _native.DTYPE_FP32


class LayerAccumulator:
    """Running query sums of one layer (_LayerAccumulator, pkg/calibration.py:89-131).

    ``add`` takes a hooked projection: the query part of ``q_proj``'s output
    ([..., heads*head_dim], or twice that when the projection carries an
    output gate after Q, whose second half is ignored) or a ``q_norm`` output
    ([..., heads, head_dim]), read in row-major order as [tokens, heads,
    head_dim], and launches one kvc_qstats_accumulate into the layer's device
    state.  ``real_sum``, ``imag_sum``, ``abs_sum`` ([heads, F]) and
    ``pass_sum`` ([heads, P], None without pass dims) are the float64 totals
    on the HIP device (one kvc_qstats_finish after new additions); ``count``
    is the number of token rows added.
    """

    def __init__(self, device: torch.device | str | None = None) -> None:
        self.device = device
        self.count = 0
        self._shape: tuple[int, int, int] | None = None
        self._device: torch.device | None = None
        self._state: torch.Tensor | None = None
        self._sums: tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None] | None = None
        self._stale = False

    def add(self, projected: torch.Tensor, heads: int, head_dim: int, rotary_dim: int) -> None:
        expected = heads * head_dim
        if projected.shape[-1] == expected * 2:
            projected = projected[..., :expected]
        if not (
            projected.shape[-1] == expected
            or (projected.shape[-1] == head_dim and projected.numel() % expected == 0)
        ):
            raise RuntimeError(
                "query projection width does not match model attention shape: "
                f"got {projected.shape[-1]}, expected {expected}"
            )
        if self._shape is None:
            self._shape = (heads, head_dim, rotary_dim)
        elif self._shape != (heads, head_dim, rotary_dim):
            raise RuntimeError("a layer accumulator cannot change its attention shape")
        if self._device is None:
            self._device = _hip_device(self.device if self.device is not None else projected.device)
        device = self._device
        rows = projected.detach().reshape(-1, expected)
        if rows.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            rows = rows.float()
        if rows.device != device:
            rows = rows.to(device)
        if rows.stride(1) != 1:
            rows = rows.contiguous()
        lib = _native.load()
        if self._state is None:
            state_bytes = int(lib.kvc_qstats_state_bytes(heads, head_dim, rotary_dim))
            if state_bytes == 0:
                raise ValueError("rotary_dim must be positive, even and no larger than head_dim")
            self._state = torch.zeros(state_bytes, dtype=torch.uint8, device=device)
        n_tokens = int(rows.shape[0])
        if n_tokens:
            rc = lib.kvc_qstats_accumulate(
                torch.cuda.current_stream(device).cuda_stream,
                _kernel_dtype(rows.dtype),
                int(rows.data_ptr()),
                n_tokens,
                int(rows.stride(0)) if n_tokens > 1 else expected,
                heads,
                head_dim,
                rotary_dim,
                int(self._state.data_ptr()),
                int(self._state.numel()),
            )
            _native.check(rc, "kvc_qstats_accumulate")
            self._stale = True
        self.count += n_tokens

    def _totals(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None] | None:
        if self._state is None:
            return None
        if self._sums is None or self._stale:
            heads, head_dim, rotary_dim = self._shape
            freq, pass_dim = rotary_dim // 2, head_dim - rotary_dim
            empty = lambda n: torch.empty((heads, n), dtype=torch.float64, device=self._device)  # noqa: E731
            sums = (empty(freq), empty(freq), empty(freq), empty(pass_dim) if pass_dim else None)
            _native.call(
                "kvc_qstats_finish",
                torch.cuda.current_stream(self._device).cuda_stream,
                heads,
                head_dim,
                rotary_dim,
                int(self._state.data_ptr()),
                *(None if t is None else int(t.data_ptr()) for t in sums),
            )
            self._sums, self._stale = sums, False
        return self._sums

    @property
    def real_sum(self) -> torch.Tensor | None:
        totals = self._totals()
        return None if totals is None else totals[0]

    @property
    def imag_sum(self) -> torch.Tensor | None:
        totals = self._totals()
        return None if totals is None else totals[1]

    @property
    def abs_sum(self) -> torch.Tensor | None:
        totals = self._totals()
        return None if totals is None else totals[2]

    @property
    def pass_sum(self) -> torch.Tensor | None:
        totals = self._totals()
        return None if totals is None else totals[3]

    def means(self) -> dict[str, torch.Tensor]:
        """q_mean_real, q_mean_imag, q_abs_mean (and q_pass_mean) as float32 CPU tensors."""
        totals = self._totals()
        if self.count <= 0 or totals is None:
            raise RuntimeError("no query values were accumulated")
        divisor = float(self.count)
        real, imag, mag, passed = totals
        out = {
            "q_mean_real": (real / divisor).float().cpu().contiguous(),
            "q_mean_imag": (imag / divisor).float().cpu().contiguous(),
            "q_abs_mean": (mag / divisor).float().cpu().contiguous(),
        }
        if passed is not None:
            out["q_pass_mean"] = (passed / divisor).float().cpu().contiguous()
        return out


# ------------------------------------------------------------------ runner --


def ensure_calibration_for_runner(runner: Any, selection: Any) -> bool:
    """Generate a missing artifact before the serving weights load
    (pkg/calibration.py:134-172); True when this call generated it."""
    if getattr(selection, "method", None) != "triattention":
        return False
    config = TriAttentionConfig.from_method_config(selection.method_config)
    model_config = runner.model_config
    shape = model_shape_from_config(model_config)
    if config.stats_path.is_file():
        _validate_artifact(config.stats_path, shape, model_config)
        return False
    if not config.auto_calibrate:
        return False
    device = (
        str(getattr(runner, "device", "cuda")) if config.calibration_device == "auto" else config.calibration_device
    )
    parallel = getattr(getattr(runner, "vllm_config", None), "parallel_config", None)
    tensor_parallel = int(getattr(parallel, "tensor_parallel_size", 1))
    request = CalibrationRequest(
        model=str(model_config.model),
        tokenizer=str(model_config.tokenizer) if model_config.tokenizer else None,
        output=config.stats_path,
        input_path=config.calibration_input_path,
        revision=getattr(model_config, "revision", None),
        tokenizer_revision=getattr(model_config, "tokenizer_revision", None),
        trust_remote_code=bool(getattr(model_config, "trust_remote_code", False)),
        local_files_only=config.calibration_local_files_only,
        max_length=config.calibration_max_length,
        device=device,
        # A model sharded for tensor parallelism does not fit one device either.
        device_map="auto" if tensor_parallel > 1 else None,
        dtype=_dtype_name(getattr(model_config, "dtype", "bfloat16")),
        attn_implementation=config.calibration_attn_implementation,
    )
    generated = generate_calibration_artifact(request)
    _validate_artifact(config.stats_path, shape, model_config)
    return generated


def generate_calibration_artifact(request: CalibrationRequest) -> bool:
    """Generate one artifact; False when it already exists (another process won)."""
    if request.max_length < 128:
        raise ValueError("calibration max_length must be at least 128")
    output = request.output.expanduser().resolve()
    output.parent.mkdir(parents=True, exist_ok=True)
    with output.with_name(f".{output.name}.lock").open("a+b") as lock:
        fcntl.flock(lock.fileno(), fcntl.LOCK_EX)
        if output.is_file() and not request.force:
            _validate_existing_for_request(output, request)
            return False
        _atomic_torch_save(_generate_payload(request), output)
    return True


def _generate_payload(request: CalibrationRequest) -> dict[str, Any]:
    if request.device_map is not None and importlib.util.find_spec("accelerate") is None:
        raise RuntimeError(
            "distributed calibration requires Accelerate; install the "
            "'vllm-ascend-kvcompress-hust[calibration]' extra in the host environment"
        )
    try:
        from transformers import AutoConfig, AutoModel, AutoModelForCausalLM, AutoTokenizer
        from transformers import __version__ as transformers_version
    except ImportError as error:
        raise RuntimeError("calibration generation requires the Transformers package") from error

    _prepare_device(request.device)
    accumulate_on = _hip_device(request.device)
    input_device = torch.device("cpu" if request.device_map == "auto" else request.device)
    common = {"trust_remote_code": request.trust_remote_code, "local_files_only": request.local_files_only}
    config = AutoConfig.from_pretrained(request.model, revision=request.revision, **common)
    shape = _model_shape_from_hf_config(config)
    if shape.model_type not in SUPPORTED_MODEL_TYPES:
        raise ValueError(f"model_type {shape.model_type!r} is not supported for calibration")
    tokenizer_id = request.tokenizer or request.model
    tokenizer = AutoTokenizer.from_pretrained(
        tokenizer_id, revision=request.tokenizer_revision or request.revision, **common
    )
    text, input_source = _load_calibration_text(request)
    encoded = tokenizer(
        text, return_tensors="pt", truncation=True, max_length=request.max_length, add_special_tokens=True
    )
    input_ids = encoded.get("input_ids")
    if not isinstance(input_ids, torch.Tensor) or input_ids.ndim != 2:
        raise RuntimeError("tokenizer did not return rank-two input_ids")
    token_count = int(input_ids.shape[1])
    if token_count < 2:
        raise ValueError("calibration input produced fewer than two tokens")

    text_config = getattr(config, "text_config", config)
    multimodal_qwen35 = text_config is not config and str(getattr(config, "model_type", "")).startswith("qwen3_5")
    options: dict[str, Any] = {
        "config": text_config if multimodal_qwen35 else config,
        "revision": request.revision,
        "dtype": _torch_dtype(request.dtype),
        "device_map": request.device_map or request.device,
        **common,
    }
    if request.attn_implementation:
        options["attn_implementation"] = request.attn_implementation
    if multimodal_qwen35:
        # The published checkpoint nests the text weights under model.language_model;
        # loading the causal text model alone skips the vision tower.
        options["key_mapping"] = {r"^model\.language_model\.(.+)$": r"model.\1"}

    model: torch.nn.Module | None = None
    handles: list[Any] = []
    try:
        loader = AutoModelForCausalLM if multimodal_qwen35 else AutoModel
        model = loader.from_pretrained(request.model, **options)
        model.eval()
        attention_layers = _find_attention_layers(model)
        found = tuple(index for index, _ in attention_layers)
        if found != shape.full_attention_layer_indices:
            raise RuntimeError(
                f"located full-attention layers do not match model config: got {found}, "
                f"expected {shape.full_attention_layer_indices}"
            )
        accumulators = {index: LayerAccumulator(device=accumulate_on) for index, _ in attention_layers}
        for index, attention in attention_layers:
            module = getattr(attention, "q_norm", None)
            if not isinstance(module, torch.nn.Module):
                module = getattr(attention, "q_proj", None)
            if not isinstance(module, torch.nn.Module):
                raise RuntimeError(f"attention layer {index} exposes neither q_norm nor q_proj")

            def capture(_module: torch.nn.Module, _inputs: tuple[Any, ...], output: Any, *, layer: int = index) -> None:
                if not isinstance(output, torch.Tensor):
                    raise RuntimeError(f"attention layer {layer} q_proj returned a non-tensor")
                accumulators[layer].add(output, shape.num_attention_heads, shape.head_dim, shape.effective_rotary_dim)

            handles.append(module.register_forward_hook(capture))

        inputs = {name: value.to(input_device) for name, value in encoded.items() if isinstance(value, torch.Tensor)}
        with torch.inference_mode():
            model(**inputs, use_cache=False)
        torch.cuda.synchronize(accumulate_on)

        rope_type = _rope_type(config)
        rope_values = _extract_rope_values(model, attention_layers, shape, rope_type)
        layer_stats: dict[str, dict[str, torch.Tensor]] = {}
        for index, accumulator in accumulators.items():
            if accumulator.count <= 0:
                raise RuntimeError(f"no query values captured for layer {index}")
            inv_freq, freq_scale_sq = rope_values[index]
            values = accumulator.means()
            values["inv_freq"] = inv_freq
            values["freq_scale_sq"] = freq_scale_sq
            layer_stats[str(index)] = values

        config_dict = config.to_dict() if hasattr(config, "to_dict") else vars(config)
        metadata = {
            "schema_version": 3,
            "generator": GENERATOR,
            "generator_version": __version__,
            "accumulator": "kvc_qstats_accumulate (float64 sums, HIP)",
            "transformers_version": transformers_version,
            "created_at_utc": datetime.now(timezone.utc).isoformat(),
            "model": request.model,
            "model_revision": request.revision or "default",
            "model_source_fingerprint": _model_source_fingerprint(request.model, request.revision),
            "tokenizer": tokenizer_id,
            "tokenizer_revision": request.tokenizer_revision or request.revision or "default",
            "model_config_sha256": _sha256_json(config_dict),
            "input_source": input_source,
            "input_sha256": hashlib.sha256(text.encode("utf-8")).hexdigest(),
            "token_count": token_count,
            "requested_max_length": request.max_length,
            "num_traces": 1,
            "model_type": shape.model_type,
            "num_layers": shape.num_layers,
            "num_attention_heads": shape.num_attention_heads,
            "num_kv_heads": shape.num_kv_heads,
            "head_dim": shape.head_dim,
            "rotary_dim": shape.effective_rotary_dim,
            "attention_layer_indices": list(shape.full_attention_layer_indices),
            "rope_theta": shape.rope_theta,
            "rope_style": "half",
            "rope_type": rope_type,
            "dtype": request.dtype,
            "attn_implementation": request.attn_implementation,
        }
        payload = {"metadata": metadata, "layer_stats": layer_stats}
        reasons = _load_payload(payload).validate(shape)
        if reasons:
            raise ValueError("generated calibration is incompatible: " + "; ".join(reasons))
        return payload
    finally:
        for handle in handles:
            handle.remove()
        del model
        gc.collect()
        _empty_device_cache(request.device, all_devices=request.device_map == "auto")


# --------------------------------------------------------------- artifacts --


def _load_payload(payload: Mapping[str, Any]) -> CalibrationStats:
    """Read a payload back through the safe loader and validator."""
    handle, raw = tempfile.mkstemp(suffix=".pt")
    os.close(handle)
    path = Path(raw)
    try:
        torch.save(dict(payload), path)
        return CalibrationStats.load(path)
    finally:
        path.unlink(missing_ok=True)


def _validate_artifact(path: Path, shape: ModelShape, model_config: Any | None = None) -> None:
    artifact = CalibrationStats.load(path)
    reasons = list(artifact.validate(shape))
    if model_config is not None and artifact.metadata.get("generator") == GENERATOR:
        model = str(model_config.model)
        revision = getattr(model_config, "revision", None)
        expected = {
            "model": model,
            "model_revision": revision or "default",
            "model_source_fingerprint": _model_source_fingerprint(model, revision),
        }
        for key, want in expected.items():
            got = artifact.metadata.get(key)
            if got != want:
                reasons.append(f"calibration {key} {got!r} does not match {want!r}")
    if reasons:
        raise ValueError(f"calibration artifact {path} is incompatible: " + "; ".join(reasons))


def _validate_existing_for_request(path: Path, request: CalibrationRequest) -> None:
    try:
        from transformers import AutoConfig
    except ImportError as error:
        raise RuntimeError("calibration validation requires the Transformers package") from error
    config = AutoConfig.from_pretrained(
        request.model,
        revision=request.revision,
        trust_remote_code=request.trust_remote_code,
        local_files_only=request.local_files_only,
    )
    model_config = type("ModelConfig", (), {"model": request.model, "revision": request.revision})()
    _validate_artifact(path, _model_shape_from_hf_config(config), model_config)


def _atomic_torch_save(payload: Mapping[str, Any], output: Path) -> None:
    """Write next to ``output``, flush to disk, then rename over it."""
    descriptor, raw = tempfile.mkstemp(prefix=f".{output.name}.", suffix=".tmp", dir=output.parent)
    temporary = Path(raw)
    try:
        with os.fdopen(descriptor, "wb") as stream:
            torch.save(dict(payload), stream)
            stream.flush()
            os.fsync(stream.fileno())
        os.replace(temporary, output)
    except Exception:
        with suppress(OSError):
            os.close(descriptor)
        temporary.unlink(missing_ok=True)
        raise


# ------------------------------------------------------------ model walking --


def _find_transformer_backbone(model: torch.nn.Module) -> torch.nn.Module:
    """Breadth-first through ``model`` / ``language_model`` / ``text_model``
    wrappers to the module that holds the decoder ``layers``."""
    queue: list[torch.nn.Module] = [model]
    seen: set[int] = set()
    while queue:
        candidate = queue.pop(0)
        if id(candidate) in seen:
            continue
        seen.add(id(candidate))
        if isinstance(getattr(candidate, "layers", None), torch.nn.ModuleList):
            return candidate
        for name in ("model", "language_model", "text_model"):
            child = getattr(candidate, name, None)
            if isinstance(child, torch.nn.Module):
                queue.append(child)
    raise RuntimeError("cannot locate transformer decoder layers")


def _find_attention_layers(model: torch.nn.Module) -> list[tuple[int, torch.nn.Module]]:
    layers = _find_transformer_backbone(model).layers
    return [
        (index, layer.self_attn)
        for index, layer in enumerate(list(layers))
        if isinstance(getattr(layer, "self_attn", None), torch.nn.Module)
    ]


def _extract_rope_values(
    model: torch.nn.Module,
    attention_layers: Sequence[tuple[int, torch.nn.Module]],
    shape: ModelShape,
    rope_type: str,
) -> dict[int, tuple[torch.Tensor, torch.Tensor]]:
    """(inv_freq [F], freq_scale_sq [1, F]) per layer from the model's rotary
    embedding: the layer's own, else the backbone's shared one."""
    shared = getattr(_find_transformer_backbone(model), "rotary_emb", None)
    freq = shape.effective_rotary_dim // 2
    values: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
    for index, attention in attention_layers:
        rotary = getattr(attention, "rotary_emb", shared)
        inv_freq = getattr(rotary, "inv_freq", None)
        if isinstance(inv_freq, torch.Tensor):
            inv_freq = inv_freq.detach().float().cpu().flatten()
        elif rope_type == "default":
            exponents = torch.arange(0, shape.effective_rotary_dim, 2, dtype=torch.float32)
            inv_freq = 1.0 / (shape.rope_theta ** (exponents / shape.effective_rotary_dim))
        else:
            raise RuntimeError(f"scaled RoPE layer {index} does not expose exact inv_freq")
        if inv_freq.numel() != freq:
            raise RuntimeError(f"layer {index} inv_freq has {inv_freq.numel()} values; expected {freq}")
        scale = torch.as_tensor(getattr(rotary, "attention_scaling", 1.0), dtype=torch.float32).cpu().flatten()
        if scale.numel() == 1:
            scale = scale.expand(freq)
        elif scale.numel() in {shape.head_dim, shape.effective_rotary_dim}:
            scale = scale[:freq]
        elif scale.numel() != freq:
            raise RuntimeError(f"layer {index} attention scaling has {scale.numel()} values")
        values[index] = (inv_freq.contiguous(), scale.square().unsqueeze(0).contiguous())
    return values


def _model_shape_from_hf_config(config: Any) -> ModelShape:
    holder = type("ModelConfig", (), {"hf_text_config": getattr(config, "text_config", config)})()
    return model_shape_from_config(holder)


def _rope_type(config: Any) -> str:
    config = getattr(config, "text_config", config)
    parameters = getattr(config, "rope_parameters", None)
    raw = parameters if isinstance(parameters, Mapping) else getattr(config, "rope_scaling", None)
    if isinstance(raw, Mapping):
        return str(raw.get("rope_type", raw.get("type", "default")) or "default")
    return "default"


# ------------------------------------------------------------------ inputs --


def _load_calibration_text(request: CalibrationRequest) -> tuple[str, str]:
    """(text, input_source): the request's file, or the built-in text repeated
    to about six characters per requested token."""
    if request.input_path is not None:
        path = request.input_path.expanduser().resolve()
        if not path.is_file():
            raise ValueError(f"calibration input file does not exist: {path}")
        text = path.read_text(encoding="utf-8")
        if not text.strip():
            raise ValueError(f"calibration input file is empty: {path}")
        return text, str(path)
    target = request.max_length * 6
    blocks: list[str] = []
    length = 0
    round_index = 0
    while length < target:
        round_index += 1
        for section_index, section in enumerate(_BUILTIN_SECTIONS, 1):
            block = f"Part {round_index}.{section_index}\n{section}\n"
            blocks.append(block)
            length += len(block)
    return "\n".join(blocks), BUILTIN_INPUT_SOURCE


def _prepare_device(device: str) -> None:
    if str(device).startswith("npu"):
        raise RuntimeError("calibration runs on HIP devices ('cuda' in torch); 'npu' is not available")


def _empty_device_cache(device: str, *, all_devices: bool = False) -> None:
    if not torch.cuda.is_available():
        return
    current = torch.cuda.current_device()
    indices = range(torch.cuda.device_count()) if all_devices else (current,)
    for index in indices:
        with torch.cuda.device(index):
            torch.cuda.empty_cache()


def _dtype_name(value: Any) -> str:
    name = str(value).replace("torch.", "").lower()
    return {"half": "float16", "float": "float32", "auto": "bfloat16"}.get(name, name)


def _torch_dtype(value: str) -> torch.dtype:
    choices = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
    try:
        return choices[_dtype_name(value)]
    except KeyError as error:
        raise ValueError(f"unsupported calibration dtype: {value}") from error


def _sha256_json(value: Any) -> str:
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), default=str)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def _model_source_fingerprint(model: str, revision: str | None) -> str:
    """Identity of the model source: a local checkpoint directory by its file
    manifest (names, sizes, modification times; weights are not re-read), any
    other model id by id and revision.  Same format as pkg/calibration.py:530-552,
    so artifacts validate on either side."""
    path = Path(model).expanduser()
    if not path.is_dir():
        return "identifier:" + hashlib.sha256(f"{model}@{revision or 'default'}".encode()).hexdigest()
    patterns = ("*.safetensors", "*.bin", "*.pt", "*.index.json", "config.json")
    files = sorted({p for pattern in patterns for p in path.glob(pattern) if p.is_file()})
    if not files:
        raise ValueError(f"model directory contains no recognized checkpoint files: {path}")
    entries = [(str(p.relative_to(path)), int(p.stat().st_size), int(p.stat().st_mtime_ns)) for p in files]
    return "local-manifest:" + _sha256_json(entries)


# --------------------------------------------------------------------- CLI --


def _build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(description="Generate model-matched TriAttention calibration statistics.")
    parser.add_argument("--model", required=True)
    parser.add_argument("--output", required=True, type=Path)
    parser.add_argument("--input", dest="input_path", type=Path)
    parser.add_argument("--tokenizer")
    parser.add_argument("--revision")
    parser.add_argument("--tokenizer-revision")
    parser.add_argument("--max-length", type=int, default=4096)
    parser.add_argument("--device", default="cuda")
    parser.add_argument(
        "--device-map", choices=("auto",), help="Distribute a large temporary calibration model across visible devices."
    )
    parser.add_argument("--dtype", choices=("float16", "bfloat16", "float32"), default="bfloat16")
    parser.add_argument("--attn-implementation", choices=("eager", "sdpa", "flash_attention_2"), default="eager")
    parser.add_argument("--trust-remote-code", action="store_true")
    parser.add_argument("--local-files-only", action="store_true")
    parser.add_argument("--force", action="store_true")
    return parser


def main(argv: Sequence[str] | None = None) -> int:
    args = _build_parser().parse_args(argv)
    request = CalibrationRequest(
        model=args.model,
        output=args.output,
        input_path=args.input_path,
        tokenizer=args.tokenizer,
        revision=args.revision,
        tokenizer_revision=args.tokenizer_revision,
        trust_remote_code=args.trust_remote_code,
        local_files_only=args.local_files_only,
        max_length=args.max_length,
        device=args.device,
        device_map=args.device_map,
        dtype=args.dtype,
        attn_implementation=args.attn_implementation,
        force=args.force,
    )
    generated = generate_calibration_artifact(request)
    print(f"{'generated' if generated else 'reused'} calibration artifact: {args.output}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
