"""Model-matched TriAttention calibration artifacts, accumulated on the GPU.

The TriAttention scorer needs, per full-attention layer and query head, the
mean pre-RoPE query of a calibration run (real and imaginary parts per RoPE
frequency, the mean magnitude per frequency, the mean of the unrotated dims)
and the rotary frequencies the model itself uses.  This module produces that
artifact from a Hugging Face checkpoint.

How a generation runs (generate_calibration_artifact):

  _OutputLock      exclusive lock on ".<name>.lock" beside the output, so the
                   workers of one deployment that all find the artifact
                   missing produce it once; a worker that gets the lock after
                   the file appeared checks it against its request instead.
  _Checkpoint      the checkpoint's Hugging Face config, tokenizer and model
                   (for a multimodal Qwen3.5 checkpoint the causal text model
                   alone, its weights remapped from model.language_model.*).
  _DecoderView     the decoder stack inside the loaded model: each
                   full-attention layer's query module (q_norm where the layer
                   normalises queries, else q_proj) and its rotary embedding.
  _QueryCapture    forward hooks that hand every query output to the layer's
                   LayerAccumulator; one kvc_qstats_accumulate launch per
                   output sums it into a float64 state on the HIP device.
  _artifact        means, rotary tables and provenance metadata as a schema-3
                   payload, read back through CalibrationStats' safe loader
                   and validator, then written beside the output and renamed
                   over it (readers never see a partial file).

Kept identical to the reference generator (pkg/calibration.py) because other
tools read or write the same files: the CalibrationRequest fields, the
command-line flags, the schema-3 layout and metadata keys, and the
model-source fingerprint ("identifier:" + SHA-256 of "<model>@<revision>", or
"local-manifest:" + SHA-256 of the checkpoint directory's file manifest), so an
artifact validates on either side.  Artifacts name the reference's
generator ("generator": "vllm-ascend-kvcompress-hust"), because the
reference's loader holds an artifact to its recorded model source only under
that name (pkg/calibration.py:426-452); this package is recorded under
"producer" / "producer_version".  The model-source provenance check here
applies to either generator name.  The built-in calibration text is this
package's own (input_source "builtin:mi355x-systems-v1").
"""

from __future__ import annotations

import argparse
import fcntl
import fnmatch
import gc
import hashlib
import importlib.util
import json
import os
import tempfile
from collections.abc import Iterator, Mapping, Sequence
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

# The software that wrote an artifact ("producer") and the generator name its
# metadata carries: the reference's, so that its loader checks provenance.
GENERATOR = "kvcompress-mi355x"
REFERENCE_GENERATOR = "vllm-ascend-kvcompress-hust"
# Generators whose artifacts record the model source they were made from.
PROVENANCE_GENERATORS = frozenset({GENERATOR, REFERENCE_GENERATOR})
BUILTIN_INPUT_SOURCE = "builtin:mi355x-systems-v1"
SCHEMA_VERSION = 3
MIN_MAX_LENGTH = 128

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

# Checkpoint files that identify a local model directory (top level only).
_MANIFEST_PATTERNS = ("*.safetensors", "*.bin", "*.pt", "*.index.json", "config.json")

_TORCH_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
_DTYPE_ALIASES = {"half": "float16", "float": "float32", "auto": "bfloat16"}


def dtype_name(value: Any) -> str:
    """Canonical dtype name of a torch dtype or a dtype string ("torch.float16",
    "half", "auto" -> "float16", "float16", "bfloat16")."""
    name = str(value).lower().removeprefix("torch.")
    return _DTYPE_ALIASES.get(name, name)


def torch_dtype(value: Any) -> torch.dtype:
    try:
        return _TORCH_DTYPES[dtype_name(value)]
    except KeyError:
        raise ValueError(f"unsupported calibration dtype: {value}") from None


@dataclass(frozen=True)
class CalibrationRequest:
    """One artifact to generate (the reference's request fields,
    pkg/calibration.py:71-86).  ``device`` is where the temporary model runs
    ("cuda", "cuda:N" or "cpu"); the statistics are always accumulated on a
    HIP device."""

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

    @classmethod
    def for_runner(cls, runner: Any, config: TriAttentionConfig) -> CalibrationRequest:
        """The request a serving worker makes for its own model: the model
        config's identity and dtype, the method's calibration options, the
        worker's device (calibration_device "auto"), and a model spread over
        the visible devices when the deployment is tensor parallel (the
        checkpoint then does not fit one device either)."""
        mc = runner.model_config
        device = config.calibration_device
        if device == "auto":
            device = str(getattr(runner, "device", "cuda"))
        parallel = getattr(getattr(runner, "vllm_config", None), "parallel_config", None)
        tp = int(getattr(parallel, "tensor_parallel_size", 1))
        return cls(
            model=str(mc.model),
            output=config.stats_path,
            input_path=config.calibration_input_path,
            tokenizer=str(mc.tokenizer) if mc.tokenizer else None,
            revision=getattr(mc, "revision", None),
            tokenizer_revision=getattr(mc, "tokenizer_revision", None),
            trust_remote_code=bool(getattr(mc, "trust_remote_code", False)),
            local_files_only=config.calibration_local_files_only,
            max_length=config.calibration_max_length,
            device=device,
            device_map="auto" if tp > 1 else None,
            dtype=dtype_name(getattr(mc, "dtype", "bfloat16")),
            attn_implementation=config.calibration_attn_implementation,
        )


# -------------------------------------------------------------- provenance --


def canonical_digest(value: Any) -> str:
    """SHA-256 of the canonical JSON form of ``value`` (sorted keys, no spaces,
    non-JSON values by their str)."""
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), default=str)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def model_source_fingerprint(model: str, revision: str | None) -> str:
    """Identity of a model source.  A model id: "identifier:" + SHA-256 of
    "<id>@<revision or default>".  A local checkpoint directory: its top-level
    checkpoint files (weights, index, config) as (name, size, mtime_ns) in name
    order, "local-manifest:" + their canonical digest; the weights are not
    read."""
    directory = Path(model).expanduser()
    if not directory.is_dir():
        return "identifier:" + hashlib.sha256(f"{model}@{revision or 'default'}".encode()).hexdigest()
    manifest = []
    for entry in sorted(os.scandir(directory), key=lambda e: e.name):
        if entry.is_file() and any(fnmatch.fnmatchcase(entry.name, p) for p in _MANIFEST_PATTERNS):
            info = entry.stat()
            manifest.append((entry.name, int(info.st_size), int(info.st_mtime_ns)))
    if not manifest:
        raise ValueError(f"no checkpoint files (weights, index or config.json) in model directory {directory}")
    return "local-manifest:" + canonical_digest(manifest)


def shape_from_hf_config(hf_config: Any) -> ModelShape:
    """ModelShape of a Hugging Face config (its text config for multimodal ones)."""
    return model_shape_from_config(_HostModelConfig(hf_text_config=getattr(hf_config, "text_config", hf_config)))


@dataclass(frozen=True)
class _HostModelConfig:
    """The parts of a serving host's model config the checks read."""

    hf_text_config: Any = None
    model: str = ""
    revision: str | None = None


def rope_type_of(hf_config: Any) -> str:
    """RoPE type named by rope_parameters (or rope_scaling), "default" if none."""
    text = getattr(hf_config, "text_config", hf_config)
    for entry in (getattr(text, "rope_parameters", None), getattr(text, "rope_scaling", None)):
        if isinstance(entry, Mapping):
            return str(entry.get("rope_type", entry.get("type", "default")) or "default")
    return "default"


# -------------------------------------------------------------------- text --


def calibration_text(request: CalibrationRequest) -> tuple[str, str]:
    """(text, input_source): the request's file, or the built-in sections
    repeated under numbered headings to about six characters per requested
    token (the tokenizer truncates to max_length)."""
    if request.input_path is not None:
        path = request.input_path.expanduser().resolve()
        if not path.is_file():
            raise ValueError(f"calibration input file does not exist: {path}")
        text = path.read_text(encoding="utf-8")
        if not text.strip():
            raise ValueError(f"calibration input file is empty: {path}")
        return text, str(path)
    wanted = 6 * request.max_length
    parts: list[str] = []
    size = 0
    repeat = 0
    while size < wanted:
        repeat += 1
        for number, section in enumerate(_BUILTIN_SECTIONS, 1):
            part = f"Part {repeat}.{number}\n{section}\n"
            parts.append(part)
            size += len(part)
    return "\n".join(parts), BUILTIN_INPUT_SOURCE


# ------------------------------------------------------------ accumulation --


def _hip_device(device: torch.device | str | None) -> torch.device:
    """The HIP device the statistics are accumulated on (the current one when
    the model itself runs elsewhere)."""
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
    """Running query sums of one layer (the reference's _LayerAccumulator,
    pkg/calibration.py:89-131).

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
                f"hooked query output has {projected.shape[-1]} values per row; the attention shape "
                f"({heads} heads x {head_dim}) needs {expected} (or {2 * expected} with an output gate)"
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


# ------------------------------------------------------------------- model --

_WRAPPER_ATTRIBUTES = ("model", "language_model", "text_model")


class _DecoderView:
    """The decoder stack inside a loaded model and its attention layers.

    The stack is the shallowest module holding a ``layers`` ModuleList,
    searched level by level through the usual wrapper attributes (a causal-LM
    head's ``model``, a multimodal model's ``language_model`` / ``text_model``).
    Every layer with a ``self_attn`` module is a full-attention layer; hybrid
    models' linear-attention layers have none."""

    def __init__(self, model: torch.nn.Module) -> None:
        self.stack = self._find_stack(model)
        self.attention = [
            (index, layer.self_attn)
            for index, layer in enumerate(self.stack.layers)
            if isinstance(getattr(layer, "self_attn", None), torch.nn.Module)
        ]

    @staticmethod
    def _find_stack(model: torch.nn.Module) -> torch.nn.Module:
        level: list[torch.nn.Module] = [model]
        visited: set[int] = set()
        while level:
            for module in level:
                if isinstance(getattr(module, "layers", None), torch.nn.ModuleList):
                    return module
            visited.update(id(m) for m in level)
            level = [
                child
                for module in level
                for child in (getattr(module, name, None) for name in _WRAPPER_ATTRIBUTES)
                if isinstance(child, torch.nn.Module) and id(child) not in visited
            ]
        raise RuntimeError("no decoder layer stack found in the calibration model")

    @property
    def layer_indices(self) -> tuple[int, ...]:
        return tuple(index for index, _ in self.attention)

    def query_modules(self) -> Iterator[tuple[int, torch.nn.Module]]:
        """(layer, module whose output is the layer's pre-RoPE query)."""
        for index, attention in self.attention:
            module = next(
                (m for m in (getattr(attention, "q_norm", None), getattr(attention, "q_proj", None))
                 if isinstance(m, torch.nn.Module)),
                None,
            )
            if module is None:
                raise RuntimeError(f"attention layer {index} has neither a q_norm nor a q_proj module to observe")
            yield index, module

    def rotary_tables(self, shape: ModelShape, rope_type: str) -> dict[int, tuple[torch.Tensor, torch.Tensor]]:
        """(inv_freq [F], freq_scale_sq [1, F]) per attention layer from the
        rotary embedding the layer uses (its own, else the stack's shared one):
        its exact inverse frequencies (the theta default for unscaled RoPE
        when the module exposes none) and the square of its attention scaling
        (a scalar, or per frequency, or per dim of which the first F count)."""
        shared = getattr(self.stack, "rotary_emb", None)
        freq = shape.effective_rotary_dim // 2
        tables = {}
        for index, attention in self.attention:
            rotary = getattr(attention, "rotary_emb", shared)
            inv_freq = getattr(rotary, "inv_freq", None)
            if isinstance(inv_freq, torch.Tensor):
                inv_freq = inv_freq.detach().to("cpu", torch.float32).reshape(-1)
            elif rope_type == "default":
                steps = torch.arange(0, shape.effective_rotary_dim, 2, dtype=torch.float32)
                inv_freq = 1.0 / (shape.rope_theta ** (steps / shape.effective_rotary_dim))
            else:
                raise RuntimeError(f"layer {index} uses {rope_type!r} RoPE but exposes no exact inv_freq")
            if inv_freq.numel() != freq:
                raise RuntimeError(f"layer {index} inv_freq has {inv_freq.numel()} values; expected {freq}")
            scaling = torch.as_tensor(getattr(rotary, "attention_scaling", 1.0), dtype=torch.float32).cpu().reshape(-1)
            if scaling.numel() == 1:
                scaling = scaling.repeat(freq)
            elif scaling.numel() in (shape.head_dim, shape.effective_rotary_dim):
                scaling = scaling[:freq]
            elif scaling.numel() != freq:
                raise RuntimeError(f"layer {index} attention scaling has {scaling.numel()} values")
            tables[index] = (inv_freq.contiguous(), scaling.square().reshape(1, freq).contiguous())
        return tables


class _QueryCapture:
    """Forward hooks from every attention layer's query module into that
    layer's LayerAccumulator, removed on exit."""

    def __init__(self, decoder: _DecoderView, shape: ModelShape, device: torch.device) -> None:
        self.decoder = decoder
        self.shape = shape
        self.accumulators = {index: LayerAccumulator(device=device) for index in decoder.layer_indices}
        self._handles: list[Any] = []

    def _hook(self, index: int):
        acc, shape = self.accumulators[index], self.shape

        def observe(_module: torch.nn.Module, _args: tuple[Any, ...], output: Any) -> None:
            if not isinstance(output, torch.Tensor):
                raise RuntimeError(f"query module of attention layer {index} returned {type(output).__name__}, not a tensor")
            acc.add(output, shape.num_attention_heads, shape.head_dim, shape.effective_rotary_dim)

        return observe

    def __enter__(self) -> _QueryCapture:
        for index, module in self.decoder.query_modules():
            self._handles.append(module.register_forward_hook(self._hook(index)))
        return self

    def __exit__(self, *exc: object) -> None:
        while self._handles:
            self._handles.pop().remove()


class _Checkpoint:
    """A request's Hugging Face config, tokenizer and (on demand) model."""

    def __init__(self, request: CalibrationRequest) -> None:
        if request.device_map is not None and importlib.util.find_spec("accelerate") is None:
            raise RuntimeError(
                "device_map='auto' spreads the calibration model with the accelerate package, which this "
                "environment lacks (the package's [calibration] extra provides it)"
            )
        try:
            import transformers
        except ImportError as error:
            raise RuntimeError("calibration generation requires the Transformers package") from error
        if str(request.device).startswith("npu"):
            raise RuntimeError("calibration runs on HIP devices ('cuda' in torch); 'npu' is not available")
        self.request = request
        self.transformers = transformers
        self.loader_options = {"trust_remote_code": request.trust_remote_code, "local_files_only": request.local_files_only}
        self.config = transformers.AutoConfig.from_pretrained(request.model, revision=request.revision, **self.loader_options)
        self.shape = shape_from_hf_config(self.config)
        if self.shape.model_type not in SUPPORTED_MODEL_TYPES:
            raise ValueError(f"model_type {self.shape.model_type!r} is not supported for calibration")
        self.tokenizer_id = request.tokenizer or request.model
        self.tokenizer = transformers.AutoTokenizer.from_pretrained(
            self.tokenizer_id, revision=request.tokenizer_revision or request.revision, **self.loader_options
        )

    @property
    def text_only_multimodal(self) -> bool:
        """A multimodal Qwen3.5 checkpoint, calibrated through its causal text model."""
        text = getattr(self.config, "text_config", self.config)
        return text is not self.config and str(getattr(self.config, "model_type", "")).startswith("qwen3_5")

    def encode(self, text: str) -> dict[str, torch.Tensor]:
        encoded = self.tokenizer(
            text, return_tensors="pt", truncation=True, max_length=self.request.max_length, add_special_tokens=True
        )
        ids = encoded.get("input_ids")
        if not isinstance(ids, torch.Tensor) or ids.ndim != 2:
            raise RuntimeError("the tokenizer returned no [batch, tokens] input_ids tensor")
        if ids.shape[1] < 2:
            raise ValueError("calibration input produced fewer than two tokens")
        return {name: value for name, value in encoded.items() if isinstance(value, torch.Tensor)}

    def load_model(self) -> torch.nn.Module:
        request, tf = self.request, self.transformers
        options: dict[str, Any] = {
            "revision": request.revision,
            "dtype": torch_dtype(request.dtype),
            "device_map": request.device_map or request.device,
            **self.loader_options,
        }
        if request.attn_implementation:
            options["attn_implementation"] = request.attn_implementation
        if self.text_only_multimodal:
            # Text weights sit under model.language_model.* in the multimodal
            # checkpoint; the causal text model expects them under model.*.
            options["config"] = self.config.text_config
            options["key_mapping"] = {r"^model\.language_model\.(.+)$": r"model.\1"}
            model = tf.AutoModelForCausalLM.from_pretrained(request.model, **options)
        else:
            options["config"] = self.config
            model = tf.AutoModel.from_pretrained(request.model, **options)
        return model.eval()


def _release_device_memory(request: CalibrationRequest) -> None:
    if not torch.cuda.is_available():
        return
    devices = range(torch.cuda.device_count()) if request.device_map == "auto" else (torch.cuda.current_device(),)
    for index in devices:
        with torch.cuda.device(index):
            torch.cuda.empty_cache()


def _artifact(request: CalibrationRequest) -> dict[str, Any]:
    """The schema-3 payload of one calibration run over the request's text."""
    checkpoint = _Checkpoint(request)
    shape = checkpoint.shape
    text, input_source = calibration_text(request)
    inputs = checkpoint.encode(text)
    token_count = int(inputs["input_ids"].shape[1])
    input_device = torch.device("cpu" if request.device_map == "auto" else request.device)
    accumulate_on = _hip_device(request.device)
    rope_type = rope_type_of(checkpoint.config)

    model = None
    try:
        model = checkpoint.load_model()
        decoder = _DecoderView(model)
        if decoder.layer_indices != shape.full_attention_layer_indices:
            raise RuntimeError(
                f"the model's attention layers {decoder.layer_indices} differ from the config's full-attention "
                f"layers {shape.full_attention_layer_indices}"
            )
        with _QueryCapture(decoder, shape, accumulate_on) as capture, torch.inference_mode():
            model(**{name: value.to(input_device) for name, value in inputs.items()}, use_cache=False)
        torch.cuda.synchronize(accumulate_on)
        rotary = decoder.rotary_tables(shape, rope_type)
        layer_stats = {}
        for index, acc in capture.accumulators.items():
            if acc.count <= 0:
                raise RuntimeError(f"the forward pass produced no queries for attention layer {index}")
            inv_freq, freq_scale_sq = rotary[index]
            layer_stats[str(index)] = {**acc.means(), "inv_freq": inv_freq, "freq_scale_sq": freq_scale_sq}
    finally:
        del model
        gc.collect()
        _release_device_memory(request)

    hf_dict = checkpoint.config.to_dict() if hasattr(checkpoint.config, "to_dict") else vars(checkpoint.config)
    metadata = {
        # provenance
        "schema_version": SCHEMA_VERSION,
        "generator": REFERENCE_GENERATOR,
        "producer": GENERATOR,
        "producer_version": __version__,
        "accumulator": "kvc_qstats_accumulate (float64 sums, HIP)",
        "transformers_version": checkpoint.transformers.__version__,
        "created_at_utc": datetime.now(timezone.utc).isoformat(),
        "model": request.model,
        "model_revision": request.revision or "default",
        "model_source_fingerprint": model_source_fingerprint(request.model, request.revision),
        "tokenizer": checkpoint.tokenizer_id,
        "tokenizer_revision": request.tokenizer_revision or request.revision or "default",
        "model_config_sha256": canonical_digest(hf_dict),
        # calibration input
        "input_source": input_source,
        "input_sha256": hashlib.sha256(text.encode("utf-8")).hexdigest(),
        "token_count": token_count,
        "requested_max_length": request.max_length,
        "num_traces": 1,
        # model shape the statistics belong to
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
    problems = _round_trip(payload).validate(shape)
    if problems:
        raise ValueError("the generated calibration does not fit its own model: " + "; ".join(problems))
    return payload


# -------------------------------------------------------------- validation --


def _round_trip(payload: Mapping[str, Any]) -> CalibrationStats:
    """The payload as the safe loader reads it back from disk."""
    with tempfile.TemporaryDirectory() as scratch:
        path = Path(scratch) / "payload.pt"
        torch.save(dict(payload), path)
        return CalibrationStats.load(path)


def validate_artifact(path: Path, shape: ModelShape, model_config: Any | None = None) -> None:
    """Raise ValueError unless the artifact at ``path`` fits ``shape`` and, for
    an artifact whose generator records its model source, comes from
    ``model_config``'s model (id, revision and source fingerprint)."""
    artifact = CalibrationStats.load(path)
    problems = list(artifact.validate(shape))
    md = artifact.metadata
    if model_config is not None and md.get("generator") in PROVENANCE_GENERATORS:
        model, revision = str(model_config.model), getattr(model_config, "revision", None)
        for key, want in (
            ("model", model),
            ("model_revision", revision or "default"),
            ("model_source_fingerprint", model_source_fingerprint(model, revision)),
        ):
            if md.get(key) != want:
                problems.append(f"calibration {key} {md.get(key)!r} does not match {want!r}")
    if problems:
        raise ValueError(f"calibration artifact {path} is incompatible: " + "; ".join(problems))


def _validate_for_request(path: Path, request: CalibrationRequest) -> None:
    """Check an artifact another worker published against this request's model."""
    try:
        from transformers import AutoConfig
    except ImportError as error:
        raise RuntimeError("calibration validation requires the Transformers package") from error
    hf_config = AutoConfig.from_pretrained(
        request.model,
        revision=request.revision,
        trust_remote_code=request.trust_remote_code,
        local_files_only=request.local_files_only,
    )
    validate_artifact(path, shape_from_hf_config(hf_config), _HostModelConfig(model=request.model, revision=request.revision))


# --------------------------------------------------------------- publishing --


class _OutputLock:
    """Exclusive flock on ".<output name>.lock" beside the output for the span
    of one generation; ``publish`` writes a payload next to the output, syncs
    it and renames it over the output."""

    def __init__(self, output: Path) -> None:
        self.output = output
        self._lock_file = None

    def __enter__(self) -> _OutputLock:
        self.output.parent.mkdir(parents=True, exist_ok=True)
        self._lock_file = open(self.output.with_name(f".{self.output.name}.lock"), "a+b")  # noqa: SIM115
        fcntl.flock(self._lock_file.fileno(), fcntl.LOCK_EX)
        return self

    def __exit__(self, *exc: object) -> None:
        if self._lock_file is not None:
            fcntl.flock(self._lock_file.fileno(), fcntl.LOCK_UN)
            self._lock_file.close()
            self._lock_file = None

    def publish(self, payload: Mapping[str, Any]) -> None:
        staged = tempfile.NamedTemporaryFile(
            prefix=f".{self.output.name}.", suffix=".tmp", dir=self.output.parent, delete=False
        )
        try:
            with staged:
                torch.save(dict(payload), staged)
                staged.flush()
                os.fsync(staged.fileno())
            os.replace(staged.name, self.output)
        except BaseException:
            Path(staged.name).unlink(missing_ok=True)
            raise


# ------------------------------------------------------------ entry points --


def generate_calibration_artifact(request: CalibrationRequest) -> bool:
    """Generate the request's artifact.  False when the output already exists
    (generated by another worker while this one waited for the lock, or
    before; it is validated against the request) and ``force`` is not set."""
    if request.max_length < MIN_MAX_LENGTH:
        raise ValueError(f"calibration max_length must be at least {MIN_MAX_LENGTH}")
    output = request.output.expanduser().resolve()
    with _OutputLock(output) as lock:
        if output.is_file() and not request.force:
            _validate_for_request(output, request)
            return False
        lock.publish(_artifact(request))
    return True


def ensure_calibration_for_runner(runner: Any, selection: Any) -> bool:
    """Serving-startup hook (called before the serving weights load, so the
    temporary calibration model is gone by then): for a TriAttention selection
    whose statistics file is missing and auto_calibrate is on, generate it for
    the runner's model; an existing file is validated against the model.
    True when this call generated the artifact."""
    if getattr(selection, "method", None) != "triattention":
        return False
    config = TriAttentionConfig.from_method_config(selection.method_config)
    shape = model_shape_from_config(runner.model_config)
    if not config.stats_path.is_file():
        if not config.auto_calibrate:
            return False
        generated = generate_calibration_artifact(CalibrationRequest.for_runner(runner, config))
    else:
        generated = False
    validate_artifact(config.stats_path, shape, runner.model_config)
    return generated


def build_parser() -> argparse.ArgumentParser:
    """Command line of the generator (the reference's flags and defaults, with
    a HIP device by default)."""
    p = argparse.ArgumentParser(description="Generate model-matched TriAttention calibration statistics.")
    p.add_argument("--model", required=True, help="model id or local checkpoint directory")
    p.add_argument("--output", required=True, type=Path, help="artifact path (.pt)")
    p.add_argument("--input", dest="input_path", type=Path, help="calibration text file (default: built-in text)")
    p.add_argument("--tokenizer", help="tokenizer id or directory (default: the model)")
    p.add_argument("--revision")
    p.add_argument("--tokenizer-revision")
    p.add_argument("--max-length", type=int, default=4096, help="calibration tokens (at least 128)")
    p.add_argument("--device", default="cuda", help="where the temporary model runs")
    p.add_argument("--device-map", choices=("auto",), help="spread a large temporary model over the visible devices")
    p.add_argument("--dtype", choices=tuple(_TORCH_DTYPES), default="bfloat16")
    p.add_argument("--attn-implementation", choices=("eager", "sdpa", "flash_attention_2"), default="eager")
    p.add_argument("--trust-remote-code", action="store_true")
    p.add_argument("--local-files-only", action="store_true")
    p.add_argument("--force", action="store_true", help="regenerate even if the output exists")
    return p


def main(argv: Sequence[str] | None = None) -> int:
    args = vars(build_parser().parse_args(argv))
    request = CalibrationRequest(**args)
    generated = generate_calibration_artifact(request)
    print(f"{'generated' if generated else 'reused'} calibration artifact: {request.output}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
