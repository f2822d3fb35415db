"""Host-side contracts of the method boundary (no GPU): options, registry,
calibration loading, cache validation and the C-ABI library's exports."""

from __future__ import annotations

import re
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from kvcompress_mi355x.methods.base import (
    CompressionRequest,
    CompressionResult,
    KVCompressionMethod,
    LayerCache,
    MethodRuntimeSpec,
    ModelShape,
)
from kvcompress_mi355x.methods.registry import MethodRegistry
from kvcompress_mi355x.methods.triattention import TriAttentionConfig
from kvcompress_mi355x.methods.triattention import method as tri_method
from kvcompress_mi355x.methods.triattention.stats import CalibrationStats, LayerCalibrationStats

REPO = Path(__file__).resolve().parents[1]


# ----------------------------------------------------------------- config --


def test_config_accepts_documented_values() -> None:
    config = TriAttentionConfig.from_method_config(
        {
            "stats_path": "/tmp/stats.pt",
            "kv_budget": 2048,
            "recompute_window": 128,
            "position_policy": "v3",
            "protected_prefix_window": 128,
            "protected_recent_window": 64,
            "position_segments": 8,
            "score_aggregation": "max",
            "layer_aggregation": "mean",
            "score_chunk_size": 512,
            "score_layer_stride": 8,
            "min_output_tokens_for_compression": 64,
            "auto_calibrate": True,
            "calibration_input_path": "/tmp/calibration.txt",
            "calibration_max_length": 8192,
            "calibration_device": "cuda:0",
            "calibration_attn_implementation": "eager",
            "calibration_local_files_only": True,
        }
    )
    assert config.stats_path == Path("/tmp/stats.pt")
    assert config.compression_threshold_tokens == 2176
    assert config.position_policy == "v3" and config.protected_prefix_window == 128
    assert config.calibration_input_path == Path("/tmp/calibration.txt")


@pytest.mark.parametrize(
    ("option", "value"),
    [
        ("kv_budget", 2000),
        ("recompute_window", 0),
        ("score_chunk_size", 129),
        ("score_layer_stride", 0),
        ("min_output_tokens_for_compression", -1),
        ("protected_prefix_window", -1),
        ("protected_recent_window", -1),
        ("position_segments", 0),
        ("position_policy", "unknown"),
        ("score_aggregation", "median"),
        ("auto_calibrate", 1),
        ("calibration_max_length", 127),
        ("calibration_attn_implementation", "unknown"),
        ("kv_budget", True),
    ],
)
def test_config_rejects_invalid_values(option: str, value: object) -> None:
    with pytest.raises(ValueError):
        TriAttentionConfig.from_method_config({"stats_path": "/tmp/stats.pt", option: value})


def test_config_rejects_unknown_option_and_windows_over_budget() -> None:
    with pytest.raises(ValueError, match="unknown"):
        TriAttentionConfig.from_method_config({"stats_path": "/tmp/stats.pt", "typo": 1})
    with pytest.raises(ValueError):
        TriAttentionConfig.from_method_config(
            {"stats_path": "/tmp/s.pt", "kv_budget": 256, "protected_prefix_window": 200, "protected_recent_window": 100}
        )


# --------------------------------------------------------------- registry --


class _Method(KVCompressionMethod):
    @property
    def name(self) -> str:
        return "test_method"

    @property
    def runtime_spec(self) -> MethodRuntimeSpec:
        return MethodRuntimeSpec(True, 256, 128, 128)

    def compatibility_reasons(self, worker: object) -> tuple[str, ...]:
        return ()

    def bind_model_runner(self, runner: object, layer_caches: tuple[LayerCache, ...]) -> None:
        return None

    def compress(self, request: CompressionRequest) -> CompressionResult:
        return CompressionResult(physical_num_tokens=128)


def _shape() -> ModelShape:
    return ModelShape("qwen2", 1, 1, 1, 128, 10_000.0, False)


def test_registry_creates_and_rejects() -> None:
    registry = MethodRegistry()
    registry.register("test_method", lambda o, c, s: _Method())
    method = registry.create("test_method", {}, SimpleNamespace(), _shape())
    assert isinstance(method, _Method) and method.query_window_tokens == 0
    assert registry.names() == ("test_method",)
    with pytest.raises(ValueError, match="already registered"):
        registry.register("test_method", lambda o, c, s: _Method())
    with pytest.raises(ValueError, match="available: test_method"):
        registry.create("missing", {}, SimpleNamespace(), _shape())
    registry.register("broken", lambda o, c, s: object())  # type: ignore[arg-type,return-value]
    with pytest.raises(TypeError, match="expected KVCompressionMethod"):
        registry.create("broken", {}, SimpleNamespace(), _shape())
    registry.register("renamed", lambda o, c, s: _Method())
    with pytest.raises(ValueError, match="returned method named"):
        registry.create("renamed", {}, SimpleNamespace(), _shape())


def test_registry_names_and_origins() -> None:
    from kvcompress_mi355x.methods.registry import canonical_method_name

    registry = MethodRegistry()
    registry.register("  Test_Method ", lambda o, c, s: _Method())
    registry.register("other-method", lambda o, c, s: _Method(), origin="entry point pkg.mod:factory")
    assert registry.names() == ("other-method", "test_method")
    assert registry.origin("TEST_METHOD") == "in-process"
    assert registry.origin("other-method") == "entry point pkg.mod:factory"
    assert canonical_method_name("Tri-Attention_2") == "tri-attention_2"
    for bad in ("", "  ", None, 3):
        with pytest.raises(ValueError, match="non-empty string"):
            canonical_method_name(bad)
    for bad in ("-", "_-", "tri attention", "tri.attention"):
        with pytest.raises(ValueError, match="only letters, digits"):
            canonical_method_name(bad)
    with pytest.raises(TypeError, match="must be callable"):
        registry.register("not_callable", 5)  # type: ignore[arg-type]


def test_builtin_method_registered_and_api_version() -> None:
    import kvcompress_mi355x

    assert "triattention" in kvcompress_mi355x.available_methods()
    assert kvcompress_mi355x.METHOD_API_VERSION == 1


def test_scoring_layer_sample_kats() -> None:
    """The reference's layer-sample cases (tests/test_selection.py:283-366):
    five layers at stride 2 score layers 0, 2, 4; six layers score the same
    three (the last layer is not added)."""
    assert tri_method.scoring_layer_indices(5, 2) == (0, 2, 4)
    assert tri_method.scoring_layer_indices(6, 2) == (0, 2, 4)
    assert tri_method.scoring_layer_indices(48, 8) == (0, 8, 16, 24, 32, 40)
    assert tri_method.scoring_layer_indices(3, 1) == (0, 1, 2)
    with pytest.raises(ValueError):
        tri_method.scoring_layer_indices(4, 0)


def test_mtp_layer_names_and_gqa_width() -> None:
    assert tri_method.is_mtp_cache_layer("mtp.layers.0.self_attn.attn")
    assert tri_method.is_mtp_cache_layer("draft_model.mtp.layers.1.self_attn.attn")
    assert not tri_method.is_mtp_cache_layer("language_model.model.layers.3.self_attn.attn")
    shape = ModelShape("qwen3_5_moe_text", 40, 16, 2, 256, 1e7, False, 64, tuple(range(3, 40, 4)))
    assert tri_method.queries_per_kv_head(shape) == 8


# ------------------------------------------------------------ calibration --


def _write_flat(path: Path, layers: int = 2, heads: int = 4) -> None:
    stats = {
        f"layer{l:02d}_head{h:02d}": {
            "q_mean_real": torch.full((4,), float(l + h)),
            "q_mean_imag": torch.zeros(4),
            "q_abs_mean": torch.ones(4),
        }
        for l in range(layers)
        for h in range(heads)
    }
    torch.save({"metadata": {"head_dim": 8, "rope_style": "half", "rope_type": "default"}, "stats": stats}, path)


def test_flat_stats_load_and_group(tmp_path: Path) -> None:
    _write_flat(tmp_path / "s.pt")
    cal = CalibrationStats.load(tmp_path / "s.pt")
    model = ModelShape("qwen3", 2, 4, 2, 8, 10000.0, False)
    assert cal.validate(model) == ()
    dev = cal.to_device(model, torch.device("cpu"))
    assert dev[0].q_mean_real.shape == (2, 2, 4) and dev[1].omega.shape == (4,)
    torch.testing.assert_close(dev[1].q_mean_real[1, 0], torch.full((4,), 3.0))


def test_incomplete_heads_fail_closed(tmp_path: Path) -> None:
    _write_flat(tmp_path / "s.pt", layers=1, heads=2)
    payload = torch.load(tmp_path / "s.pt", weights_only=True)
    del payload["stats"]["layer00_head00"]
    torch.save(payload, tmp_path / "s.pt")
    with pytest.raises(ValueError, match="complete and contiguous"):
        CalibrationStats.load(tmp_path / "s.pt")


def test_scaled_rope_needs_exact_stats(tmp_path: Path) -> None:
    _write_flat(tmp_path / "s.pt", layers=1, heads=2)
    reasons = CalibrationStats.load(tmp_path / "s.pt").validate(ModelShape("qwen3", 1, 2, 1, 8, 10000.0, True))
    assert any("inv_freq" in r for r in reasons) and any("freq_scale_sq" in r for r in reasons)


def test_invalid_values_fail_closed() -> None:
    cal = CalibrationStats(
        metadata={"head_dim": 8, "rope_style": "half"},
        layers={
            0: LayerCalibrationStats(
                q_mean_real=torch.tensor([[float("nan"), 0.0, 0.0, 0.0]]),
                q_mean_imag=torch.zeros(1, 4),
                q_abs_mean=torch.tensor([[-1.0, 1.0, 1.0, 1.0]]),
                freq_scale_sq=torch.tensor([[0.0, 1.0, 1.0, 1.0]]),
            )
        },
    )
    reasons = cal.validate(ModelShape("qwen3", 1, 1, 1, 8, 10000.0, False))
    assert any("non-finite" in r for r in reasons)
    assert any("negative" in r for r in reasons)
    assert any("freq_scale_sq must be positive" in r for r in reasons)


def test_partial_rope_stats_and_tp_shard() -> None:
    layer = LayerCalibrationStats(
        q_mean_real=torch.arange(16 * 32, dtype=torch.float32).reshape(16, 32),
        q_mean_imag=torch.zeros(16, 32),
        q_abs_mean=torch.ones(16, 32),
        freq_scale_sq=torch.ones(1, 32),
        inv_freq=torch.ones(32),
        q_pass_mean=torch.ones(16, 192),
    )
    cal = CalibrationStats(
        metadata={"model_type": "qwen3_5_moe_text", "num_layers": 8, "head_dim": 256, "rotary_dim": 64,
                  "attention_layer_indices": [3, 7], "rope_style": "half"},
        layers={3: layer, 7: layer},
    )
    model = ModelShape("qwen3_5_moe_text", 8, 16, 2, 256, 1e7, False, 64, (3, 7))
    assert cal.validate(model) == ()
    dev = cal.to_device(model, torch.device("cpu"))
    assert set(dev) == {3, 7} and dev[3].q_mean_real.shape == (2, 8, 32) and dev[3].q_pass_mean.shape == (2, 8, 192)
    r0 = cal.to_device(model, torch.device("cpu"), tensor_parallel_rank=0, tensor_parallel_size=2)[3]
    r1 = cal.to_device(model, torch.device("cpu"), tensor_parallel_rank=1, tensor_parallel_size=2)[3]
    assert r0.q_mean_real.shape == (1, 8, 32) and not torch.equal(r0.q_mean_real, r1.q_mean_real)


def test_kv_head_stats_expand_across_group() -> None:
    cal = CalibrationStats(
        metadata={"head_dim": 8, "rope_style": "half"},
        layers={0: LayerCalibrationStats(torch.tensor([[1.0, 2, 3, 4], [5, 6, 7, 8]]), torch.zeros(2, 4), torch.ones(2, 4), torch.full((2, 4), 4.0))},
    )
    model = ModelShape("qwen3", 1, 4, 2, 8, 10000.0, False)
    assert cal.validate(model) == ()
    g = cal.to_device(model, torch.device("cpu"))[0]
    torch.testing.assert_close(g.q_mean_real[0, 0], g.q_mean_real[0, 1])
    torch.testing.assert_close(g.freq_scale_sq, torch.full((2, 2, 4), 4.0))


# --------------------------------------------------------- device checks --


def test_product_path_rejects_host_tensors() -> None:
    from kvcompress_mi355x.methods.triattention import selection

    with pytest.raises(ValueError, match="HIP device"):
        selection.select_keep_indices(torch.zeros(10), budget=4, protected_prefix=0, protected_recent=0, segments=1, policy="global")


def test_cache_validation_matches_reference_contract() -> None:
    from kvcompress_mi355x.methods.triattention import _device as dev

    with pytest.raises(ValueError):
        dev.validate_cache(torch.zeros(2, 128, 1, 8), "k")  # host tensor


@pytest.mark.parametrize("pad, accepted", [(0, True), (8, True), (64, True), (4, False), (2, False), (12, False)])
def test_page_stride_must_keep_16_byte_pages(pad: int, accepted: bool) -> None:
    """The scorers read 16-byte words: K/V views of a shared buffer pass when
    the per-page padding is a multiple of 8 bf16 elements and are refused
    with a clear error otherwise (the reference accepts any stride of at least
    one page, pkg/provider.py:1224-1230; tests/test_cache.py:50-94 pads 4)."""
    from kvcompress_mi355x.methods.triattention import _device as dev

    kv, dim, pages = 2, 64, 3
    page = 128 * kv * dim
    stride = 2 * page + pad
    raw = torch.zeros(pages * stride + 64, dtype=torch.bfloat16)
    offset = (-raw.data_ptr() // 2) % 8  # a 16-byte aligned start inside the allocation
    shape, strides = (pages, 128, kv, dim), (stride, kv * dim, dim, 1)
    k = torch.as_strided(raw, shape, strides, offset)
    v = torch.as_strided(raw, shape, strides, offset + page)
    for view in (k, v):
        if accepted:
            dev.require_16_byte_pages(view, "k_cache")
        else:
            with pytest.raises(ValueError, match="multiples of 16 bytes"):
                dev.require_16_byte_pages(view, "k_cache")
    misaligned = torch.as_strided(raw, shape, (2 * page, kv * dim, dim, 1), offset + 1)
    with pytest.raises(ValueError, match="16 bytes"):
        dev.require_16_byte_pages(misaligned, "k_cache")


class _FakeTensor:
    def __init__(self, key):
        self.key = key
        self.device = "dev0"
        self.recorded = []

    def record_stream(self, stream):
        self.recorded.append(stream)


def test_descriptor_cache_pins_captured_entries_and_records_streams() -> None:
    """One-sequence descriptors: least-recently-used eviction outside graph
    capture, entries made or used during capture never evicted, and a
    descriptor used on another stream than its allocation's recorded there."""
    from kvcompress_mi355x.methods.triattention._device import DescriptorCache

    state = {"capturing": False, "stream": "s0"}
    made = []

    def make(key):
        made.append(key)
        return _FakeTensor(key)

    cache = DescriptorCache(maxsize=2, make=make, capturing=lambda: state["capturing"],
                            current_stream=lambda device: state["stream"])
    a = cache.get(("a",))
    assert cache.get(("a",)) is a and made == [("a",)]
    state["capturing"] = True
    cap = cache.get(("captured",))
    assert cache.pinned(("captured",))
    state["capturing"] = False
    for i in range(10):
        cache.get((i,))
    assert cache.get(("captured",)) is cap  # never evicted
    assert made.count(("captured",)) == 1
    assert cache.get(("a",)) is not a  # evicted and made again
    # An entry used (not made) during capture is pinned too.
    state["capturing"] = True
    cache.get((9,))
    state["capturing"] = False
    for i in range(20, 30):
        cache.get((i,))
    assert cache.pinned((9,)) and made.count((9,)) == 1
    # Use on another stream records the descriptor there.
    state["stream"] = "s1"
    t = cache.get(("captured",))
    assert t.recorded == ["s1"]
    state["stream"] = "s0"
    cache.get(("captured",))
    assert t.recorded == ["s1"]


# ------------------------------------------------------------------ C ABI --


def test_library_exports_every_header_symbol() -> None:
    from kvcompress_mi355x import _native

    header = (REPO / "include" / "kvcompress_mi355x.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(kvc_\w+)\s*\(", header, flags=re.M))
    assert declared, "no declarations parsed from the header"
    assert declared == set(_native.SIGNATURES), "binding table and header disagree"
    lib = _native.load()
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.kvc_abi_version() == _native.ABI_VERSION


def test_workspace_query_and_argument_validation_without_gpu() -> None:
    from kvcompress_mi355x import _native

    lib = _native.load()
    assert lib.kvc_score_workspace_bytes(6, 8, 128, 128, 5, 16, 16384) > 0
    assert lib.kvc_score_workspace_bytes(1, 2, 8, 8, 2, 1, 10) == 0  # rotary 8 is not a multiple of 16
    assert lib.kvc_score_workspace_bytes(1, 2, 128, 128, 9, 1, 10) == 0  # qpk > 8
    with pytest.raises(ValueError, match="budget"):
        _native.call("kvc_select_keep", None, 1, 10, None, None, None, 20, 0, 0, 1, 0, None, 20)
    with pytest.raises(ValueError):
        _native.call("kvc_compact", None, 1, None, None, 10, 16, 8, 2, 1, None, None, None, None, None, None, 4, 4, None, 0, 0)
    with pytest.raises(ValueError, match="layer order"):
        _native.call("kvc_compact", None, 1, None, None, 10, 16, 8, 2, 1, None, None, None, None, None, None, 4, 4, None, 0, 7)


def test_max_scorer_queries_and_validation_without_gpu() -> None:
    """kvc_score_paged_max: workspace at least the mean scorer's (kvc_head_stats
    reads its partial sums in place), and its argument checks, which run
    before anything touches a device."""
    from kvcompress_mi355x import _native

    lib = _native.load()
    shape = (6, 8, 128, 128, 5, 16, 16384)
    mean_ws = lib.kvc_score_workspace_bytes(*shape)
    assert lib.kvc_score_max_workspace_bytes(*shape, 16) > mean_ws
    assert lib.kvc_score_max_workspace_bytes(*shape, 18) > lib.kvc_score_max_workspace_bytes(*shape, 16)
    assert lib.kvc_score_max_workspace_bytes(*shape, 0) == 0
    fake = 4096  # non-null placeholders; every check below fails before a dereference
    ws = lib.kvc_score_max_workspace_bytes(*shape, 33)

    def call(n_offsets, head_dim=128, rotary=128, dtype=0, workspace_bytes=ws, kv=8):
        return lib.kvc_score_paged_max(
            None, dtype, 6, fake, 100, 128 * kv * head_dim, kv, head_dim, rotary, 5, 0, 16, 16384, fake, fake, fake,
            fake, fake, fake, fake, fake, fake, fake, fake, n_offsets, 0, fake, 0, 1, 16384, fake, workspace_bytes,
        )

    assert call(0) == _native.EINVAL
    assert "n_offsets" in lib.kvc_last_error().decode()
    assert call(33) == _native.EINVAL
    assert "32 offsets" in lib.kvc_last_error().decode()
    # The vector-ALU path keeps every offset's weights of one query head in LDS:
    # 32 offsets x 256 frequencies do not fit.
    big = lib.kvc_score_max_workspace_bytes(6, 1, 512, 512, 5, 16, 16384, 32)
    assert call(32, head_dim=512, rotary=512, kv=1, workspace_bytes=big) == _native.EINVAL
    assert "LDS" in lib.kvc_last_error().decode()
    assert call(16, dtype=2) == _native.EINVAL  # float32 caches are not scored
    assert call(16, workspace_bytes=mean_ws) == _native.EINVAL
    assert "workspace too small" in lib.kvc_last_error().decode()


def test_max_scorer_rejects_oversized_fold_before_launch() -> None:
    """A bf16 shape whose per-offset weight fold would need more work-items than
    one dispatch holds (8192 sequences x 64 layers x 8 KV heads x 5 query heads:
    one 256-thread workgroup per column, 5.4e9 fold threads) is rejected with
    KVC_EINVAL by the host check, which runs before any launch."""
    import torch

    from kvcompress_mi355x import _native

    if torch.cuda.is_available():
        pytest.skip("placeholder pointers: run where no device could be reached by a launch")
    lib = _native.load()
    n_layers, kv, head_dim, qpk, n_seq, max_len, n_off = 64, 8, 128, 5, 8192, 256, 32
    ws = lib.kvc_score_max_workspace_bytes(n_layers, kv, head_dim, head_dim, qpk, n_seq, max_len, n_off)
    assert ws > 0
    fake = 4096
    rc = lib.kvc_score_paged_max(
        None, 0, n_layers, fake, 100, 128 * kv * head_dim, kv, head_dim, head_dim, qpk, 0, n_seq, max_len, fake,
        fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, n_off, 0, fake, 0, 1, 256, fake, ws,
    )
    assert rc == _native.EINVAL
    assert "exceed one dispatch" in lib.kvc_last_error().decode()


def test_raw_layout_names_the_scorer_without_gpu() -> None:
    """Matrix-core shapes (bf16 or fp16, half or interleaved RoPE, head_dim and
    F multiples of 32, qpk <= 8) get head-major raw scores; the rest token-major."""
    from kvcompress_mi355x import _native

    lib = _native.load()
    bf16, fp16 = 0, 1
    half, interleaved = 0, 1
    head, token = _native.RAW_HEAD_MAJOR, _native.RAW_TOKEN_MAJOR
    cases = [
        ((bf16, half, 8, 128, 128, 5), head),
        ((fp16, half, 8, 128, 128, 5), head),
        ((bf16, interleaved, 8, 128, 128, 5), head),
        ((fp16, interleaved, 2, 256, 64, 8), head),
        ((bf16, half, 4, 128, 32, 4), token),  # F = 16
        ((fp16, interleaved, 2, 96, 96, 6), token),  # F = 48
    ]
    for args, want in cases:
        assert lib.kvc_score_raw_layout(*args) == want, args
    assert lib.kvc_score_raw_layout(7, half, 8, 128, 128, 5) < 0  # unknown dtype


def test_backward_compatible_config_alias():
    # tri/method.py:518-519, exported at tri/__init__.py:7,15.
    from kvcompress_mi355x.methods import triattention

    assert triattention.TriAttentionAscendConfig is TriAttentionConfig
    assert "TriAttentionAscendConfig" in triattention.__all__


class _FakeEvent:
    """Stands in for a HIP event: done when the test says so, with a set time."""

    def __init__(self, clock):
        self.clock = clock
        self.t = None

    def record(self):
        self.t = self.clock["now"]

    def query(self):
        return self.clock["done"]

    def elapsed_time(self, other):
        return other.t - self.t


def _drive_choice(times_ms, rows=100, done=True):
    """Run CompactionFormChoice through its schedule with fake events; each
    call of form f takes times_ms[f][k] for its k-th timed run."""
    from kvcompress_mi355x.methods.triattention.pipeline import CompactionFormChoice

    clock = {"now": 0.0, "done": done}
    choice = CompactionFormChoice(event_factory=lambda: _FakeEvent(clock), capturing=lambda: False)
    forms, count = [], {"layer_major": 0, "interleaved": 0}
    for _ in range(len(CompactionFormChoice.SCHEDULE) + 2):
        form, marks = choice.next_call()
        forms.append((form, marks is not None))
        if marks is not None:
            marks[0].record()
            clock["now"] += times_ms[form][count[form]]
            count[form] += 1
            marks[1].record()
            choice.timed(form, marks, rows)
    return choice, forms


def test_compaction_form_schedule_and_margin():
    choice, forms = _drive_choice({"layer_major": [4.45, 4.46], "interleaved": [4.30, 4.25]})
    assert forms[:6] == [("layer_major", False), ("interleaved", False), ("layer_major", True), ("interleaved", True),
                         ("layer_major", True), ("interleaved", True)]
    assert choice.chosen == "interleaved"  # 4.25 < 0.99 * 4.45
    assert forms[6:] == [("interleaved", False), ("interleaved", False)]
    assert choice.per_row_ms == {"layer_major": 4.45 / 100, "interleaved": 4.25 / 100}


def test_compaction_form_keeps_planned_inside_margin_and_when_slower():
    assert _drive_choice({"layer_major": [4.45, 4.46], "interleaved": [4.42, 4.43]})[0].chosen == "layer_major"
    # 1.6% faster (a placement seen on the Qwen2.5-14B pool) is past the margin.
    assert _drive_choice({"layer_major": [4.38, 4.40], "interleaved": [4.31, 4.32]})[0].chosen == "interleaved"
    assert _drive_choice({"layer_major": [4.45, 4.46], "interleaved": [5.07, 5.08]})[0].chosen == "layer_major"
    # A slow first timed trial does not decide: the faster of each form's two counts.
    assert _drive_choice({"layer_major": [6.0, 4.45], "interleaved": [4.25, 7.0]})[0].chosen == "interleaved"


def test_compaction_form_fixed_order_skips_trials(monkeypatch):
    from kvcompress_mi355x.methods.triattention.pipeline import CompactionFormChoice

    choice = CompactionFormChoice(event_factory=lambda: None, capturing=lambda: False, fixed="interleaved")
    assert [choice.next_call() for _ in range(3)] == [("interleaved", None)] * 3
    with pytest.raises(ValueError, match="unknown compaction layer order"):
        CompactionFormChoice(fixed="sideways")
    monkeypatch.delenv(tri_method.COMPACTION_ORDER_ENV, raising=False)
    assert tri_method.compaction_order_setting() == "auto"
    monkeypatch.setenv(tri_method.COMPACTION_ORDER_ENV, "layer_major")
    assert tri_method.compaction_order_setting() == "layer_major"
    monkeypatch.setenv(tri_method.COMPACTION_ORDER_ENV, "fastest")
    with pytest.raises(ValueError, match="must be one of auto, layer_major, interleaved"):
        tri_method.compaction_order_setting()


def test_compaction_form_waits_for_events_and_capture():
    from kvcompress_mi355x.methods.triattention.pipeline import CompactionFormChoice

    choice, forms = _drive_choice({"layer_major": [4.45, 4.46], "interleaved": [4.0, 4.0]}, done=False)
    # Trials still in flight: the planned form runs outside the schedule.
    assert choice.chosen is None and forms[6:] == [("layer_major", False), ("layer_major", False)]
    # settle() decides from whatever has completed, the planned form if nothing has.
    choice.settle()
    assert choice.chosen == "layer_major"
    captured = CompactionFormChoice(event_factory=lambda: None, capturing=lambda: True)
    assert captured.next_call() == ("layer_major", None) and captured._next == 0
