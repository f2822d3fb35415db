"""Seeded synthetic paged caches and calibration for benchmarking and tests.

Shapes follow the TriAttention benchmark configurations: a tiny correctness
case, a Qwen2.5-14B-shaped cache, Qwen3.5-35B-A3B-shaped hybrid layers with
partial RoPE, a long-context in-place compaction stress and a batch of
ragged decode-time sequences.  No model weights are involved: K/V are random
normals and the calibration centres are random complex vectors.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import torch

from .config import KERNEL_BLOCK_SIZE
from .methods.base import ModelShape
from .methods.triattention.stats import CalibrationStats, LayerCalibrationStats


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    n_layers: int
    score_layer_stride: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    rotary_dim: int
    rope_theta: float
    dtype: torch.dtype
    seq_lens: tuple[int, ...]
    budget: int
    recent: int
    prefix: int = 0
    segments: int = 8
    policy: str = "global"
    max_model_len: int = 32768
    inplace: bool = False
    channel_scale_sigma: float = 0.0
    outlier_fraction: float = 0.0
    outlier_scale: float = 8.0
    scheduler_block: int = KERNEL_BLOCK_SIZE
    permute_pages: bool = True
    pool_pages: int | None = None
    model_type: str = "qwen2"
    # "separate": one [pages, 128, kv, D] tensor per layer and K/V;
    # "interleaved": K and V of a layer are views of one buffer whose page i
    # holds K's page, then V's page, then `page_pad` elements of padding (the
    # shared-buffer layout of pkg/provider.py:1201-1230, tests/test_cache.py:50-94).
    kv_layout: str = "separate"
    page_pad: int = 0
    notes: tuple[str, ...] = field(default_factory=tuple)

    @property
    def qpk(self) -> int:
        return self.num_attention_heads // self.num_kv_heads

    @property
    def scoring_layers(self) -> tuple[int, ...]:
        return tuple(range(0, self.n_layers, self.score_layer_stride))

    @property
    def total_tokens(self) -> int:
        return sum(self.seq_lens)

    @property
    def row_bytes(self) -> int:
        return self.num_kv_heads * self.head_dim * 2

    def model_shape(self) -> ModelShape:
        return ModelShape(
            model_type=self.model_type,
            num_layers=self.n_layers,
            num_attention_heads=self.num_attention_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            rope_theta=self.rope_theta,
            has_rope_scaling=False,
            rotary_dim=None if self.rotary_dim == self.head_dim else self.rotary_dim,
        )

    def algorithmic_bytes(self) -> dict[str, int]:
        """Bytes the path must move: K of the scoring layers read once; the
        aggregate written and read once plus the keep indices; kept K and V
        read once and written once in every layer."""
        s = len(self.scoring_layers)
        n = self.total_tokens
        score = s * n * self.row_bytes
        select = n * 4 * 2 + len(self.seq_lens) * self.budget * 8
        compact = self.n_layers * len(self.seq_lens) * self.budget * self.row_bytes * 2 * 2
        return {"score": score, "select": select, "compact": compact, "total": score + select + compact}


def _lognormal_lengths(n: int, median: float, sigma: float, lo: int, hi: int, seed: int) -> tuple[int, ...]:
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(n, generator=g, dtype=torch.float64)
    lengths = torch.exp(math.log(median) + sigma * z).round().clamp(lo, hi).to(torch.int64)
    return tuple(int(x) for x in lengths)


def _uniform_lengths(n: int, lo: int, hi: int, seed: int) -> tuple[int, ...]:
    g = torch.Generator().manual_seed(seed)
    return tuple(int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g))


def config_spec(index: int, **overrides) -> WorkloadSpec:
    """The five benchmark configurations (1-based), optionally overridden."""
    if index == 1:
        spec = WorkloadSpec(
            name="tiny-1x4096-8q2kv-d128",
            n_layers=1,
            score_layer_stride=1,
            num_attention_heads=8,
            num_kv_heads=2,
            head_dim=128,
            rotary_dim=128,
            rope_theta=1e6,
            dtype=torch.bfloat16,
            seq_lens=(4096,),
            budget=2048,
            recent=128,
            permute_pages=False,
        )
    elif index == 2:
        spec = WorkloadSpec(
            name="qwen2.5-14b-16x16384",
            n_layers=48,
            score_layer_stride=8,
            num_attention_heads=40,
            num_kv_heads=8,
            head_dim=128,
            rotary_dim=128,
            rope_theta=1e6,
            dtype=torch.bfloat16,
            seq_lens=(16384,) * 16,
            budget=4096,
            recent=128,
            channel_scale_sigma=0.25,
        )
    elif index == 3:
        spec = WorkloadSpec(
            name="qwen3.5-35b-a3b-hybrid-8x8k-64k",
            n_layers=10,
            score_layer_stride=2,
            num_attention_heads=16,
            num_kv_heads=2,
            head_dim=256,
            rotary_dim=64,
            rope_theta=1e7,
            dtype=torch.bfloat16,
            seq_lens=_uniform_lengths(8, 8192, 65536, seed=3),
            budget=4608,
            recent=512,
            prefix=128,
            segments=8,
            policy="v3",
            max_model_len=262144,
            scheduler_block=2048,
            model_type="qwen3_5_moe_text",
            notes=("budget 4608 measured at 128-token kernel-block granularity (36 blocks)",),
        )
    elif index == 4:
        spec = WorkloadSpec(
            name="qwen2.5-14b-4x131072-inplace",
            n_layers=48,
            score_layer_stride=8,
            num_attention_heads=40,
            num_kv_heads=8,
            head_dim=128,
            rotary_dim=128,
            rope_theta=1e6,
            dtype=torch.bfloat16,
            seq_lens=(131072,) * 4,
            budget=4608,
            recent=256,
            max_model_len=131072,
            inplace=True,
            outlier_fraction=0.01,
            pool_pages=4096,
        )
    elif index == 5:
        lengths = _lognormal_lengths(256, 6144.0, 0.5, 2048, 32768, seed=5)
        triggered = tuple(n for n in lengths if n >= 4096 + 128)
        spec = WorkloadSpec(
            name="qwen2.5-14b-decode-triggered-fp16",
            n_layers=24,
            score_layer_stride=8,
            num_attention_heads=40,
            num_kv_heads=8,
            head_dim=128,
            rotary_dim=128,
            rope_theta=1e6,
            dtype=torch.float16,
            seq_lens=triggered,
            budget=4096,
            recent=128,
            notes=(
                f"{len(triggered)} of 256 lognormal(median 6144, sigma 0.5) sequences crossed budget+128",
                "24 of 48 layers materialised: 48 layers of this cache exceed one GPU's HBM",
            ),
        )
    else:
        raise ValueError(f"unknown workload configuration {index}")
    return replace(spec, **overrides) if overrides else spec


@dataclass
class SyntheticCache:
    spec: WorkloadSpec
    k_caches: list[torch.Tensor]
    v_caches: list[torch.Tensor]
    source_tables: list[torch.Tensor]
    destination_tables: list[torch.Tensor] | None
    calibration: CalibrationStats
    round_starts: list[int]
    kv_buffers: list[torch.Tensor] | None = None  # the interleaved layout's per-layer buffers

    @property
    def seq_lens(self) -> list[int]:
        return list(self.spec.seq_lens)


# Padding elements of the interleaved layout hold this value (NaN) so that a
# kernel reading them shows up in its results; compaction must leave them alone.
PAD_VALUE = float("nan")


def interleaved_views(buffer: torch.Tensor, num_pages: int, spec: WorkloadSpec) -> tuple[torch.Tensor, torch.Tensor]:
    """K and V [pages, 128, kv, D] views of one layer's interleaved buffer."""
    row = spec.num_kv_heads * spec.head_dim
    page = KERNEL_BLOCK_SIZE * row
    stride = 2 * page + spec.page_pad
    shape = (num_pages, KERNEL_BLOCK_SIZE, spec.num_kv_heads, spec.head_dim)
    strides = (stride, row, spec.head_dim, 1)
    return torch.as_strided(buffer, shape, strides, 0), torch.as_strided(buffer, shape, strides, page)


def padding_view(buffer: torch.Tensor, num_pages: int, spec: WorkloadSpec) -> torch.Tensor:
    """[pages, page_pad] view of the padding of an interleaved buffer."""
    page = KERNEL_BLOCK_SIZE * spec.num_kv_heads * spec.head_dim
    return buffer.view(num_pages, 2 * page + spec.page_pad)[:, 2 * page :]


def synthetic_calibration(spec: WorkloadSpec, seed: int = 1) -> CalibrationStats:
    """Random complex query centres per layer and query head (float32)."""
    g = torch.Generator().manual_seed(seed)
    freq = spec.rotary_dim // 2
    pass_dim = spec.head_dim - spec.rotary_dim
    layers = {}
    for layer in range(spec.n_layers):
        qr = torch.randn(spec.num_attention_heads, freq, generator=g)
        qi = torch.randn(spec.num_attention_heads, freq, generator=g)
        q_abs = torch.sqrt(qr.square() + qi.square()) + torch.randn(spec.num_attention_heads, freq, generator=g).abs()
        q_pass = torch.randn(spec.num_attention_heads, pass_dim, generator=g) if pass_dim else None
        layers[layer] = LayerCalibrationStats(
            q_mean_real=qr,
            q_mean_imag=qi,
            q_abs_mean=q_abs,
            freq_scale_sq=torch.ones(1, freq),
            q_pass_mean=q_pass,
        )
    metadata = {
        "rope_style": "half",
        "head_dim": spec.head_dim,
        "rotary_dim": spec.rotary_dim,
        "num_attention_heads": spec.num_attention_heads,
        "num_kv_heads": spec.num_kv_heads,
        "rope_theta": spec.rope_theta,
        "model_type": spec.model_type,
        "num_layers": spec.n_layers,
    }
    return CalibrationStats(metadata=metadata, layers=layers)


def _page_tables(spec: WorkloadSpec, seed: int) -> tuple[int, list[list[int]], list[list[int]] | None]:
    """Source (and private destination) tables of 128-token kernel blocks."""
    k = spec.scheduler_block // KERNEL_BLOCK_SIZE
    logical_per_seq = [-(-n // spec.scheduler_block) for n in spec.seq_lens]
    dst_logical = -(-spec.budget // spec.scheduler_block)
    needed = sum(logical_per_seq) + (0 if spec.inplace else dst_logical * len(spec.seq_lens))
    pool_logical = needed
    if spec.pool_pages is not None:
        pool_logical = max(needed, spec.pool_pages // k)
    g = torch.Generator().manual_seed(seed)
    order = torch.randperm(pool_logical, generator=g) if spec.permute_pages else torch.arange(pool_logical)
    order = [int(x) for x in order]
    cursor = 0
    src, dst = [], []
    for count in logical_per_seq:
        src.append(order[cursor : cursor + count])
        cursor += count
    if not spec.inplace:
        for _ in spec.seq_lens:
            dst.append(order[cursor : cursor + dst_logical])
            cursor += dst_logical

    def expand(ids: list[int]) -> list[int]:
        return [i * k + j for i in ids for j in range(k)]

    budget_blocks = -(-spec.budget // KERNEL_BLOCK_SIZE)
    src_tables = [expand(ids) for ids in src]
    dst_tables = None if spec.inplace else [expand(ids)[:budget_blocks] for ids in dst]
    return pool_logical * k, src_tables, dst_tables


def build_synthetic_cache(
    spec: WorkloadSpec, device: torch.device | str, *, seed: int = 0, arena: bool = False
) -> SyntheticCache:
    """Allocate and fill every layer's K/V pool on ``device`` (seeded).

    ``arena=True`` carves all layers' K and V page pools out of one allocation
    ([K_0, V_0, K_1, V_1, ...], each a [pages, 128, kv_heads, head_dim] view);
    ``arena=False`` allocates one tensor per layer and kind.  The data are the
    same either way."""
    device = torch.device(device)
    num_pages, src_tables, dst_tables = _page_tables(spec, seed + 17)
    g = torch.Generator(device=device).manual_seed(seed)
    shape = (num_pages, KERNEL_BLOCK_SIZE, spec.num_kv_heads, spec.head_dim)
    k_caches, v_caches = [], []
    # A pool larger than the workload (a serving-sized pool) fills only the
    # pages the tables name; the others hold zeros.
    named = sorted({p for t in src_tables for p in t} | {p for t in (dst_tables or []) for p in t})
    used = range(num_pages) if len(named) == num_pages else named
    used_index = None if len(named) == num_pages else torch.tensor(named, dtype=torch.int64, device=device)
    outlier_rows = None
    if spec.outlier_fraction > 0:
        # Outlier tokens: the same (page, row) slots in every layer, K and V scaled.
        go = torch.Generator().manual_seed(seed + 29)
        slots = len(used) * KERNEL_BLOCK_SIZE
        count = int(round(spec.outlier_fraction * slots))
        outlier_rows = torch.randperm(slots, generator=go)[:count]
        if used_index is not None:
            pages = used_index.cpu()[outlier_rows // KERNEL_BLOCK_SIZE]
            outlier_rows = pages * KERNEL_BLOCK_SIZE + outlier_rows % KERNEL_BLOCK_SIZE
        outlier_rows = outlier_rows.to(device)
    cg = torch.Generator().manual_seed(seed + 7)
    pool = None
    kv_buffers = None
    if spec.kv_layout not in ("separate", "interleaved"):
        raise ValueError(f"unknown KV layout {spec.kv_layout!r}")
    if spec.kv_layout == "interleaved":
        if arena:
            raise ValueError("the interleaved KV layout has one buffer per layer; it has no arena form")
        page = KERNEL_BLOCK_SIZE * spec.num_kv_heads * spec.head_dim
        kv_buffers = [
            torch.full((num_pages * (2 * page + spec.page_pad),), PAD_VALUE, dtype=spec.dtype, device=device)
            for _ in range(spec.n_layers)
        ]
        if used_index is not None:
            for buf in kv_buffers:
                k_view, v_view = interleaved_views(buf, num_pages, spec)
                k_view.zero_()
                v_view.zero_()
    elif spec.page_pad:
        raise ValueError("page padding applies to the interleaved KV layout")
    if arena:
        alloc = torch.empty if used_index is None else torch.zeros
        pool = alloc((2 * spec.n_layers * num_pages,) + shape[1:], dtype=spec.dtype, device=device)
    for layer in range(spec.n_layers):
        caches = []
        for kind in range(2):
            if kv_buffers is not None:
                cache = interleaved_views(kv_buffers[layer], num_pages, spec)[kind]
            elif pool is not None:
                start = (2 * layer + kind) * num_pages
                cache = pool[start : start + num_pages]
            else:
                cache = (torch.empty if used_index is None else torch.zeros)(shape, dtype=spec.dtype, device=device)
            step = max(1, (1 << 26) // (KERNEL_BLOCK_SIZE * spec.num_kv_heads * spec.head_dim))  # bounded float32 chunks
            scale = None
            if spec.channel_scale_sigma > 0:
                scale = (1.0 + spec.channel_scale_sigma * torch.randn(spec.num_kv_heads, spec.head_dim, generator=cg)).to(device)
            for start in range(0, len(used), step):
                stop = min(len(used), start + step)
                chunk = torch.randn((stop - start,) + shape[1:], generator=g, device=device, dtype=torch.float32)
                if scale is not None:
                    chunk.mul_(scale)
                if used_index is None:
                    cache[start:stop].copy_(chunk)
                else:
                    cache.index_copy_(0, used_index[start:stop], chunk.to(spec.dtype))
            if outlier_rows is not None:
                pages = outlier_rows // KERNEL_BLOCK_SIZE
                offs = outlier_rows % KERNEL_BLOCK_SIZE
                cache[pages, offs] = (cache[pages, offs].float() * spec.outlier_scale).to(spec.dtype)
            caches.append(cache)
        k_caches.append(caches[0])
        v_caches.append(caches[1])
    to_dev = lambda rows: [torch.tensor(r, dtype=torch.int64, device=device) for r in rows]  # noqa: E731
    return SyntheticCache(
        spec=spec,
        k_caches=k_caches,
        v_caches=v_caches,
        source_tables=to_dev(src_tables),
        destination_tables=None if dst_tables is None else to_dev(dst_tables),
        calibration=synthetic_calibration(spec, seed + 1),
        round_starts=list(spec.seq_lens),
        kv_buffers=kv_buffers,
    )


def move_cache(cache: SyntheticCache, device: torch.device | str) -> SyntheticCache:
    """Copy a cache built on one device (e.g. the CPU, for oracle checks) to another."""
    to = lambda ts: [t.to(device) for t in ts]  # noqa: E731
    kv_buffers = None
    if cache.kv_buffers is not None:
        # Views keep their layout only if the buffers move and the views are rebuilt.
        kv_buffers = to(cache.kv_buffers)
        num_pages = int(cache.k_caches[0].shape[0])
        views = [interleaved_views(buf, num_pages, cache.spec) for buf in kv_buffers]
        k_caches, v_caches = [k for k, _ in views], [v for _, v in views]
    else:
        k_caches, v_caches = to(cache.k_caches), to(cache.v_caches)
    return SyntheticCache(
        spec=cache.spec,
        k_caches=k_caches,
        v_caches=v_caches,
        source_tables=to(cache.source_tables),
        destination_tables=None if cache.destination_tables is None else to(cache.destination_tables),
        calibration=cache.calibration,
        round_starts=list(cache.round_starts),
        kv_buffers=kv_buffers,
    )


def build_pipeline(cache: SyntheticCache, *, score_aggregation: str = "mean", layer_aggregation: str = "mean",
                   compaction_order: str = "auto"):
    """CompressionPipeline + Batch over a synthetic cache (all sequences)."""
    from .methods.triattention.pipeline import Batch, CompressionPipeline, ScoringTables
    from .methods.triattention.scoring import build_geometric_offsets

    spec = cache.spec
    device = cache.k_caches[0].device
    stats = cache.calibration.to_device(spec.model_shape(), device)
    offsets = build_geometric_offsets(spec.max_model_len, device)
    scoring = spec.scoring_layers
    tables = ScoringTables.from_layer_stats([stats[layer] for layer in scoring], offsets)
    pipeline = CompressionPipeline(
        scoring_k_caches=[cache.k_caches[layer] for layer in scoring],
        k_caches=cache.k_caches,
        v_caches=cache.v_caches,
        tables=tables,
        budget=spec.budget,
        protected_prefix=spec.prefix,
        protected_recent=spec.recent,
        segments=spec.segments,
        policy=spec.policy,
        layer_aggregation=layer_aggregation,
        max_seqs=len(spec.seq_lens),
        max_seq_len=max(spec.seq_lens),
        max_tokens=spec.total_tokens,
        score_aggregation=score_aggregation,
        compaction_order=compaction_order,
    )
    batch = Batch.build(
        device,
        list(spec.seq_lens),
        cache.round_starts,
        cache.source_tables,
        cache.destination_tables,
        budget=spec.budget,
    )
    return pipeline, batch
