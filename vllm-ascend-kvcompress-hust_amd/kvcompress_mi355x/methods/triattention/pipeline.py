"""Batched TriAttention compression step on one GPU.

One call of :meth:`CompressionPipeline.step` runs, for every sequence of a
batch at once, the work the reference does per request in
TriAttentionMethod._select_keep_indices and compress (tri/method.py:256-475):

  1. phase table      kvc_mean_phases      [n_seq, S, F]
                      (kvc_offset_phases [n_seq, S, O, F] for score_aggregation "max")
  2. score            kvc_score_paged      raw scores (layout below) + partial sums
                      (kvc_score_paged_max: maximum over the offsets)
  3. head statistics  kvc_head_stats       mean/var [S, n_seq, H_q]
  4. aggregate        kvc_aggregate        agg [sum N] (head max, layer mean, sanitise)
  5. select           kvc_select_keep      keep [n_seq, budget] ascending
                      (kvc_select_keep_split for a few long sequences)
  6. compact          kvc_compact          kept K/V rows of every layer
  7. block tables     kvc_rewrite_block_tables

Raw scores are held [S, H_q, sum N] (head-major) when the matrix-core scorer
serves the shape and [S, sum N, H_q] otherwise (kvc_score_raw_layout); the
reference's workspace is [H_kv, qpk, max_len] per layer (tri/method.py:232-240).

Everything is enqueued on the current stream; nothing synchronises.  Device
buffers are sized once for a capacity (sequences, tokens, longest sequence)
and reused, as the reference keeps address-stable workspaces
(tri/method.py:205-254).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ... import _native
from . import _device as dev
from .cache import compact_layers, compact_workspace_bytes, rewrite_block_tables
from .selection import POLICY_CODES, prefers_split, select_keep_indices_batched, select_workspace, validate_selection


@dataclass(frozen=True)
class ScoringTables:
    """Calibration of the scoring layers, stacked for the kernel.

    q_real, q_imag, freq_scale (sqrt of freq_scale_sq), extra
    (q_abs_mean - sqrt(q_real^2 + q_imag^2 + 1e-8)): [S, kv_heads, qpk, F];
    q_pass: [S, kv_heads, qpk, P] or None; omega: [S, F]; offsets: [n_offsets].
    """

    q_real: torch.Tensor
    q_imag: torch.Tensor
    freq_scale: torch.Tensor
    extra: torch.Tensor
    q_pass: torch.Tensor | None
    omega: torch.Tensor
    offsets: torch.Tensor
    rotary_dim: int
    rope_style: str = "half"

    @property
    def n_layers(self) -> int:
        return int(self.q_real.shape[0])

    @property
    def kv_heads(self) -> int:
        return int(self.q_real.shape[1])

    @property
    def qpk(self) -> int:
        return int(self.q_real.shape[2])

    @property
    def freq(self) -> int:
        return int(self.q_real.shape[3])

    @classmethod
    def from_layer_stats(cls, stats: list, offsets: torch.Tensor) -> ScoringTables:
        """Stack DeviceLayerCalibrationStats of the scoring layers, with the
        bind-time precompute of tri/method.py:161-165."""
        q_real = torch.stack([s.q_mean_real for s in stats]).float().contiguous()
        q_imag = torch.stack([s.q_mean_imag for s in stats]).float().contiguous()
        scale = torch.sqrt(torch.stack([s.freq_scale_sq for s in stats]).float()).contiguous()
        q_abs = torch.stack([s.q_abs_mean for s in stats]).float()
        extra = (q_abs - torch.sqrt(q_real.square() + q_imag.square() + 1e-8)).contiguous()
        passes = [s.q_pass_mean for s in stats]
        q_pass = None if passes[0] is None else torch.stack(passes).float().contiguous()
        omega = torch.stack([s.omega for s in stats]).float().contiguous()
        rotary = stats[0].rotary_dim if stats[0].rotary_dim is not None else 2 * int(q_real.shape[-1])
        return cls(q_real, q_imag, scale, extra, q_pass, omega, offsets.float().contiguous(), int(rotary), stats[0].rope_style)


@dataclass
class Batch:
    """Device descriptors of one batch of sequences."""

    n_seq: int
    seq_lens_host: list[int]
    round_starts_host: list[int]
    src_lengths_host: list[int]
    seq_lens: torch.Tensor
    token_offsets: torch.Tensor
    round_starts: torch.Tensor
    src_offsets: torch.Tensor
    src_ids: torch.Tensor
    dst_offsets: torch.Tensor | None
    dst_ids: torch.Tensor | None
    rewrite_buffers: dict = field(default_factory=dict)

    @property
    def total_tokens(self) -> int:
        return sum(self.seq_lens_host)

    @property
    def inplace(self) -> bool:
        return self.dst_ids is None

    @classmethod
    def build(
        cls,
        device: torch.device,
        seq_lens: list[int],
        round_starts: list[int],
        source_tables: list,
        destination_tables: list | None = None,
        *,
        block_size: int = 128,
        budget: int | None = None,
    ) -> Batch:
        n = len(seq_lens)
        if n == 0 or len(round_starts) != n or len(source_tables) != n:
            raise ValueError("a batch needs matching lengths, round starts and source tables")
        src_off, src_ids, src_lens = dev.ragged(list(source_tables), device)
        for length, blocks in zip(seq_lens, src_lens):
            if length < 0 or blocks * block_size < length:
                raise ValueError("source block table does not cover the sequence")
        dst_off = dst_ids = None
        if destination_tables is not None:
            if len(destination_tables) != n:
                raise ValueError("one destination table per sequence")
            dst_off, dst_ids, dst_lens = dev.ragged(list(destination_tables), device)
            if budget is not None:
                need = (budget + block_size - 1) // block_size
                if any(d < need for d in dst_lens):
                    raise ValueError("destination table too short for the budget")
        offsets = [0]
        for length in seq_lens:
            offsets.append(offsets[-1] + int(length))
        return cls(
            n_seq=n,
            seq_lens_host=[int(x) for x in seq_lens],
            round_starts_host=[int(x) for x in round_starts],
            src_lengths_host=src_lens,
            seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
            token_offsets=torch.tensor(offsets, dtype=torch.int64, device=device),
            round_starts=torch.tensor(round_starts, dtype=torch.int64, device=device),
            src_offsets=src_off,
            src_ids=src_ids,
            dst_offsets=dst_off,
            dst_ids=dst_ids,
        )


class CompressionPipeline:
    """Device state and launches of the batched compression step."""

    def __init__(
        self,
        *,
        scoring_k_caches: list[torch.Tensor],
        k_caches: list[torch.Tensor],
        v_caches: list[torch.Tensor],
        tables: ScoringTables,
        budget: int,
        protected_prefix: int,
        protected_recent: int,
        segments: int,
        policy: str,
        layer_aggregation: str,
        max_seqs: int,
        max_seq_len: int,
        max_tokens: int | None = None,
        score_aggregation: str = "mean",
        compaction_order: str = "auto",
    ) -> None:
        if not scoring_k_caches or len(scoring_k_caches) != tables.n_layers:
            raise ValueError("one scoring K cache per scoring layer is required")
        if not k_caches or len(k_caches) != len(v_caches):
            raise ValueError("matching K and V cache lists are required")
        reference = k_caches[0]
        for i, cache in enumerate([*scoring_k_caches, *k_caches, *v_caches]):
            dev.validate_cache(cache, f"cache[{i}]")
            if cache.shape != reference.shape or cache.stride() != reference.stride() or cache.dtype != reference.dtype:
                raise ValueError("every cache layer must share shape, strides and dtype")
            dev.require_16_byte_pages(cache, f"cache[{i}]")
        if layer_aggregation not in ("mean", "max"):
            raise ValueError(f"unsupported layer aggregation {layer_aggregation!r}")
        if score_aggregation not in ("mean", "max"):
            raise ValueError(f"unsupported score aggregation: {score_aggregation}")
        if policy not in POLICY_CODES:
            raise ValueError(f"unsupported position policy: {policy}")
        self.device = reference.device
        self.dtype = reference.dtype
        self.num_pages = int(reference.shape[0])
        self.page_stride = int(reference.stride(0))
        self.kv_heads = int(reference.shape[2])
        self.head_dim = int(reference.shape[3])
        self.row_elems = self.kv_heads * self.head_dim
        if tables.kv_heads != self.kv_heads:
            raise ValueError("calibration KV-head count does not match cache keys")
        if 2 * tables.freq != tables.rotary_dim or tables.rotary_dim > self.head_dim:
            raise ValueError("calibration frequency count does not match cache keys")
        pass_dim = self.head_dim - tables.rotary_dim
        if pass_dim and (tables.q_pass is None or tables.q_pass.shape[-1] != pass_dim):
            raise ValueError("partial-RoPE scoring requires q_pass_mean")
        self.tables = tables
        self.budget = int(budget)
        self.protected_prefix = int(protected_prefix)
        self.protected_recent = int(protected_recent)
        self.segments = int(segments)
        self.policy = policy
        self.select_shape = "auto"  # "auto", "single" or "split" (kvc_select_keep / _split)
        self.layer_aggregation = layer_aggregation
        self.score_aggregation = score_aggregation
        self.n_heads = tables.kv_heads * tables.qpk
        self.scoring_ptrs = dev.pointer_table(scoring_k_caches, self.device)
        self.k_ptrs = dev.pointer_table(k_caches, self.device)
        self.v_ptrs = dev.pointer_table(v_caches, self.device)
        self._caches = (scoring_k_caches, k_caches, v_caches)  # keep the bound storage alive
        if compaction_order not in COMPACTION_ORDERS:
            raise ValueError(f"compaction_order must be one of {', '.join(COMPACTION_ORDERS)}, got {compaction_order!r}")
        self.compaction_form = CompactionFormChoice(fixed=None if compaction_order == "auto" else compaction_order)
        self._allocate(max_seqs, max_seq_len, max_tokens or max_seqs * max_seq_len)

    # ------------------------------------------------------------ buffers --
    def _allocate(self, max_seqs: int, max_seq_len: int, max_tokens: int) -> None:
        s = self.tables.n_layers
        self.max_seqs, self.max_seq_len, self.max_tokens = int(max_seqs), int(max_seq_len), int(max_tokens)
        dev_ = self.device
        n_off = int(self.tables.offsets.numel())
        if self.score_aggregation == "max":
            # Per-offset phases [n_seq, S, O, F] (kvc_offset_phases).
            self.phase_cos = torch.empty((self.max_seqs, s, n_off, self.tables.freq), dtype=torch.float32, device=dev_)
        else:
            self.phase_cos = torch.empty((self.max_seqs, s, self.tables.freq), dtype=torch.float32, device=dev_)
        self.phase_sin = torch.empty_like(self.phase_cos)
        layout = _native.load().kvc_score_raw_layout(
            dev.cache_dtype_code(self.dtype),
            dev.rope_style_code(self.tables.rope_style),
            self.kv_heads,
            self.head_dim,
            self.tables.rotary_dim,
            self.tables.qpk,
        )
        if layout < 0:
            _native.check(layout, "kvc_score_raw_layout")
        self.head_major = layout == _native.RAW_HEAD_MAJOR
        if self.head_major:
            # Token axis padded to 64 so every head row starts 256-byte aligned.
            padded = -(-self.max_tokens // 64) * 64
            self.raw = torch.empty((s, self.n_heads, padded), dtype=torch.float32, device=dev_)
        else:
            self.raw = torch.empty((s, self.max_tokens, self.n_heads), dtype=torch.float32, device=dev_)
        self.mean = torch.empty((s, self.max_seqs, self.n_heads), dtype=torch.float32, device=dev_)
        self.var = torch.empty_like(self.mean)
        self.agg = torch.empty(self.max_tokens, dtype=torch.float32, device=dev_)
        self.keep = torch.empty((self.max_seqs, self.budget), dtype=torch.int64, device=dev_)
        self.select_ws = select_workspace(self.max_seqs, self.segments, self.policy, dev_)
        self.compact_ws = torch.empty(compact_workspace_bytes(self.max_seqs, self.budget), dtype=torch.uint8, device=dev_)
        self.layer_scores = None  # flat per-layer head maxima, viewed [S, tokens]; made on first use
        shape = (s, self.kv_heads, self.head_dim, self.tables.rotary_dim, self.tables.qpk, self.max_seqs, self.max_seq_len)
        if self.score_aggregation == "max":
            ws = _native.load().kvc_score_max_workspace_bytes(*shape, n_off)
        else:
            ws = _native.load().kvc_score_workspace_bytes(*shape)
        if ws == 0:
            raise ValueError("unsupported scoring shape for the MI355X kernel")
        self.workspace_bytes = int(ws)
        self.workspace = torch.empty(self.workspace_bytes, dtype=torch.uint8, device=dev_)

    def raw_strides(self) -> tuple[int, int, int]:
        """(layer, token, head) element strides of the raw-score buffer."""
        if self.head_major:
            return int(self.raw.stride(0)), 1, int(self.raw.stride(1))
        return int(self.raw.stride(0)), int(self.raw.stride(1)), 1

    def head_statistics(self, batch: Batch) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-head mean and population variance of the last scored batch as
        [S, batch.n_seq, H_q] views (kvc_head_stats writes them densely for the
        batch, whatever the capacity of the buffers)."""
        shape = (self.tables.n_layers, batch.n_seq, self.n_heads)
        count = shape[0] * shape[1] * shape[2]
        return self.mean.view(-1)[:count].view(shape), self.var.view(-1)[:count].view(shape)

    def raw_scores(self) -> torch.Tensor:
        """Raw scores as a [S, tokens, H_q] view, whatever the buffer layout."""
        return self.raw.transpose(1, 2) if self.head_major else self.raw

    def ensure_capacity(self, batch: Batch) -> None:
        if (
            batch.n_seq > self.max_seqs
            or max(batch.seq_lens_host) > self.max_seq_len
            or batch.total_tokens > self.max_tokens
        ):
            self._allocate(
                max(batch.n_seq, self.max_seqs),
                max(max(batch.seq_lens_host), self.max_seq_len),
                max(batch.total_tokens, self.max_tokens),
            )

    def validate(self, batch: Batch) -> None:
        for n in batch.seq_lens_host:
            validate_selection(
                n,
                budget=self.budget,
                protected_prefix=self.protected_prefix,
                protected_recent=self.protected_recent,
                segments=self.segments,
                policy=self.policy,
            )

    # -------------------------------------------------------------- steps --
    def score(self, batch: Batch) -> None:
        """Phase table, raw scores and head statistics."""
        t = self.tables
        stream = dev.stream_handle(self.device)
        max_len = max(batch.seq_lens_host)
        n_off = int(t.offsets.numel())
        max_mode = self.score_aggregation == "max"
        _native.call(
            "kvc_offset_phases" if max_mode else "kvc_mean_phases",
            stream,
            batch.n_seq,
            t.n_layers,
            t.freq,
            dev.ptr(batch.round_starts),
            dev.ptr(t.offsets),
            n_off,
            dev.ptr(t.omega),
            dev.ptr(self.phase_cos),
            dev.ptr(self.phase_sin),
        )
        phase_args = (
            (dev.ptr(self.phase_cos), dev.ptr(self.phase_sin), n_off, t.n_layers * n_off * t.freq)
            if max_mode
            else (dev.ptr(self.phase_cos), dev.ptr(self.phase_sin), t.n_layers * t.freq)
        )
        _native.call(
            "kvc_score_paged_max" if max_mode else "kvc_score_paged",
            stream,
            dev.cache_dtype_code(self.dtype),
            t.n_layers,
            dev.ptr(self.scoring_ptrs),
            self.num_pages,
            self.page_stride,
            self.kv_heads,
            self.head_dim,
            t.rotary_dim,
            t.qpk,
            dev.rope_style_code(t.rope_style),
            batch.n_seq,
            max_len,
            dev.ptr(batch.seq_lens),
            dev.ptr(batch.token_offsets),
            dev.ptr(batch.src_offsets),
            dev.ptr(batch.src_ids),
            dev.ptr(t.q_real),
            dev.ptr(t.q_imag),
            dev.ptr(t.freq_scale),
            dev.ptr(t.extra),
            dev.ptr(t.q_pass),
            *phase_args,
            dev.ptr(self.raw),
            *self.raw_strides(),
            dev.ptr(self.workspace),
            self.workspace_bytes,
        )
        _native.call(
            "kvc_head_stats",
            stream,
            t.n_layers,
            self.kv_heads,
            self.head_dim,
            t.rotary_dim,
            t.qpk,
            batch.n_seq,
            max_len,
            dev.ptr(batch.seq_lens),
            dev.ptr(self.workspace),
            self.workspace_bytes,
            dev.ptr(self.mean),
            dev.ptr(self.var),
        )

    def aggregate(self, batch: Batch) -> None:
        t = self.tables
        _native.call(
            "kvc_aggregate",
            dev.stream_handle(self.device),
            t.n_layers,
            self.n_heads,
            batch.n_seq,
            max(batch.seq_lens_host),
            dev.ptr(batch.seq_lens),
            dev.ptr(batch.token_offsets),
            dev.ptr(self.raw),
            *self.raw_strides(),
            dev.ptr(self.mean),
            dev.ptr(self.var),
            # kvc_head_stats wrote [S][batch.n_seq][H_q] densely; the buffer
            # itself is sized for the pipeline's capacity.
            batch.n_seq * self.n_heads,
            self.n_heads,
            _native.LAYER_MEAN if self.layer_aggregation == "mean" else _native.LAYER_MAX,
            _native.AGG_FINALIZE,
            dev.ptr(self.agg),
        )

    # ---------------------------------------------- tensor-parallel halves --
    def local_layer_scores(self, batch: Batch) -> torch.Tensor:
        """Per-layer head maxima over this pipeline's query heads, [S, sum N]
        (after ``score``): the tensor the reference's TP path all-reduces with
        MAX across the ranks that hold the other KV heads
        (tri/method.py:316-322,447-461).  Contiguous (collectives take
        contiguous tensors); rewritten by every call."""
        t = self.tables
        total = batch.total_tokens
        if self.layer_scores is None or self.layer_scores.numel() < t.n_layers * total:
            self.layer_scores = torch.empty(t.n_layers * max(total, self.max_tokens), dtype=torch.float32, device=self.device)
        scores = self.layer_scores[: t.n_layers * total].view(t.n_layers, total)
        _native.call(
            "kvc_layer_head_max",
            dev.stream_handle(self.device),
            t.n_layers,
            self.n_heads,
            batch.n_seq,
            max(batch.seq_lens_host),
            dev.ptr(batch.seq_lens),
            dev.ptr(batch.token_offsets),
            dev.ptr(self.raw),
            *self.raw_strides(),
            dev.ptr(self.mean),
            dev.ptr(self.var),
            batch.n_seq * self.n_heads,
            self.n_heads,
            0,
            dev.ptr(scores),
            total,
        )
        return scores

    def combine_layer_scores(self, batch: Batch, layer_scores: torch.Tensor) -> None:
        """The aggregate from layer scores reduced across the TP group: layers
        combined in order, mean division and nan_to_num (tri/method.py:455-467)."""
        if layer_scores.ndim != 2 or layer_scores.shape[0] != self.tables.n_layers or layer_scores.stride(1) != 1:
            raise ValueError("layer scores must be [scoring layers, tokens] with contiguous rows")
        _native.call(
            "kvc_combine_layer_scores",
            dev.stream_handle(self.device),
            self.tables.n_layers,
            batch.total_tokens,
            dev.ptr(layer_scores),
            int(layer_scores.stride(0)),
            _native.LAYER_MEAN if self.layer_aggregation == "mean" else _native.LAYER_MAX,
            _native.AGG_FINALIZE,
            dev.ptr(self.agg),
        )

    def select_step_sharded(self, batch: Batch, all_reduce_max) -> torch.Tensor:
        """Score the local heads, reduce the per-layer head maxima across the
        group with ``all_reduce_max`` and select on the shared aggregate
        (tri/method.py:315-322,447-475): every rank gets the same keep set."""
        self.validate(batch)
        self.ensure_capacity(batch)
        self.score(batch)
        scores = self.local_layer_scores(batch)
        all_reduce_max(scores)
        self.combine_layer_scores(batch, scores)
        return self.select(batch)

    def step_sharded(self, batch: Batch, all_reduce_max, *, rewrite: bool = True):
        """The step of one tensor-parallel rank whose caches and calibration
        tables hold a shard of the KV heads: score the local heads, reduce the
        per-layer head maxima with ``all_reduce_max(tensor)`` (an in-place
        elementwise MAX over the group, e.g. torch.distributed.all_reduce with
        ReduceOp.MAX on a RCCL group; the library itself issues no collective),
        then select on the shared aggregate and compact the local heads.  Every
        rank of the group gets the same keep indices."""
        keep = self.select_step_sharded(batch, all_reduce_max)
        self.compact(batch)
        if not rewrite:
            return keep, None, None
        tables, freed = self.rewrite(batch)
        return keep, tables, freed

    def select(self, batch: Batch) -> torch.Tensor:
        shape = self.select_shape
        if shape == "auto":
            split = prefers_split(
                batch.seq_lens_host,
                protected_prefix=self.protected_prefix,
                protected_recent=self.protected_recent,
                segments=self.segments,
                policy=self.policy,
            )
            shape = "split" if split else "single"
        select_keep_indices_batched(
            self.agg,
            batch.seq_lens,
            batch.token_offsets,
            batch.seq_lens_host,
            self.keep,
            budget=self.budget,
            protected_prefix=self.protected_prefix,
            protected_recent=self.protected_recent,
            segments=self.segments,
            policy=self.policy,
            shape=shape,
            workspace=self.select_ws,
            validate=False,  # select_step and the callers of select validate the batch first
        )
        return self.keep[: batch.n_seq]

    def compact(self, batch: Batch) -> None:
        """kvc_compact over every layer, in the layer order this cache's
        trials chose (CompactionFormChoice).  Every order writes identical
        caches."""
        form, marks = self.compaction_form.next_call(self.device)
        if marks is not None:
            marks[0].record()
        compact_layers(
            self.k_ptrs,
            self.v_ptrs,
            num_pages=self.num_pages,
            page_stride=self.page_stride,
            row_elems=self.row_elems,
            seq_lens=batch.seq_lens,
            src_block_offsets=batch.src_offsets,
            src_block_ids=batch.src_ids,
            dst_block_offsets=batch.dst_offsets,
            dst_block_ids=batch.dst_ids,
            keep=self.keep,
            budget=self.budget,
            workspace=self.compact_ws,
            layer_order=form,
        )
        if marks is not None:
            marks[1].record()
            self.compaction_form.timed(form, marks, batch.n_seq * self.budget)

    def settle_compaction(self, batch: Batch, *, repeat_in_place: bool = False) -> str:
        """Run the compaction layer-order trials on this batch now and wait
        for them (the calls compact's first steps on a new cache would
        otherwise make lazily); returns the order kept.  Each trial is a full
        compaction of the batch: with private destinations that rewrites the
        same destination rows every time, but in place the second trial would
        compact an already compacted cache, so an in-place batch is refused
        unless ``repeat_in_place`` says the caller restores its pages (or
        does not need them) afterwards."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("settle_compaction waits for its trials and cannot run under graph capture")
        if batch.inplace and not repeat_in_place:
            raise ValueError("settle_compaction repeats the compaction: an in-place batch needs repeat_in_place=True")
        choice = self.compaction_form
        for _ in range(len(choice.SCHEDULE)):
            if choice.chosen is not None:
                break
            self.compact(batch)
        torch.cuda.synchronize(self.device)
        choice.settle()
        return choice.chosen

    def rewrite(self, batch: Batch) -> tuple[torch.Tensor, list[torch.Tensor]]:
        return rewrite_block_tables(
            budget=self.budget,
            src_block_offsets=batch.src_offsets,
            src_block_ids=batch.src_ids,
            src_lengths=batch.src_lengths_host,
            dst_block_offsets=batch.dst_offsets,
            dst_block_ids=batch.dst_ids,
            buffers=batch.rewrite_buffers,
        )

    def select_step(self, batch: Batch) -> torch.Tensor:
        """Score, aggregate and select: the keep indices of every sequence."""
        self.validate(batch)
        self.ensure_capacity(batch)
        self.score(batch)
        self.aggregate(batch)
        return self.select(batch)

    def step(self, batch: Batch, *, rewrite: bool = True) -> tuple[torch.Tensor, torch.Tensor | None, list[torch.Tensor] | None]:
        """The whole compression step for a batch."""
        keep = self.select_step(batch)
        self.compact(batch)
        if not rewrite:
            return keep, None, None
        tables, freed = self.rewrite(batch)
        return keep, tables, freed

    def capture(self, batch: Batch, *, rewrite: bool = True) -> StepGraph:
        """Record the whole step for ``batch`` as one HIP graph.

        A step is about ten kernel launches; for small batches their host cost
        exceeds the kernels' run time, and a replay issues them as one graph
        launch.  The graph holds every launch argument, so replays run on the
        same batch descriptors and pipeline buffers (their contents may change
        between replays: new keys in the same pages, new calibration values,
        new round starts).  Capacity is grown and one eager step runs first, so
        nothing is allocated while capturing; the step makes no allocation, no
        synchronisation and no memset of its own.
        """
        self.validate(batch)
        self.ensure_capacity(batch)
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.step(batch, rewrite=rewrite)
        torch.cuda.current_stream(self.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            outputs = self.step(batch, rewrite=rewrite)
        return StepGraph(graph, *outputs)


# "auto": time both layer orders on the cache and keep the faster (CompactionFormChoice).
COMPACTION_ORDERS = ("auto", "layer_major", "interleaved")


class CompactionFormChoice:
    """Which layer order a pipeline's planned compaction uses for its cache.

    kvc_compact's planned copy moves the same bytes in either order, but
    which is faster depends on where the cache's pages sit in HBM, which is
    fixed for the life of the cache and invisible to the kernels: on the
    Qwen2.5-14B 16 x 16384 batch, over five fresh allocations of the same
    pool, one layer at a time ran 4.37 - 4.49 ms in every one, every layer
    interleaved 4.12 - 4.24 ms in three and 4.59 - 4.77 ms in two.  The
    first two calls on a cache run one order each untimed (first touches),
    the next four alternate the orders with HIP events on the stream, read
    back later without waiting; once all four have completed, the
    interleaved order is kept if its faster trial moved a row at least 1%
    faster than the layer-major order's (repeated trials of one order differ
    by 0.2 - 0.5%), else the layer-major order.  Until
    then, and under graph capture, the layer-major order runs outside the
    trial schedule.  A ``fixed`` order is used from the first call, with no
    trials.
    """

    FORMS = ("layer_major", "interleaved")
    SCHEDULE = (("layer_major", False), ("interleaved", False), ("layer_major", True), ("interleaved", True),
                ("layer_major", True), ("interleaved", True))
    MARGIN = 0.99

    def __init__(self, event_factory=None, capturing=None, fixed: str | None = None) -> None:
        if fixed is not None and fixed not in self.FORMS:
            raise ValueError(f"unknown compaction layer order {fixed!r}")
        self.chosen: str | None = fixed
        self.per_row_ms: dict[str, float] | None = None
        self._next = 0
        self._trials: list[tuple[str, tuple, int]] = []
        self._event = event_factory or (lambda: torch.cuda.Event(enable_timing=True))
        self._capturing = capturing or torch.cuda.is_current_stream_capturing

    def next_call(self, device: torch.device | None = None) -> tuple[str, tuple | None]:
        """The form of the next compaction and, for a timed trial, the two
        events to record around it (then report them with ``timed``)."""
        if self.chosen is not None:
            return self.chosen, None
        if self._capturing():
            return "layer_major", None
        self._decide()
        if self.chosen is not None:
            return self.chosen, None
        if self._next < len(self.SCHEDULE):
            form, timed = self.SCHEDULE[self._next]
            self._next += 1
            if not timed:
                return form, None
            return form, (self._event(), self._event())
        return "layer_major", None  # timed trials still in flight

    def timed(self, form: str, marks: tuple, rows: int) -> None:
        self._trials.append((form, marks, max(int(rows), 1)))

    def settle(self) -> None:
        """Decide now, after the caller has synchronised the device with every
        trial run (the layer-major order if the schedule did not complete)."""
        self._decide()
        if self.chosen is None:
            self.chosen = "layer_major"

    def _decide(self) -> None:
        n_timed = sum(1 for _, timed in self.SCHEDULE if timed)
        if len(self._trials) < n_timed or not all(m[1].query() for _, m, _ in self._trials):
            return
        best: dict[str, float] = {}
        for form, m, rows in self._trials:
            ms = m[0].elapsed_time(m[1]) / rows
            best[form] = min(best.get(form, ms), ms)
        self.per_row_ms = best
        self.chosen = "interleaved" if best["interleaved"] < self.MARGIN * best["layer_major"] else "layer_major"
        self._trials.clear()


@dataclass
class StepGraph:
    """A captured compression step; ``replay()`` enqueues it on the current
    stream and the outputs are the step's own buffers, rewritten in place."""

    graph: torch.cuda.CUDAGraph
    keep: torch.Tensor
    tables: torch.Tensor | None
    freed: list[torch.Tensor] | None

    def replay(self) -> None:
        self.graph.replay()


def max_all_reducer(group):
    """In-place elementwise MAX over a torch.distributed process group, the
    collective of the reference's TP path (tri/method.py:447-453), as the
    ``all_reduce_max`` argument of :meth:`CompressionPipeline.step_sharded`.
    An RCCL ("nccl") group reduces the device tensor itself; gloo takes host
    tensors, so a device tensor goes through a host copy and back."""
    import torch.distributed as dist

    host_copy = dist.get_backend(group) == "gloo"

    def all_reduce_max(tensor: torch.Tensor) -> None:
        if host_copy and tensor.device.type != "cpu":
            host = tensor.to("cpu")
            dist.all_reduce(host, op=dist.ReduceOp.MAX, group=group)
            tensor.copy_(host)
        else:
            dist.all_reduce(tensor, op=dist.ReduceOp.MAX, group=group)

    return all_reduce_max
