"""Tensor-parallel score synchronisation over a real process group (CPU, gloo).

Two processes stand for two TP ranks, each holding half of the KV heads
(tri/stats.py:315-323).  Every rank computes, with the oracle, the per-layer
maximum of its own heads' normalised scores, reduces it across the group with
the product's ``max_all_reducer`` (torch.distributed.all_reduce, ReduceOp.MAX,
tri/method.py:447-453), then combines the layers and selects
(tri/method.py:455-475).  Both ranks must hold the unsharded oracle's aggregate
bit for bit (a maximum is exact, and the layer sum runs in the same order) and
its keep set.
"""

from __future__ import annotations

import os
import socket

import pytest
import torch
import torch.multiprocessing as mp

from oracle import triattention_ref as ref

KV, QPK, DIM, TOKENS, LAYERS = 4, 2, 64, 3000, 2
CFG = ref.MethodConfig(budget=1024, recent=64, prefix=16, segments=4, policy="v3", score_chunk_size=1024)


def _problem():
    g = torch.Generator().manual_seed(5)
    pages = -(-TOKENS // 128)
    caches = [torch.randn(pages + 2, 128, KV, DIM, generator=g).to(torch.bfloat16) for _ in range(LAYERS)]
    freq = DIM // 2
    stats = []
    for _ in range(LAYERS):
        qr = torch.randn(KV, QPK, freq, generator=g)
        qi = torch.randn(KV, QPK, freq, generator=g)
        qa = torch.sqrt(qr.square() + qi.square()) + torch.rand(KV, QPK, freq, generator=g)
        fs = torch.rand(KV, QPK, freq, generator=g) + 0.5
        omega = 1.0 / (1e6 ** (torch.arange(0, DIM, 2, dtype=torch.float32) / DIM))
        stats.append(ref.LayerStats(qr, qi, qa, fs, omega))
    blocks = torch.randperm(pages + 2, generator=g)[:pages]
    return caches, stats, blocks


def _shard(stats: ref.LayerStats, heads: slice) -> ref.LayerStats:
    return ref.LayerStats(
        stats.q_mean_real[heads], stats.q_mean_imag[heads], stats.q_abs_mean[heads], stats.freq_scale_sq[heads],
        stats.omega, stats.rope_style, stats.rotary_dim, stats.q_pass_mean,
    )


def _rank_main(rank: int, world: int, port: int, out: str) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    import torch.distributed as dist

    from kvcompress_mi355x.methods.triattention.pipeline import max_all_reducer

    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        caches, stats, blocks = _problem()
        local = KV // world
        heads = slice(rank * local, (rank + 1) * local)
        offsets = ref.build_geometric_offsets(32768)
        raws, head_stats = ref.score_layers(
            [c[:, :, heads].contiguous() for c in caches], [_shard(s, heads) for s in stats], blocks, TOKENS, TOKENS,
            offsets, CFG,
        )
        layer_scores = torch.stack(
            [ref.normalize_head_scores(raw, mean, var).amax(dim=(0, 1)) for raw, (var, mean) in zip(raws, head_stats)]
        )
        max_all_reducer(dist.group.WORLD)(layer_scores)
        agg = layer_scores[0].clone()
        for layer in range(1, LAYERS):
            agg.add_(layer_scores[layer])
        agg.div_(float(LAYERS))
        agg.nan_to_num_(nan=float("-inf"), posinf=1e30, neginf=float("-inf"))
        keep = ref.select_keep_indices(
            agg, budget=CFG.budget, protected_prefix=CFG.prefix, protected_recent=CFG.recent, segments=CFG.segments,
            policy=CFG.policy,
        )
        torch.save({"agg": agg, "keep": keep}, out)
    finally:
        dist.destroy_process_group()


def _free_port() -> int:
    with socket.socket(socket.AF_INET, socket.SOCK_STREAM) as s:
        s.bind(("127.0.0.1", 0))
        return int(s.getsockname()[1])


def test_sharded_scores_meet_in_one_max_all_reduce(tmp_path) -> None:
    world = 2
    outs = [str(tmp_path / f"rank{r}.pt") for r in range(world)]
    port = _free_port()
    ctx = mp.get_context("spawn")
    procs = [ctx.Process(target=_rank_main, args=(r, world, port, outs[r])) for r in range(world)]
    for p in procs:
        p.start()
    for p in procs:
        p.join(timeout=240)
        if p.is_alive():
            p.kill()
            pytest.fail("a rank did not finish")
        assert p.exitcode == 0, f"rank exited with {p.exitcode}"
    caches, stats, blocks = _problem()
    want = ref.method_select(caches, stats, blocks, TOKENS, TOKENS, ref.build_geometric_offsets(32768), CFG)
    for out in outs:
        got = torch.load(out, weights_only=True)
        assert torch.equal(got["agg"], want["agg"]), "sharded aggregate differs from the unsharded one"
        assert torch.equal(got["keep"], want["keep"])
