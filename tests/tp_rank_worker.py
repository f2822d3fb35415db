"""One tensor-parallel rank of TriAttentionMethod on the local GPU.

Test helper, run as a subprocess by tests/test_gpu_tensor_parallel.py: the
rank joins a gloo group, binds the method to its shard of the KV heads of a
seeded synthetic cache (tensor_parallel_size = world size), selects and
compresses one request, and saves its keep indices and compacted rows.
vLLM's tensor-parallel group coordinator is stood in for by a module that
provides ``get_tp_group()`` with ``rank_in_group`` and ``device_group``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import types
from pathlib import Path
from types import SimpleNamespace

REPO = Path(__file__).resolve().parents[1]
sys.path[:0] = [str(REPO / "vllm-ascend-kvcompress-hust_amd"), str(REPO)]


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--rank", type=int, required=True)
    parser.add_argument("--world", type=int, required=True)
    parser.add_argument("--port", type=int, required=True)
    parser.add_argument("--job", required=True, help="JSON: spec overrides, method options")
    parser.add_argument("--out", required=True)
    args = parser.parse_args()
    job = json.loads(Path(args.job).read_text())
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(args.port)

    import torch
    import torch.distributed as dist

    print(f"rank {args.rank}: joining the group", flush=True)
    dist.init_process_group("gloo", rank=args.rank, world_size=args.world)
    coordinator = SimpleNamespace(rank_in_group=args.rank, device_group=dist.group.WORLD)
    vllm = types.ModuleType("vllm")
    vllm_distributed = types.ModuleType("vllm.distributed")
    vllm_distributed.get_tp_group = lambda: coordinator
    vllm.distributed = vllm_distributed
    sys.modules["vllm"] = vllm
    sys.modules["vllm.distributed"] = vllm_distributed

    from kvcompress_mi355x import workloads
    from kvcompress_mi355x.methods import create_method
    from kvcompress_mi355x.methods.base import CompressionRequest, LayerCache
    from kvcompress_mi355x.methods.triattention.cache import token_slots

    spec = workloads.config_spec(job["config"], **job["overrides"])
    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    local = spec.num_kv_heads // args.world
    heads = slice(args.rank * local, (args.rank + 1) * local)
    device = torch.device("cuda:0")
    ks = [k[:, :, heads].contiguous().to(device) for k in host.k_caches]
    vs = [v[:, :, heads].contiguous().to(device) for v in host.v_caches]
    vllm_config = SimpleNamespace(
        parallel_config=SimpleNamespace(tensor_parallel_size=args.world),
        model_config=SimpleNamespace(max_model_len=spec.max_model_len),
        speculative_config=None,
    )
    method = create_method("triattention", job["options"], vllm_config, spec.model_shape())
    layers = tuple(LayerCache(f"model.layers.{i}.self_attn.attn", i, ks[i], vs[i]) for i in range(spec.n_layers))
    method.bind_model_runner(SimpleNamespace(device=device), layers)
    src = host.source_tables[0].to(device)
    dst = host.destination_tables[0].to(device)
    n = spec.seq_lens[0]
    rs = host.round_starts[0]
    print(f"rank {args.rank}: selecting", flush=True)
    keep = method.select_keep_indices(src, n, rs)
    request = CompressionRequest(
        request_id="r0",
        semantic_num_tokens=rs,
        physical_num_tokens=n,
        source_block_ids=(tuple(src.cpu().tolist()),),
        destination_block_ids=(tuple(dst.cpu().tolist()),),
        source_block_ids_device=src,
        destination_block_ids_device=dst,
    )
    print(f"rank {args.rank}: compressing", flush=True)
    result = method.compress(request)
    torch.cuda.synchronize()
    budget = result.physical_num_tokens
    slots = token_slots(dst, torch.arange(budget, device=device), 128)
    k_rows = torch.stack([k.view(-1, local, spec.head_dim)[slots] for k in ks]).cpu()
    v_rows = torch.stack([v.view(-1, local, spec.head_dim)[slots] for v in vs]).cpu()
    torch.save({"keep": keep.cpu(), "k": k_rows, "v": v_rows, "budget": budget}, args.out)
    dist.destroy_process_group()
    print(f"rank {args.rank}: done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
