"""Write the config-1 golden vectors from the CPU oracle.

Inputs are regenerated from their seeds (workloads.build_synthetic_cache with
seed 0 on the CPU); the fixture stores checksums of those inputs plus the
oracle's aggregate scores, per-head statistics and keep set, so a drift in the
generator or the oracle is caught.  Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO / "vllm-ascend-kvcompress-hust_amd"))
sys.path.insert(0, str(REPO))

from kvcompress_mi355x import workloads  # noqa: E402
from oracle import stats_ref  # noqa: E402
from oracle import triattention_ref as ref  # noqa: E402


def sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def compute() -> dict:
    spec = workloads.config_spec(1)
    host = workloads.build_synthetic_cache(spec, "cpu", seed=0)
    # The calibration laid out by the oracle's own restatement of the device
    # layout (tri/stats.py:262-360), not by the product's loader.
    model = spec.model_shape()
    stats = stats_ref.layer_stats_for_device(
        host.calibration.layers,
        host.calibration.metadata,
        num_attention_heads=model.num_attention_heads,
        num_kv_heads=model.num_kv_heads,
        head_dim=model.head_dim,
        rotary_dim=model.effective_rotary_dim,
        rope_theta=model.rope_theta,
    )
    layer_stats = [stats[layer] for layer in spec.scoring_layers]
    cfg = ref.MethodConfig(budget=spec.budget, recent=spec.recent, score_chunk_size=8192, score_layer_stride=1)
    out = ref.method_select(
        [host.k_caches[layer] for layer in spec.scoring_layers],
        layer_stats,
        host.source_tables[0],
        spec.seq_lens[0],
        host.round_starts[0],
        ref.build_geometric_offsets(spec.max_model_len),
        cfg,
    )
    var, mean = out["stats"][0]
    return {
        "spec": spec,
        "inputs": {
            "k_sha256": sha256(host.k_caches[0]),
            "v_sha256": sha256(host.v_caches[0]),
            "q_real_sha256": sha256(stats[0].q_mean_real),
            "source_table": host.source_tables[0].tolist(),
            "destination_table": host.destination_tables[0].tolist(),
            "round_start": host.round_starts[0],
        },
        "agg": out["agg"].numpy(),
        "keep": out["keep"].numpy(),
        "mean": mean.reshape(-1).numpy(),
        "var": var.reshape(-1).numpy(),
    }


def main() -> None:
    r = compute()
    np.save(HERE / "config1_agg.npy", r["agg"].astype(np.float32))
    np.save(HERE / "config1_keep.npy", r["keep"].astype(np.int64))
    meta = {
        "workload": r["spec"].name,
        "generator": "kvcompress_mi355x.workloads.build_synthetic_cache(config_spec(1), 'cpu', seed=0)",
        "oracle": "oracle.triattention_ref.method_select (torch CPU restatement of the reference torch path) "
        "on calibration laid out by oracle.stats_ref.layer_stats_for_device",
        "torch": torch.__version__,
        "inputs": r["inputs"],
        "head_mean": [float(x) for x in r["mean"]],
        "head_var": [float(x) for x in r["var"]],
        "keep_sha256": hashlib.sha256(r["keep"].astype(np.int64).tobytes()).hexdigest(),
    }
    (HERE / "config1_expected.json").write_text(json.dumps(meta, indent=1) + "\n")
    print("wrote", HERE / "config1_expected.json")


if __name__ == "__main__":
    main()
