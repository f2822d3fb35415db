"""The committed config-1 fixtures are reproduced by the seeded generator and the oracle."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_config1_fixture_reproduces() -> None:
    import sys

    sys.path.insert(0, str(GOLDEN))
    try:
        import make_golden
    finally:
        sys.path.pop(0)
    meta = json.loads((GOLDEN / "config1_expected.json").read_text())
    r = make_golden.compute()
    assert r["inputs"]["k_sha256"] == meta["inputs"]["k_sha256"], "seeded K generator drifted"
    assert r["inputs"]["v_sha256"] == meta["inputs"]["v_sha256"], "seeded V generator drifted"
    assert r["inputs"]["q_real_sha256"] == meta["inputs"]["q_real_sha256"], "calibration generator drifted"
    assert r["inputs"]["source_table"] == meta["inputs"]["source_table"]
    agg = np.load(GOLDEN / "config1_agg.npy", allow_pickle=False)
    keep = np.load(GOLDEN / "config1_keep.npy", allow_pickle=False)
    np.testing.assert_allclose(r["agg"], agg, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(r["mean"], np.array(meta["head_mean"], dtype=np.float32), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r["var"], np.array(meta["head_var"], dtype=np.float32), rtol=1e-5, atol=1e-6)
    assert keep.shape == (2048,) and np.all(np.diff(keep) > 0)
    assert set(keep[-128:].tolist()) == set(range(4096 - 128, 4096)), "recent window must be kept"
    assert len(set(r["keep"].tolist()) ^ set(keep.tolist())) == 0
