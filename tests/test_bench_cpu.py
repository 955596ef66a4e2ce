"""bench.py's CPU-side pieces: its FLOP convention agrees with the oracle's
pair count, its CPU baseline runs, and --gpus > 1 is refused."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


@pytest.mark.parametrize("sq,sk,causal,window", [(4096, 4096, True, -1), (1, 32768, False, -1), (4, 32768, False, -1),
                                                 (16384, 16384, False, 4096), (300, 100, True, 16),
                                                 (100, 300, True, 7), (333, 222, False, 5)])
def test_pair_count_matches_oracle(oracle_lib, sq, sk, causal, window):
    import bench

    assert bench.valid_pairs(sq, sk, causal, window) == oracle_lib.valid_pairs(sq, sk, causal, window)


def test_rope_interleaved_matches_oracle(oracle_lib):
    import numpy as np
    import torch

    import bench

    cos, sin = bench.rope_tables(40, 64)
    x = torch.randn(1, 2, 40, 64)
    got = bench.rope_interleaved(x, cos, sin)
    ref = oracle_lib.rope(x.numpy(), cos.numpy(), sin.numpy(), round_f16=False)
    np.testing.assert_allclose(got.numpy(), ref, atol=1e-6)


def test_cpu_baseline_small():
    import bench

    spec = (1, 4, 2, 256, 256, 64, True, -1, True, 0, 1.0)
    q, k, v, cos, sin = bench.make_inputs(spec)
    r = bench.cpu_baseline(spec, q, k, v, cos, sin, budget_s=0.5)
    assert r["value"] > 0 and r["cores"] >= 1 and r["kind"] == "port"


def test_multi_gpu_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
