"""bench.py's contract on the CPU: the multi-GPU refusal, the roofline object,
HBM traffic from the committed rocprofv3 figures, the algorithmic flop count of
config 2, and the CPU-baseline leg on a bounded sample (no GPU needed)."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path.insert(0, REPO)

import bench  # noqa: E402


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args], capture_output=True,
                       text=True, timeout=300, env={**os.environ, **env})
    assert r.returncode == 2
    assert "one MI355X only" in r.stderr
    assert r.stdout == ""


def test_roofline_fields():
    r = bench._roofline(881.0, bench.PEAK_MFMA_16, "TFLOP/s", "mfma", 123)
    assert r == {"bound": "mfma", "achieved": 881.0, "peak": 2500.0, "unit": "TFLOP/s",
                 "frac": round(881.0 / 2500.0, 4), "traffic": 123}
    assert bench.PEAK_HBM == 8000.0


def test_traffic_comes_from_the_committed_profile():
    with open(os.path.join(REPO, "profiles", "hbm_traffic.json")) as f:
        prof = json.load(f)
    assert bench._traffic("c2_fwd") == prof["kernels"]["c2_fwd"]["hbm_bytes"]
    both = prof["kernels"]["c3_dkdv"]["hbm_bytes"] + prof["kernels"]["c3_dq"]["hbm_bytes"]
    assert bench._traffic("c3_dkdv", "c3_dq") == both
    assert bench._traffic("no_such_kernel") is None
    # scaled FETCH / WRITE counters against the algorithmic bytes of each launch
    for key, k in prof["kernels"].items():
        scaled = k["fetch_size_kib"] * 1024 * prof["calibration"]["fetch_scale"] + \
            k["write_size_kib"] * 1024 * prof["calibration"]["write_scale"]
        assert abs(scaled - k["hbm_bytes"]) <= 2048, key
        assert 0.99 <= k["hbm_bytes"] / k["algorithmic_bytes"] <= 1.5, key


def test_config2_flops_are_the_kept_block_count():
    """4 * BM * BN * D flop per kept 64x64 block per (b, h): 8143 blocks x 32 heads,
    the flops_per_step bench.py divides by."""
    from oracle import streaming_oracle as so

    kept = int(so.block_mask(16384, 16384, 4, 2048, 64, 64).sum())
    assert kept == 8143
    assert 4 * 64 * 64 * 128 * kept * 32 == 546467479552


def test_cpu_baseline_leg_on_a_small_sample():
    """The timed leg runs the oracle's eager path (S 4, W 2048, 64x64 blocks, as
    config 2) head by head within its budget and reports kept-block TFLOP/s."""
    import torch

    from oracle import streaming_oracle as so

    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 512, 64, generator=g) * 0.5 for _ in range(3))
    mask = torch.from_numpy(so.block_mask(512, 512, 4, 2048, 64, 64))
    kept = int(mask.sum())
    out = bench.cpu_baseline((q, k, v, mask), kept, budget_s=0.5)
    assert out["kind"] == "port" and out["unit"] == "TFLOP/s"
    assert out["value"] > 0 and out["cores"] >= 1
    assert "of 2 heads" in out["sample"]
