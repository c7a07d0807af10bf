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
        # plausible: at least the algorithmic bytes, at most 2x (the heaviest-first
        # forward order re-reads the K / V rows of each head's short q tiles)
        assert 0.99 <= k["hbm_bytes"] / k["algorithmic_bytes"] <= 2.0, key


def test_config2_flops_are_the_kept_block_count():
    """4 * BM * BN * D flop per kept 64x64 block per (b, h): 8143 blocks x 32 heads,
    the flops_per_step bench.py divides by."""
    from oracle import streaming_oracle as so

    kept = int(so.block_mask(16384, 16384, 4, 2048, 64, 64).sum())
    assert kept == 8143
    assert 4 * 64 * 64 * 128 * kept * 32 == 546467479552


def test_block_granular_bytes_count_the_ragged_last_tile():
    """Config 4: 34 kept 64-key tiles, the last (1562) holding 100000 - 99968 =
    32 tokens: 2144 tokens x 128 x 2 tensors x 2 B x 256 heads = 281,018,368 B."""
    import torch

    from oracle import streaming_oracle as so

    row = torch.from_numpy(so.block_mask(1, 100000, 4, 2048, 1, 64))[0]
    assert int(row.sum()) == 34
    tokens = bench.block_granular_tokens(row, 100000, 64)
    assert tokens == 33 * 64 + 32
    assert tokens * 128 * 2 * 2 * 8 * 32 == 281018368


def test_cpu_threads_follow_the_allotted_share(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    assert bench.cpu_threads() == min(3, len(os.sched_getaffinity(0)))
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.cpu_threads() == len(os.sched_getaffinity(0))


def test_cpu_baseline_leg_on_a_small_sample():
    """The timed leg runs the oracle's eager path head by head within its
    budget: config-2-like forward (kept-block TFLOP/s), config-3-like forward +
    backward, and a config-4-like decode slice (kept K/V GB/s)."""
    import torch

    from oracle import streaming_oracle as so

    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 512, 64, generator=g) * 0.5 for _ in range(3))
    mask = torch.from_numpy(so.block_mask(512, 512, 4, 2048, 64, 64))
    kept = int(mask.sum())
    q3, k3, v3, do3 = (torch.randn(2, 1, 256, 64, generator=g).half() for _ in range(4))
    m3 = torch.from_numpy(so.block_mask(256, 256, 4, 1024, 64, 64))
    q4 = torch.randn(1, 2, 1, 128, generator=g).bfloat16()
    k4, v4 = (torch.randn(1, 2, 3000, 128, generator=g).bfloat16() for _ in range(2))
    m4 = torch.from_numpy(so.block_mask(1, 3000, 4, 2048, 1, 64))
    extra = {"c3": (q3, k3, v3, do3, m3, int(m3.sum())), "c4": (q4, k4, v4, m4)}
    out = bench.cpu_baseline((q, k, v, mask), kept, budget_s=0.5, extra=extra)
    assert out["kind"] == "port" and out["unit"] == "TFLOP/s"
    assert out["value"] > 0 and out["cores"] == bench.cpu_threads()
    assert out["cpu_model"] and out["os_cpu_count"] == os.cpu_count()
    assert "of 2 heads" in out["sample"]
    assert out["c3"]["unit"] == "TFLOP/s" and out["c3"]["value"] > 0
    assert "of 2 (b, h) slices" in out["c3"]["sample"]
    assert out["c4"]["unit"] == "GB/s" and out["c4"]["value"] > 0
    assert out["c1"]["unit"] == "TFLOP/s" and out["c1"]["value"] > 0
