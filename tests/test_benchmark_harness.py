"""Comparative-baseline harness (graph-kernel-injection_amd/benchmark.py): the
pure parts -- percentile, the win / tie / loss rule of the reference's
docs/eval_plan.md §5, the scaled-down error shape (benchmark.py:633-648)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import benchmark as bm


def _res(label, p50, p95, err):
    return bm.BenchResult(label, "float16", 1024, 0.1, p50, p95, None, None, 0.0, err)


def test_percentile_is_linear_interpolation():
    rng = np.random.default_rng(0)
    for n in (1, 2, 7, 100):
        x = rng.random(n).tolist()
        for q in (0, 50, 95, 100):
            assert abs(bm.percentile(x, q) - np.percentile(x, q)) < 1e-12


def test_verdict_rules():
    flex = _res("flex-attention", 1.0, 1.0, 1e-3)
    assert bm.verdict(_res(bm.OURS, 0.5, 0.5, 1e-3), flex).startswith("WIN")
    assert bm.verdict(_res(bm.OURS, 0.95, 0.95, 1e-3), flex).startswith("TIE")
    assert bm.verdict(_res(bm.OURS, 1.2, 1.2, 1e-3), flex).startswith("LOSS")
    # faster but more than 2x the error: loss
    assert bm.verdict(_res(bm.OURS, 0.5, 0.5, 3e-3), flex).startswith("LOSS")
    # faster but noisy (p95 / p50 > 2): tie
    assert bm.verdict(_res(bm.OURS, 0.2, 0.5, 1e-3), flex).startswith("TIE")
    assert "no verdict" in bm.verdict(_res(bm.OURS, 1, 1, None), None)
    assert bm.verdict(_res(bm.OURS, 1, 1, None), None, "boom").endswith("no verdict (boom)")


def test_error_shape_is_scaled_down():
    cfg = bm.HarnessConfig(batch=8, heads=32, seq_len_q=1, seq_len_kv=100000, head_dim=128,
                           block_m=1, window_size=2048, dtype=torch.bfloat16)
    s = bm._error_shape(cfg)
    assert (s.batch, s.heads, s.seq_len_q, s.seq_len_kv, s.head_dim) == (1, 2, 1, 256, 64)
    assert (s.block_m, s.block_n, s.window_size, s.sink_size) == (1, 64, 128, 4)


def test_failure_text_keeps_first_line_and_the_cause():
    e = RuntimeError("SubprocException: An exception occurred in a subprocess:\n\nTraceback:\n  x\n"
                     "ValueError: bad tile\n\nSet TORCHDYNAMO_VERBOSE=1 for the internal stack trace")
    assert bm.failure_text(e) == ("RuntimeError: SubprocException: An exception occurred in a subprocess: ... "
                                  "ValueError: bad tile")
    assert bm.failure_text(RuntimeError("one line")) == "RuntimeError: one line"
    assert bm.failure_text(RuntimeError("first\nno cause here")) == "RuntimeError: first"
    assert bm.failure_text(RuntimeError()) == "RuntimeError"


def test_skip_option_names_comparison_methods_only():
    a = bm._parse(["--skip", "sdpa-causal-dense", "--skip", "eager-dense"])
    assert a.skip == ["sdpa-causal-dense", "eager-dense"]
    assert bm._parse([]).skip == []
    with pytest.raises(SystemExit):
        bm._parse(["--skip", bm.OURS])   # this build is always timed
