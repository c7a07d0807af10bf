"""The comparative-baseline harness end to end on the GPU
(graph-kernel-injection_amd/benchmark.py; reference benchmark.py:599-740 and
the win / tie / loss rule of docs/eval_plan.md:111-135): at a small prefill
shape every method runs (this build, compiled FlexAttention, SDPA with the
StreamingLLM token mask, dense causal SDPA, eager), this build's output is
within the fp16 bar of the fp64 oracle at the harness's error shape, and a
verdict against FlexAttention is produced."""

from __future__ import annotations

import pytest
import torch

import benchmark as bm

pytestmark = pytest.mark.gpu


def test_harness_runs_every_method_and_gives_a_verdict(capsys):
    cfg = bm.HarnessConfig(batch=1, heads=2, seq_len_q=256, seq_len_kv=256, head_dim=64,
                           block_m=64, block_n=64, sink_size=4, window_size=64,
                           dtype=torch.float16, warmup_iters=2, measure_iters=5)
    results = bm.run_benchmark(cfg, backward=True)
    by = {r.label: r for r in results}
    assert {bm.OURS, "sdpa-explicit-mask", "sdpa-causal-dense", "eager-dense"} <= set(by)
    ours = by[bm.OURS]
    assert ours.max_abs_err_vs_fp64 is not None and ours.max_abs_err_vs_fp64 <= 2e-2
    assert ours.fwd_p50_ms > 0 and ours.fwdbwd_p50_ms is not None
    eager = by["eager-dense"].max_abs_err_vs_fp64
    assert eager is not None and ours.max_abs_err_vs_fp64 <= 2 * max(eager, 1e-3)
    out = capsys.readouterr().out
    line = [ln for ln in out.splitlines() if ln.startswith("[verdict]")]
    assert len(line) == 1
    if "flex-attention" in by:
        assert line[0].split()[1].rstrip(":") in ("WIN", "TIE", "LOSS")
    else:
        assert "no verdict" in line[0]
