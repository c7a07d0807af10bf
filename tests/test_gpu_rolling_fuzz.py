"""Seeded random sweep of the rolling sink + ring KV cache against the fp64 oracle (GPU).

Each case builds a ``StreamingKVCache`` with a random sink (0-8), window
(0-700) and query budget (1-4), appends a random prefill (1-2500 positions,
in one to three chunks, some longer than the ring), then runs one to six
decode steps of 1..max_query new tokens (``step``: append, then attend), with
1-8 q heads per kv head, head_dim 64 / 128 and fp32 / fp16 / bf16. Every step's
output and natural-log LSE are compared with the oracle's token rule over the
whole K / V history (the last n_q positions attend; sparse_triton_kernel.py:154-181
and 657-661 semantics): O at the parity tests' element-wise tolerances, the
LSE at those of the decode parity tests.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import sparse_triton_kernel as stk
from gki.kv_cache import StreamingKVCache
from oracle import streaming_oracle as so

DEV = "cuda"
TOL = {torch.float32: (1e-5, 0.0), torch.float16: (2e-2, 1e-2), torch.bfloat16: (2e-2, 1e-2)}
LSE_TOL = {torch.float32: 1e-5, torch.float16: 5e-4, torch.bfloat16: 2.5e-3}
N_CASES = 32


def _case(seed):
    rng = np.random.default_rng(9000 + seed)
    max_query = int(rng.integers(1, 5))
    chunks = [int(x) for x in rng.integers(1, 1200, size=int(rng.integers(1, 4)))]
    steps = [int(rng.integers(1, max_query + 1)) for _ in range(int(rng.integers(1, 7)))]
    return dict(B=int(rng.integers(1, 3)), H_kv=int(rng.choice([1, 2, 4])),
                group=int(rng.choice([1, 2, 4, 8])), D=int(rng.choice([64, 128])),
                dtype=[torch.float32, torch.float16, torch.bfloat16][int(rng.integers(0, 3))],
                sink=int(rng.integers(0, 9)), window=int(rng.integers(0, 701)),
                max_query=max_query, chunks=chunks, steps=steps)


def _close(ours, ref, tol, what):
    atol, rtol = tol
    o = ours.detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).to(torch.float64)
    assert torch.isfinite(o).all(), what
    bad = (o - r).abs() > atol + rtol * r.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} out of tolerance, max err {(o - r).abs().max():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_rolling_cache_matches_oracle(seed):
    c = _case(seed)
    print(f"[case] seed {seed}: {c}", flush=True)
    B, H_kv, group, D, dtype = c["B"], c["H_kv"], c["group"], c["D"], c["dtype"]
    H, sink, window = H_kv * group, c["sink"], c["window"]
    total = sum(c["chunks"]) + sum(c["steps"])
    gen = torch.Generator().manual_seed(seed)
    k_all = torch.randn(B, H_kv, total, D, generator=gen).to(dtype)
    v_all = torch.randn(B, H_kv, total, D, generator=gen).to(dtype)
    cache = StreamingKVCache(B, H_kv, D, stk.StreamingMaskSpec(sink, window), dtype, DEV, c["max_query"])
    pos = 0
    for n in c["chunks"]:
        cache.append(k_all[:, :, pos:pos + n].to(DEV), v_all[:, :, pos:pos + n].to(DEV))
        pos += n
    kn, vn = k_all.to(torch.float64).numpy(), v_all.to(torch.float64).numpy()
    for i, n in enumerate(c["steps"]):
        q = torch.randn(B, H, n, D, generator=gen).to(dtype)
        cache.append(k_all[:, :, pos:pos + n].to(DEV), v_all[:, :, pos:pos + n].to(DEV))
        pos += n
        o, lse = cache.attend(q.to(DEV), return_lse=True)
        eff = so.token_mask(n, pos, sink, window)
        kx = so.expand_kv_heads(kn[:, :, :pos], group)
        vx = so.expand_kv_heads(vn[:, :, :pos], group)
        o_ref, lse_ref = so.attention_fwd(q.to(torch.float64).numpy(), kx, vx, eff, 1.0 / math.sqrt(D))
        tag = f"seed {seed} step {i} (length {pos}, n_q {n})"
        _close(o, o_ref, TOL[dtype], f"O {tag}")
        _close(lse, lse_ref, (LSE_TOL[dtype], 0.0), f"LSE {tag}")
