"""Seeded random sweep of the decode paths against the fp64 oracle (GPU).

Each case draws a decode geometry the prefill fuzz (``test_gpu_fuzz.py``, at
most 320 keys) does not reach: 1-4 query positions over up to ~8000 keys, so
that the split decode and its merge run, grouped-query groups of 1-16 q heads
per kv head (the matrix-core decode serves 2-32 rows per K/V stream, the
vector decode one), head_dim 64 / 128, fp32 / fp16 / bf16, a StreamingLLM mask
with a random sink (0-8) and window (0, or up to 3000) and key block size,
bottom-right aligned queries (sparse_triton_kernel.py:657-661). The output,
and on a third of the cases dQ / dK / dV through autograd, are compared with
the oracle's closed forms (sparse_triton_kernel.py:845-902 semantics) at the
parity tests' element-wise tolerances (fp32 atol 1e-5; fp16 / bf16 atol 2e-2 +
rtol 1e-2), inputs N(0, 1).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import sparse_triton_kernel as stk
from oracle import streaming_oracle as so

DEV = "cuda"
TOL = {torch.float32: (1e-5, 0.0), torch.float16: (2e-2, 1e-2), torch.bfloat16: (2e-2, 1e-2)}
N_CASES = 48


def _case(seed):
    rng = np.random.default_rng(5000 + seed)
    H_kv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 1, 2, 4, 8, 16]))
    B = min(int(rng.integers(1, 4)), max(1, 32 // (H_kv * group)))   # at most 32 q heads in all
    n_q = int(rng.integers(1, 5))
    n_kv = int(np.exp(rng.uniform(np.log(32), np.log(8000))))
    D = int(rng.choice([64, 128]))
    dtype = [torch.float32, torch.float16, torch.bfloat16][int(rng.integers(0, 3))]
    bn = int(rng.choice([16, 32, 64, 128]))
    sink = int(rng.integers(0, 9))
    window = 0 if rng.random() < 0.1 else int(rng.integers(1, 3001))
    backward = bool(rng.random() < 1 / 3)
    return dict(B=B, H_kv=H_kv, group=group, n_q=n_q, n_kv=n_kv, D=D, dtype=dtype, bn=bn, sink=sink,
                window=window, backward=backward)


def _close(ours, ref, dtype, what):
    o = ours.detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).to(torch.float64)
    assert torch.isfinite(o).all(), what
    atol, rtol = TOL[dtype]
    bad = (o - r).abs() > atol + rtol * r.abs()
    assert not bad.any(), (f"{what}: {int(bad.sum())} out of tolerance, max err {(o - r).abs().max():.3e}, "
                           f"max |ref| {r.abs().max():.3e}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_decode_matches_oracle(seed):
    c = _case(seed)
    print(f"[case] seed {seed}: {c}", flush=True)
    B, H_kv, group, n_q, n_kv, D, dtype = (c[k] for k in ("B", "H_kv", "group", "n_q", "n_kv", "D", "dtype"))
    H = H_kv * group
    bn, sink, window = c["bn"], c["sink"], c["window"]
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), 1, bn, device=DEV)
    gen = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=gen).to(dtype).to(DEV)  # noqa: E731
    q, k, v, do = mk(B, H, n_q, D), mk(B, H_kv, n_kv, D), mk(B, H_kv, n_kv, D), mk(B, H, n_q, D)
    leaves = [t.clone().requires_grad_(c["backward"]) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=1, block_n=bn, is_causal=True,
                                     sink_size=sink, window_size=window, enable_gqa=group > 1)

    eff = so.effective_mask(mask.cpu().numpy(), n_q, n_kv, 1, bn, True, sink, window)
    qn, kn, vn, don = (t.to(torch.float64).cpu().numpy() for t in (q, k, v, do))
    kx, vx = so.expand_kv_heads(kn, group), so.expand_kv_heads(vn, group)
    s = 1.0 / math.sqrt(D)
    o_ref, _ = so.attention_fwd(qn, kx, vx, eff, s)
    tag = f"seed {seed}"
    _close(out, o_ref, dtype, f"O {tag}")
    if c["backward"]:
        out.backward(do)
        dq, dk, dv = so.attention_bwd(qn, kx, vx, don, eff, s)
        refs = [dq, so.reduce_kv_grad(dk, group), so.reduce_kv_grad(dv, group)]
        for name, t, ref in zip(("dQ", "dK", "dV"), leaves, refs):
            _close(t.grad, ref, dtype, f"{name} {tag}")
