"""The reference's eager masked attention, restated for timing on host cores.

TEST INFRASTRUCTURE ONLY (same import rule as ``streaming_oracle``): this is
the ``cpu_baseline`` leg of ``bench.py`` -- the reference's CPU path
(``reference_block_sparse_attention``, sparse_triton_kernel.py:845-902):
lift the block mask to tokens, AND it with the StreamingLLM token mask,
``matmul -> * scale -> masked_fill(-inf) -> softmax -> nan_to_num -> matmul``
over ALL keys (Theta(N_Q * N_KV) work, as the reference does). To bound
memory it walks (b, h) slices and chunks of query rows; every chunk still
materialises full-width logits, so the arithmetic is the reference's.
Agreement with ``streaming_oracle.attention_fwd`` is tested in
tests/test_oracle_pins.py.
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def eager_masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           block_mask: torch.Tensor, bm: int, bn: int, causal: bool, sink: int,
                           window: int, scale: Optional[float] = None,
                           chunk: int = 2048) -> torch.Tensor:
    """fp32 eager masked attention on [B, H, N, D] CPU tensors, chunked over rows."""
    n_q, n_kv = q.shape[-2], k.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    out = torch.empty(q.shape, dtype=q.dtype)
    lifted_cols = block_mask.bool().repeat_interleave(bn, dim=1)[:, :n_kv]
    k_pos = torch.arange(n_kv)
    for r0 in range(0, n_q, chunk):
        r1 = min(n_q, r0 + chunk)
        rows = torch.arange(r0, r1)
        allowed = lifted_cols[rows // bm]
        if causal:
            q_abs = (rows + (n_kv - n_q))[:, None]
            allowed = allowed & (k_pos[None, :] <= q_abs) & (
                (k_pos[None, :] < sink) | (k_pos[None, :] >= q_abs - window + 1))
        logits = torch.matmul(q[..., r0:r1, :], k.transpose(-2, -1)) * scale
        logits = logits.masked_fill(~allowed, float("-inf"))
        probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
        out[..., r0:r1, :] = torch.matmul(probs, v)
    return out
