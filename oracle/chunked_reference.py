"""Memory-bounded exact masked attention (torch, any device) for full-size checks.

TEST INFRASTRUCTURE ONLY (same import rule as ``streaming_oracle``): used by
``tests/`` to check the HIP kernels at the configs' full sizes, where the
eager reference (sparse_triton_kernel.py:845-902) would need Theta(N^2)
memory (34 GB of fp32 logits for config 2).

It computes the same function as the eager reference -- softmax over
``lift(block_mask) & token_mask`` (causal) or ``lift(block_mask)`` -- but one
chunk of query rows at a time, over only the key columns of the mask blocks
those rows keep. Masked-out logits are exactly -inf in the eager reference,
so dropping them changes nothing. Gradients use the closed form of the
softmax-attention backward (the same algebra as ``attention_bwd`` in
``streaming_oracle``, which is pinned against autograd); empty rows give
zeros, as the eager reference's nan_to_num does.
Pinned against ``streaming_oracle`` on small shapes in tests/test_oracle_pins.py.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def _chunk_keys(mask: torch.Tensor, r0: int, r1: int, bm: int, bn: int, n_kv: int) -> torch.Tensor:
    rows = mask[r0 // bm:(r1 - 1) // bm + 1]
    cols = torch.nonzero(rows.any(dim=0), as_tuple=False).flatten()
    if cols.numel() == 0:
        return cols
    offs = torch.arange(bn, device=mask.device)
    keys = (cols[:, None] * bn + offs[None, :]).flatten()
    return keys[keys < n_kv]


def _chunk_allowed(mask: torch.Tensor, r0: int, r1: int, keys: torch.Tensor, bm: int, bn: int,
                   n_q: int, n_kv: int, causal: bool, sink: int, window: int) -> torch.Tensor:
    rows = torch.arange(r0, r1, device=mask.device)
    allowed = mask[(rows // bm)[:, None], (keys // bn)[None, :]] != 0
    if causal:
        q_abs = (rows + (n_kv - n_q))[:, None]
        k = keys[None, :]
        allowed &= (k <= q_abs) & ((k < sink) | (k >= q_abs - window + 1))
    return allowed


def _probs(qc, kk, allowed, scale):
    s = torch.matmul(qc, kk.transpose(-1, -2)) * scale
    s = s.masked_fill(~allowed, float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    e = torch.exp(s - m)
    l = e.sum(dim=-1, keepdim=True)
    safe = torch.where(l > 0, l, torch.ones_like(l))
    p = e / safe
    lse = torch.where(l[..., 0] > 0, m[..., 0] + torch.log(safe[..., 0]), torch.zeros_like(l[..., 0]))
    return p, lse


def chunked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_mask: torch.Tensor,
                      bm: int, bn: int, causal: bool, sink: int, window: int,
                      scale: Optional[float] = None, do: Optional[torch.Tensor] = None,
                      chunk: int = 1024, dtype: torch.dtype = torch.float64
                      ) -> Tuple[torch.Tensor, ...]:
    """Exact (O, LSE) and, if ``do`` is given, (dQ, dK, dV), computed in ``dtype``.

    Inputs are [B, H, N, D]; ``block_mask`` is [ceil(N_Q/bm), ceil(N_KV/bn)].
    Outputs are in ``dtype`` on the inputs' device.
    """
    n_q, n_kv, d = q.shape[-2], k.shape[-2], q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    mask = block_mask.to(device=q.device)
    o = torch.zeros(q.shape, dtype=dtype, device=q.device)
    lse = torch.zeros(q.shape[:-1], dtype=dtype, device=q.device)
    grads = do is not None
    if grads:
        dq = torch.zeros(q.shape, dtype=dtype, device=q.device)
        dk = torch.zeros(k.shape, dtype=dtype, device=q.device)
        dv = torch.zeros(v.shape, dtype=dtype, device=q.device)
    for r0 in range(0, n_q, chunk):
        r1 = min(n_q, r0 + chunk)
        keys = _chunk_keys(mask, r0, r1, bm, bn, n_kv)
        if keys.numel() == 0:
            continue
        allowed = _chunk_allowed(mask, r0, r1, keys, bm, bn, n_q, n_kv, causal, sink, window)
        qc = q[..., r0:r1, :].to(dtype)
        kk = k[..., keys, :].to(dtype)
        vv = v[..., keys, :].to(dtype)
        p, lse_c = _probs(qc, kk, allowed, scale)
        o[..., r0:r1, :] = torch.matmul(p, vv)
        lse[..., r0:r1] = lse_c
        if grads:
            g = do[..., r0:r1, :].to(dtype)
            dp = torch.matmul(g, vv.transpose(-1, -2))
            ds = p * (dp - (p * dp).sum(dim=-1, keepdim=True))
            dq[..., r0:r1, :] = scale * torch.matmul(ds, kk)
            dk.index_add_(-2, keys, scale * torch.matmul(ds.transpose(-1, -2), qc))
            dv.index_add_(-2, keys, torch.matmul(p.transpose(-1, -2), g))
        del p
    if grads:
        return o, lse, dq, dk, dv
    return o, lse
