"""Eager masked attention -- the reference's public correctness oracle API.

``reference_block_sparse_attention`` mirrors ``sparse_triton_kernel.py:845-902``:
it materialises the ``[N_Q, N_KV]`` logits, so it is Theta(N^2) memory and only
meant for validating the kernels on small shapes. It is plain PyTorch on
whatever device its inputs live on and is never called by the kernel path.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .masks import streaming_token_mask


def reference_block_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    block_mask: torch.Tensor,
    softmax_scale: Optional[float] = None,
    block_m: int = 64,
    block_n: int = 64,
    is_causal: bool = False,
    sink_size: int = 0,
    window_size: int = 0,
) -> torch.Tensor:
    """softmax(mask(Q K^T * scale)) V with mask = lift(block_mask) [& token mask].

    The block mask is lifted to tokens (each entry covers a ``block_m x
    block_n`` patch, clipped to ``[N_Q, N_KV]``); with ``is_causal`` it is
    intersected with the StreamingLLM token mask. Fully-masked rows give 0.
    """
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    n_q, n_kv = q.shape[-2], k.shape[-2]
    allowed = block_mask.to(device=q.device).bool()
    allowed = allowed.repeat_interleave(block_m, dim=0).repeat_interleave(block_n, dim=1)
    allowed = allowed[:n_q, :n_kv]
    if is_causal:
        allowed = allowed & streaming_token_mask(n_q, n_kv, sink_size, window_size, device=q.device)
    logits = torch.matmul(q, k.transpose(-2, -1)) * softmax_scale
    logits = logits.masked_fill(~allowed, float("-inf"))
    probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
    return torch.matmul(probs, v)
