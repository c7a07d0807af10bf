"""First-order gradcheck of ``block_sparse_attention`` through the HIP kernels.

The reference harness's FlashAttention-2 fp32 tier (benchmark.py:222-270,
306-319): fp32 inputs B1 H2 N64 D16 from a seed-0 device generator drawn q, k,
v in that order, 16x16 blocks, StreamingLLM S4 W16 causal; finite differences
with eps 1e-3 against the analytic Jacobian at atol = rtol = 5e-3. The op
rejects fp64, so the reference's fp64 tier has no counterpart. First order only:
the backward launches kernels and is not itself differentiable, so the
reference's gradgradcheck does not apply. A custom non-causal mask with an
empty row block checks the zero-gradient rows the same way.
"""

from __future__ import annotations

import math

import pytest
import torch

import sparse_triton_kernel as stk

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs():
    g = torch.Generator(device=DEV).manual_seed(0)
    shape = (1, 2, 64, 16)
    return [torch.randn(shape, generator=g, device=DEV, dtype=torch.float32).requires_grad_(True)
            for _ in range(3)]


def _check(fn, inputs):
    assert torch.autograd.gradcheck(fn, inputs, eps=1e-3, atol=5e-3, rtol=5e-3, nondet_tol=0.0,
                                    fast_mode=False, check_undefined_grad=False,
                                    check_batched_grad=False)


def test_gradcheck_streaming_causal_fp32():
    mask = stk.make_streaming_mask(64, 64, stk.StreamingMaskSpec(4, 16), 16, 16, device=DEV)

    def fn(q, k, v):
        return stk.block_sparse_attention(q, k, v, mask, softmax_scale=1.0 / math.sqrt(16),
                                          block_m=16, block_n=16, is_causal=True, sink_size=4,
                                          window_size=16)

    _check(fn, _inputs())


def test_gradcheck_custom_mask_with_an_empty_row_block_fp32():
    mask = torch.tensor([[1, 0, 1, 0], [0, 0, 0, 0], [1, 1, 0, 1], [0, 1, 1, 1]],
                        dtype=torch.int32, device=DEV)

    def fn(q, k, v):
        return stk.block_sparse_attention(q, k, v, mask, block_m=16, block_n=16, is_causal=False)

    q, k, v = _inputs()
    _check(fn, (q, k, v))
    out = fn(q, k, v)
    out.backward(torch.ones_like(out))
    assert torch.equal(out[:, :, 16:32], torch.zeros_like(out[:, :, 16:32]))
    assert torch.equal(q.grad[:, :, 16:32], torch.zeros_like(q.grad[:, :, 16:32]))
