"""Ragged last tiles read nothing past the tensor (``gpu``).

The last q / kv tile of a length that is not a multiple of 64 is loaded
through a buffer resource over the rows that exist, so rows past the end read
as zero. Each tensor here is the leading block of a larger contiguous
allocation whose next rows hold NaN: a load past the last row would carry a
NaN into O or a gradient (P = 0 times NaN is NaN). Forward and backward must
stay finite and match the fp64 oracle at the usual tolerances.
"""

from __future__ import annotations

import math

import pytest
import torch

import sparse_triton_kernel as stk
from test_gpu_parity import _close, _oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _nan_tailed(rows: int, D: int, dtype, gen) -> torch.Tensor:
    """[1, 1, rows, D] view at the start of a [rows + 128, D] buffer whose
    128 extra rows are NaN."""
    buf = torch.full((rows + 128, D), float("nan"), dtype=dtype, device=DEV)
    buf[:rows] = torch.randn(rows, D, generator=gen).to(dtype).to(DEV)
    view = buf[:rows].view(1, 1, rows, D)
    assert view.is_contiguous() and view.data_ptr() == buf.data_ptr()
    return view


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n_q,n_kv,D,causal,S,W", [
    (1000, 1000, 64, True, 4, 128),      # ragged q and kv tiles, streaming causal
    (200, 1000, 128, True, 4, 300),      # fewer queries than keys
    (333, 333, 64, False, 0, 0),         # non-causal, every kept tile in full
])
def test_ragged_tiles_ignore_rows_past_the_end(dtype, n_q, n_kv, D, causal, S, W):
    g = torch.Generator().manual_seed(11)
    q = _nan_tailed(n_q, D, dtype, g)
    k = _nan_tailed(n_kv, D, dtype, g)
    v = _nan_tailed(n_kv, D, dtype, g)
    do = _nan_tailed(n_q, D, dtype, g)
    if causal:
        mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), 64, 64, device=DEV)
    else:
        mask = torch.ones((math.ceil(n_q / 64), math.ceil(n_kv / 64)), dtype=torch.int32, device=DEV)
    leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, is_causal=causal, sink_size=S, window_size=W)
    out.backward(do)
    scale = 1.0 / math.sqrt(D)
    o_ref, _, grads = _oracle(q, k, v, mask, 64, 64, causal, S, W, scale, do)
    tag = f"nq{n_q} nkv{n_kv} D{D} {dtype} causal{causal}"
    _close(out, o_ref, dtype, "O " + tag)
    for name, t, ref in zip(("dQ", "dK", "dV"), leaves, grads):
        _close(t.grad, torch.from_numpy(ref), dtype, f"{name} {tag}")
