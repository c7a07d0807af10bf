"""Autograd bridge and public op: block-sparse FlashAttention on gfx950.

Drop-in for the reference's ``_BlockSparseFlashAttention`` and
``block_sparse_attention`` (``sparse_triton_kernel.py:609-837``): same
signatures, same validation order, exception types and messages, same saved
state and gradient tuple. The Triton launches are replaced by calls into the
C ABI of ``libgki_bsa.so`` on the caller's current HIP stream:

* forward  -> ``gki_bsa_fwd`` (prefill) or, for the decode step (n_q <= 4,
  head_dim 64/128), ``gki_bsa_decode`` over the schedule's token list -- or
  ``gki_rolling_decode`` over the full cache (ring length n_kv - sink) when that
  list is the plain StreamingLLM stream, which the kernel then computes,
* backward -> ``gki_bsa_bwd`` (Delta, dK/dV, dQ).

There is no CPU or eager fallback: a missing library raises ``RuntimeError``.
"""

from __future__ import annotations

import contextlib
import math
from typing import Optional, Tuple

import torch

from . import _lib
from .lists import _CACHE, bwd_schedule, decode_schedule, fwd_order, fwd_schedule

_DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_HEAD_DIMS = (16, 32, 64, 128)
_DECODE_HEAD_DIMS = (64, 128)
# decode workgroups to aim for: one 768-thread group on each of the 256 CUs
_DECODE_TARGET_WGS = 256
# fp32 dK/dV work items wanted when the kv-tile columns are fewer: the fp32
# kernel runs one workgroup per CU, two per CU of the 256 keep them all busy
_FP32_DKDV_TARGET_ITEMS = 512


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous ``t`` starting on a 16-byte boundary (the kernels move Q / K /
    V / O in 16-byte chunks; a contiguous view at an odd storage offset is
    copied)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _device_mask(block_mask: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32 contiguous copy of the mask on ``device`` (cached for CPU masks)."""
    if block_mask.device == device and block_mask.dtype == torch.int32 and block_mask.is_contiguous():
        return block_mask
    if block_mask.device.type == "cpu":
        return _CACHE.get(block_mask, ("device-copy", str(device)),
                          lambda: block_mask.to(device=device, dtype=torch.int32).contiguous())
    return block_mask.to(device=device, dtype=torch.int32).contiguous()


def _current_stream(dev: torch.device) -> int:
    """Raw handle of ``dev``'s current stream (torch's stream query without its
    Python wrapper when available)."""
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    return raw(dev.index) if raw is not None else torch.cuda.current_stream(dev).cuda_stream


def _on_device(dev: torch.device):
    """``dev`` as the current device for the launches (a no-op context when it
    already is)."""
    return contextlib.nullcontext() if dev.index == torch.cuda.current_device() else torch.cuda.device(dev)


def _decode_splits(n_tokens: int, bh: int) -> int:
    """Decode workgroups per (b, head) slot: about one per CU in total, but at
    least ~256 tokens (a few rounds per wave) per workgroup."""
    want = -(-_DECODE_TARGET_WGS // bh)
    cap = max(1, n_tokens // 256)
    return max(1, min(want, cap))


def _decode_on_mfma(dtype_code: int, D: int, group: int, n_q: int, max_rows: int) -> bool:
    """The library's ``decode_on_mfma`` rule: a computed-stream decode whose
    group * n_q query rows per K / V stream are 2 .. 2 * ``max_rows``
    (decode_tile_m: one or two 16-column blocks), 16-bit, head_dim 64 / 128,
    runs on the matrix cores, one workgroup per K / V stream (and split)."""
    return dtype_code != 0 and D in (64, 128) and 2 <= group * n_q <= 2 * max_rows


def _decode_slots(B: int, H: int, H_kv: int, n_q: int, max_q: int, mfma: bool = False) -> int:
    """(b, head) slots of the decode grid: one per K / V stream on the matrix
    cores (``mfma``); else a grouped-query group's q heads share one workgroup
    when group * n_q fits the kernel's rows (the library's
    ``decode_heads_per_workgroup`` rule), else one q head per workgroup."""
    if mfma:
        return B * H_kv
    group = H // H_kv
    gq = group if group > 1 and group * n_q <= max_q else 1
    return B * H // gq


# decode launch plans: (dtype, B, H, H_kv, n_q, D, n_tokens, computed stream) ->
# (on the matrix cores, splits, split workspace floats); a few entries per model
_DECODE_PLANS: dict = {}


def _decode_plan(lib, dtype: int, B: int, H: int, H_kv: int, N_Q: int, D: int, n_tokens: int,
                 ring: bool) -> Tuple[bool, int, int]:
    key = (dtype, B, H, H_kv, N_Q, D, n_tokens, ring)
    plan = _DECODE_PLANS.get(key)
    if plan is None:
        if len(_DECODE_PLANS) >= 4096:      # a growing full cache adds one key per step
            _DECODE_PLANS.clear()
        ts = _lib.tile_sizes()
        mfma = ring and _decode_on_mfma(dtype, D, H // H_kv, N_Q, ts["decode_tile_m"])
        n_splits = _decode_splits(n_tokens, _decode_slots(B, H, H_kv, N_Q, ts["decode_max_q"], mfma))
        ws = int(lib.gki_bsa_decode_workspace_floats(B, H, N_Q, D, n_splits)) if n_splits > 1 else 0
        plan = _DECODE_PLANS[key] = (mfma, n_splits, ws)
    return plan


def _attention_forward(q, k, v, block_mask, softmax_scale, block_m, block_n, is_causal, sink_size,
                       window_size, enable_gqa, need_lse=True):
    """Validation and the forward launch (``sparse_triton_kernel.py:615-682``):
    returns (o, lse, q, k, v, block_mask, q_offset) with q / k / v / block_mask
    as the kernels read them (16-byte aligned, int32 mask on q's device).
    Without ``need_lse`` (inference) a decode step keeps its LSE and split
    workspace in one scratch allocation and returns lse None."""
    lib = _lib.load()
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("Q/K/V must be 4-D [B, H, N, D] tensors")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("All inputs must live on a CUDA device")

    B, H, N_Q, D = q.shape
    N_KV = k.shape[2]
    if k.shape != v.shape:
        raise ValueError("K and V must share shape")
    H_kv = k.shape[1]
    heads_ok = H_kv == H or (enable_gqa and H_kv > 0 and H % H_kv == 0)
    if k.shape[0] != B or not heads_ok or k.shape[-1] != D:
        raise ValueError("Q/K/V batch/head/dim mismatch")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DTYPE_CODE:
        raise ValueError(
            f"Q/K/V must share one dtype among float32/float16/bfloat16, got "
            f"{q.dtype}/{k.dtype}/{v.dtype}")
    if D not in _HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {_HEAD_DIMS}, got {D}")

    block_m, block_n = int(block_m), int(block_n)
    n_qb = (N_Q + block_m - 1) // block_m
    n_kb = (N_KV + block_n - 1) // block_n
    if block_mask.shape != (n_qb, n_kb):
        raise ValueError(
            f"block_mask has shape {tuple(block_mask.shape)}, "
            f"expected {(n_qb, n_kb)}"
        )
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    dev = q.device
    block_mask = _device_mask(block_mask, dev)

    o = torch.empty_like(q)
    lse = None
    q_offset = N_KV - N_Q
    dtype = _DTYPE_CODE[q.dtype]
    common = (block_mask.data_ptr(), n_qb, n_kb, block_m, block_n, float(softmax_scale),
              int(bool(is_causal)), int(sink_size), int(window_size))

    with _on_device(dev):
        stream = _current_stream(dev)
        ts = _lib.tile_sizes()
        if N_Q <= ts["decode_max_q"] and D in _DECODE_HEAD_DIMS:
            sched = decode_schedule(block_mask, N_Q, N_KV, block_m, block_n, bool(is_causal),
                                    int(sink_size), int(window_size))
            _, n_splits, ws_floats = _decode_plan(lib, dtype, B, H, H_kv, N_Q, D, sched.n_tokens,
                                                  bool(sched.ring))
            n_lse = B * H * N_Q
            if need_lse:
                lse = torch.empty((B, H, N_Q), dtype=torch.float32, device=dev)
                lse_ptr = lse.data_ptr()
                ws_ptr = 0
                if ws_floats:
                    ws = torch.empty(ws_floats, dtype=torch.float32, device=dev)
                    ws_ptr = ws.data_ptr()
            else:
                # one allocation: the LSE rows (padded to 256 bytes), then the workspace
                pad = (n_lse + 63) & ~63
                scratch = torch.empty(pad + ws_floats, dtype=torch.float32, device=dev)
                lse_ptr = scratch.data_ptr()
                ws_ptr = lse_ptr + 4 * pad if ws_floats else 0
            if sched.ring:
                # the stream is the StreamingLLM one: positions computed in
                # the kernel (no list read), same stream and arithmetic
                _lib.check(lib.gki_rolling_decode(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse_ptr,
                    dtype, B, H, H_kv, N_Q, D, int(sink_size), int(window_size), sched.ring,
                    N_KV, float(softmax_scale), ws_ptr, n_splits, stream), "gki_rolling_decode")
            else:
                _lib.check(lib.gki_bsa_decode(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse_ptr, dtype,
                    B, H, H_kv, N_Q, N_KV, D, sched.tokens.data_ptr(), sched.n_tokens, *common,
                    ws_ptr, n_splits, stream), "gki_bsa_decode")
        else:
            lse = torch.empty((B, H, N_Q), dtype=torch.float32, device=dev)
            sched = fwd_schedule(block_mask, N_Q, N_KV, block_m, block_n, bool(is_causal),
                                 int(sink_size), int(window_size), q.dtype == torch.float32)
            order = fwd_order(block_mask, sched, B * H)
            _lib.check(lib.gki_bsa_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), dtype,
                B, H, H_kv, N_Q, N_KV, D, sched.lists.row_ptr.data_ptr(),
                sched.lists.row_buf.data_ptr(), sched.n_qt, order.data_ptr(), *common, stream),
                "gki_bsa_fwd")

    return o, lse, q, k, v, block_mask, q_offset


class _BlockSparseFlashAttention(torch.autograd.Function):
    """Autograd bridge between PyTorch and the gfx950 kernels."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_mask: torch.Tensor,
        softmax_scale: float,
        block_m: int,
        block_n: int,
        is_causal: bool,
        sink_size: int,
        window_size: int,
        *extra,
    ) -> torch.Tensor:
        # extra = (enable_gqa,) when given: K / V may have H_kv heads dividing H
        enable_gqa = bool(extra[0]) if extra else False
        o, lse, q, k, v, block_mask, q_offset = _attention_forward(
            q, k, v, block_mask, softmax_scale, block_m, block_n, is_causal, sink_size, window_size,
            enable_gqa)
        ctx.save_for_backward(q, k, v, o, lse, block_mask)
        ctx.softmax_scale = softmax_scale
        ctx.block_m = block_m
        ctx.block_n = block_n
        ctx.is_causal = bool(is_causal)
        ctx.sink_size = int(sink_size)
        ctx.window_size = int(window_size)
        ctx.q_offset = int(q_offset)
        ctx.n_extra = len(extra)
        return o

    @staticmethod
    def backward(  # type: ignore[override]
        ctx, do: torch.Tensor
    ) -> Tuple[Optional[torch.Tensor], ...]:
        lib = _lib.load()
        q, k, v, o, lse, block_mask = ctx.saved_tensors
        do = _aligned(do.to(q.dtype))
        B, H, N_Q, D = q.shape
        H_kv, N_KV = k.shape[1], k.shape[2]
        n_qb = (N_Q + ctx.block_m - 1) // ctx.block_m
        n_kb = (N_KV + ctx.block_n - 1) // ctx.block_n

        dq = torch.empty_like(q)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        # row terms: Delta, then the base-2 LSE rows (internal to the backward)
        delta = torch.empty((2, B, H, N_Q), dtype=torch.float32, device=q.device)
        with _on_device(q.device):
            stream = _current_stream(q.device)
            spread = _FP32_DKDV_TARGET_ITEMS if q.dtype == torch.float32 else 0
            sched = bwd_schedule(block_mask, N_Q, N_KV, ctx.block_m, ctx.block_n, ctx.is_causal,
                                 ctx.sink_size, ctx.window_size, group=H // H_kv, bh_kv=B * H_kv,
                                 spread_to=spread)
            L = sched.lists
            # fp32 dK / dV partials of the split kv tiles: [B*H_kv, n_pslots, 2, 64, D]
            tile_n = _lib.tile_sizes()["tile_n"]
            partials = torch.empty(max(B * H_kv * sched.n_pslots * 2 * tile_n * D, 1),
                                   dtype=torch.float32, device=q.device)
            _lib.check(lib.gki_bsa_bwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(),
                _DTYPE_CODE[q.dtype], B, H, H_kv, N_Q, N_KV, D, L.row_ptr.data_ptr(),
                L.row_buf.data_ptr(), sched.n_qt, L.col_ptr.data_ptr(), L.col_buf.data_ptr(),
                sched.n_kt, sched.items.data_ptr(), sched.n_items, sched.split.data_ptr(),
                sched.n_split, sched.n_pslots, partials.data_ptr(), sched.dq_order.data_ptr(),
                block_mask.data_ptr(), n_qb,
                n_kb, ctx.block_m, ctx.block_n, float(ctx.softmax_scale), int(ctx.is_causal),
                ctx.sink_size, ctx.window_size, stream), "gki_bsa_bwd")
        return (dq, dk, dv) + (None,) * (7 + ctx.n_extra)


def block_sparse_attention(
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
    enable_gqa: bool = False,
) -> torch.Tensor:
    """Differentiable block-sparse FlashAttention (``sparse_triton_kernel.py:787-837``).

    ``q, k, v``: ``[B, H, N, D]`` on the GPU, one dtype among fp32/fp16/bf16,
    ``D`` in {16, 32, 64, 128}. ``block_mask``: ``[ceil(N_Q/block_m),
    ceil(N_KV/block_n)]``, non-zero = visit. With ``is_causal=True`` every
    visited tile also applies the token rule
    ``(k <= q) & (k < sink_size | k >= q - window_size + 1)`` with queries
    bottom-right aligned (``q = N_KV - N_Q + row``). ``softmax_scale`` defaults
    to ``1/sqrt(D)``. Rows that see no key produce zeros (and zero gradients).

    ``enable_gqa`` (as in ``F.scaled_dot_product_attention``; not in the
    reference, which requires equal head counts): K and V may have ``H_kv``
    heads dividing Q's ``H``; q head ``h`` attends kv head ``h // (H // H_kv)``,
    and dK / dV sum over each kv head's q heads.
    """
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    args = (q.contiguous(), k.contiguous(), v.contiguous(), block_mask, float(softmax_scale),
            int(block_m), int(block_n), bool(is_causal), int(sink_size), int(window_size))
    if not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)):
        # nothing to differentiate (inference, a decode step): the same forward
        # without the autograd node and its saved tensors
        return _attention_forward(*args, enable_gqa, need_lse=False)[0]
    if enable_gqa:
        args += (True,)
    return _BlockSparseFlashAttention.apply(*args)
