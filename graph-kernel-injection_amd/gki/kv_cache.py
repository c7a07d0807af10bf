"""Rolling StreamingLLM KV cache for the decode step.

The reference decodes from a full ``[B, H, N_KV, D]`` cache
(``sparse_triton_kernel.py:636-641``) although a StreamingLLM query only ever
sees the ``S`` sink tokens and the last ``W`` tokens (``README.md:41-67``): its
Θ((S+W)·D) claim holds for HBM reads but not for memory. ``StreamingKVCache``
keeps only what can still be seen, per (b, h):

* ``sink_size`` sink slots: position ``p < S`` lives in slot ``p``;
* a ring of ``R = W + max_query - 1`` slots: position ``p >= S`` lives in slot
  ``S + (p - S) mod R`` -- the ring holds the last ``R`` positions, which is what
  ``max_query`` decode rows at the end of the sequence can see.

``append`` writes new tokens (a whole prefill or one token per step) with
``gki_rolling_append``; ``attend`` runs the decode kernel over the compact cache
with ``gki_rolling_decode``. Its token stream, split rule and arithmetic are
those of the full-cache decode (``block_sparse_attention`` with the StreamingLLM
mask and ``is_causal=True``), so both give the same bits.

For c4's shape (B8 H32 D128 bf16, S4 W2048) the cache holds 2055 of 100000
positions: 2 x 135 MB instead of 2 x 6.55 GB.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib
from .masks import StreamingMaskSpec
from .ops import _DTYPE_CODE, _aligned, _current_stream, _decode_plan, _on_device

_DECODE_HEAD_DIMS = (64, 128)


def ring_slot(position: int, sink_size: int, ring_size: int) -> int:
    """Cache slot of an absolute position (host-side statement of the layout)."""
    if position < sink_size:
        return position
    return sink_size + (position - sink_size) % ring_size


def rolling_stream(length: int, n_q: int, sink_size: int, window_size: int,
                   ring_size: int) -> Tuple[int, int, int]:
    """``(n_sink, window_lo, n_tokens)`` of the visible-token stream of the last
    ``n_q`` of ``length`` positions, as computed by the library."""
    lib = _lib.load()
    a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    _lib.check(lib.gki_rolling_stream(int(length), int(n_q), int(sink_size), int(window_size),
                                      int(ring_size), ctypes.byref(a), ctypes.byref(b),
                                      ctypes.byref(c)), "gki_rolling_stream")
    return a.value, b.value, c.value


class StreamingKVCache:
    """Sink + ring KV cache on the GPU for StreamingLLM decoding.

    ``k_cache`` / ``v_cache``: ``[B, H, sink_size + ring_size, D]`` in ``dtype``,
    ``H`` = ``heads`` = the K/V heads. Queries may have any multiple of ``heads``
    (grouped-query attention: q head h reads kv head h // (Hq // heads)).
    ``length`` counts the positions appended so far (0 .. length-1).
    """

    def __init__(self, batch: int, heads: int, head_dim: int, spec: StreamingMaskSpec,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda",
                 max_query: int = 4) -> None:
        if dtype not in _DTYPE_CODE:
            raise ValueError(f"dtype must be one of float32/float16/bfloat16, got {dtype}")
        if head_dim not in _DECODE_HEAD_DIMS:
            raise ValueError(f"head_dim must be one of {_DECODE_HEAD_DIMS}, got {head_dim}")
        max_q = _lib.tile_sizes()["decode_max_q"]
        if not 1 <= max_query <= max_q:
            raise ValueError(f"max_query must be in [1, {max_q}], got {max_query}")
        if batch <= 0 or heads <= 0:
            raise ValueError("batch and heads must be positive")
        self.spec = spec
        self.batch, self.heads, self.head_dim = int(batch), int(heads), int(head_dim)
        self.dtype = dtype
        self.max_query = int(max_query)
        self.sink_size = int(spec.sink_size)
        self.window_size = int(spec.window_size)
        self.ring_size = max(1, self.window_size + self.max_query - 1)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("StreamingKVCache lives on a CUDA (HIP) device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        shape = (self.batch, self.heads, self.sink_size + self.ring_size, self.head_dim)
        self.k_cache = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v_cache = torch.zeros(shape, dtype=dtype, device=self.device)
        self.length = 0

    @property
    def capacity(self) -> int:
        return self.sink_size + self.ring_size

    def reset(self) -> None:
        self.length = 0

    def _check_tokens(self, name: str, t: torch.Tensor, grouped: bool = False) -> None:
        heads_ok = t.dim() == 4 and (t.shape[1] == self.heads or
                                     (grouped and t.shape[1] % self.heads == 0 and t.shape[1] > 0))
        if t.dim() != 4 or t.shape[0] != self.batch or not heads_ok or t.shape[3] != self.head_dim:
            want = "a multiple of " + str(self.heads) if grouped else str(self.heads)
            raise ValueError(f"{name} must be [{self.batch}, {want}, n, {self.head_dim}], "
                             f"got {tuple(t.shape)}")
        if t.dtype != self.dtype:
            raise ValueError(f"{name} must be {self.dtype}, got {t.dtype}")
        if t.device != self.device:
            raise ValueError(f"{name} must live on {self.device}")

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append ``[B, H, n, D]`` keys / values at positions length .. length+n-1."""
        self._check_tokens("k", k)
        self._check_tokens("v", v)
        if k.shape != v.shape:
            raise ValueError("k and v must share shape")
        n = int(k.shape[2])
        if n == 0:
            return
        k, v = _aligned(k), _aligned(v)
        lib = _lib.load()
        with _on_device(self.device):
            stream = _current_stream(self.device)
            _lib.check(lib.gki_rolling_append(
                self.k_cache.data_ptr(), self.v_cache.data_ptr(), k.data_ptr(), v.data_ptr(),
                _DTYPE_CODE[self.dtype], self.batch, self.heads, self.head_dim, self.sink_size,
                self.ring_size, self.length, n, stream), "gki_rolling_append")
        self.length += n

    def attend(self, q: torch.Tensor, softmax_scale: Optional[float] = None,
               return_lse: bool = False):
        """Decode attention of ``q`` (``[B, Hq, n_q, D]``, the last n_q positions
        of the cache; Hq a multiple of the cache's heads) over the visible
        tokens: ``O`` (and the natural-log LSE ``[B, Hq, n_q]`` fp32 when
        ``return_lse``)."""
        self._check_tokens("q", q, grouped=True)
        n_q = int(q.shape[2])
        if not 1 <= n_q <= self.max_query:
            raise ValueError(f"q must hold 1..{self.max_query} rows, got {n_q}")
        if n_q > self.length:
            raise ValueError(f"q has {n_q} rows but the cache holds {self.length} positions")
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(self.head_dim)
        q = _aligned(q)
        _, _, n_tokens = rolling_stream(self.length, n_q, self.sink_size, self.window_size,
                                        self.ring_size)
        B, H, H_kv = self.batch, int(q.shape[1]), self.heads
        lib = _lib.load()
        dtype = _DTYPE_CODE[self.dtype]
        _, n_splits, ws_floats = _decode_plan(lib, dtype, B, H, H_kv, n_q, self.head_dim, n_tokens, True)
        o = torch.empty_like(q)
        # the LSE rows (padded to 256 bytes), then the split workspace: one allocation
        pad = (B * H * n_q + 63) & ~63
        scratch = torch.empty(pad + ws_floats, dtype=torch.float32, device=self.device)
        with _on_device(self.device):
            stream = _current_stream(self.device)
            _lib.check(lib.gki_rolling_decode(
                q.data_ptr(), self.k_cache.data_ptr(), self.v_cache.data_ptr(), o.data_ptr(),
                scratch.data_ptr(), dtype, B, H, H_kv, n_q, self.head_dim, self.sink_size,
                self.window_size, self.ring_size, self.length, float(softmax_scale),
                scratch.data_ptr() + 4 * pad if ws_floats else 0, n_splits, stream),
                "gki_rolling_decode")
        if not return_lse:
            return o
        return o, scratch[:B * H * n_q].view(B, H, n_q).clone()

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             softmax_scale: Optional[float] = None) -> torch.Tensor:
        """One decode step: append the new tokens' K / V, then attend with q."""
        self.append(k, v)
        return self.attend(q, softmax_scale)
