"""StreamingLLM block masks and token masks.

Mirrors the reference's mask API (``sparse_triton_kernel.py:81-210, 905-932``):
same names, arguments, dtypes, shapes and exceptions. Masks requested on a GPU
device are built by the gfx950 library (``gki_streaming_mask`` /
``gki_dense_mask``); masks requested on the CPU (the FX injector always builds
its mask there, ``fx_compiler_pass.py:346-368``) are computed on the host with
the same closed form.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class StreamingMaskSpec:
    """StreamingLLM sparsity parameters (``sparse_triton_kernel.py:81-101``).

    ``sink_size`` leading keys are visible to every query; a query at absolute
    position ``q`` also sees keys in ``[q - window_size + 1, q]``.
    """

    sink_size: int
    window_size: int

    def __post_init__(self) -> None:
        if self.sink_size < 0 or self.window_size < 0:
            raise ValueError("sink_size and window_size must be non-negative")


def _check_blocks(block_m: int, block_n: int) -> None:
    if int(block_m) <= 0 or int(block_n) <= 0:
        raise ValueError("block_m and block_n must be positive")


def make_streaming_mask(
    n_q: int,
    n_kv: int,
    spec: StreamingMaskSpec,
    block_m: int,
    block_n: int,
    device: torch.device | str = "cuda",
) -> torch.Tensor:
    """Block-level StreamingLLM mask (``sparse_triton_kernel.py:104-181``).

    Returns an int32 ``[ceil(n_q/block_m), ceil(n_kv/block_n)]`` tensor. Block
    ``(i, j)`` is kept iff some query of row block ``i`` (absolute positions
    ``i*block_m + n_kv - n_q + [0, block_m)``, bottom-right aligned, unclipped)
    may see some key of column block ``j`` (``j*block_n + [0, block_n)``):
    ``q_last >= k_first and (k_first < S or k_last >= q_first - W + 1)``.
    """
    if n_q <= 0 or n_kv <= 0:
        raise ValueError("n_q and n_kv must be positive")
    _check_blocks(block_m, block_n)
    n_qb = -(-n_q // block_m)
    n_kb = -(-n_kv // block_n)
    dev = torch.device(device)
    if dev.type == "cuda":
        lib = _lib.load()
        out = torch.empty((n_qb, n_kb), dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            _lib.check(
                lib.gki_streaming_mask(out.data_ptr(), n_q, n_kv, spec.sink_size, spec.window_size,
                                       block_m, block_n, stream),
                "gki_streaming_mask",
            )
        return out
    offset = n_kv - n_q
    q_first = torch.arange(n_qb, dtype=torch.int64, device=dev).unsqueeze(1) * block_m + offset
    q_last = q_first + (block_m - 1)
    k_first = torch.arange(n_kb, dtype=torch.int64, device=dev).unsqueeze(0) * block_n
    k_last = k_first + (block_n - 1)
    reach = q_last >= k_first
    sink_or_window = (k_first < spec.sink_size) | (k_last >= q_first - spec.window_size + 1)
    return (reach & sink_or_window).to(torch.int32).contiguous()


def make_dense_mask(
    n_q: int,
    n_kv: int,
    block_m: int,
    block_n: int,
    causal: bool = False,
    device: torch.device | str = "cuda",
) -> torch.Tensor:
    """All-ones or dense-causal block mask (``sparse_triton_kernel.py:184-210``).

    Requires ``block_m | n_q`` and ``block_n | n_kv``. The causal variant keeps
    ``(i, j)`` iff ``j*block_n < (i+1)*block_m`` (no bottom-right offset).
    """
    _check_blocks(block_m, block_n)
    if n_q % block_m != 0 or n_kv % block_n != 0:
        raise ValueError("block_m / block_n must divide n_q / n_kv")
    n_qb, n_kb = n_q // block_m, n_kv // block_n
    dev = torch.device(device)
    if dev.type == "cuda":
        lib = _lib.load()
        out = torch.empty((n_qb, n_kb), dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            _lib.check(lib.gki_dense_mask(out.data_ptr(), n_q, n_kv, block_m, block_n,
                                          int(bool(causal)), stream), "gki_dense_mask")
        return out
    if not causal:
        return torch.ones((n_qb, n_kb), dtype=torch.int32, device=dev)
    rows_end = (torch.arange(n_qb, device=dev).unsqueeze(1) + 1) * block_m
    cols_start = torch.arange(n_kb, device=dev).unsqueeze(0) * block_n
    return (cols_start < rows_end).to(torch.int32).contiguous()


def streaming_token_mask(
    n_q: int,
    n_kv: int,
    sink_size: int,
    window_size: int,
    device: torch.device | str = "cpu",
) -> torch.Tensor:
    """Exact token-level StreamingLLM mask (``sparse_triton_kernel.py:905-932``).

    Bool ``[n_q, n_kv]``: ``(k <= q) & (k < S | k >= q - W + 1)`` with
    ``q = n_kv - n_q + row``. Theta(n_q * n_kv) memory: a test/oracle helper.
    """
    q_abs = torch.arange(n_kv - n_q, n_kv, device=device).unsqueeze(1)
    k_abs = torch.arange(n_kv, device=device).unsqueeze(0)
    return (k_abs <= q_abs) & ((k_abs < sink_size) | (k_abs >= q_abs - window_size + 1))
