"""CPU oracle for the StreamingLLM block-sparse attention path (numpy, fp64).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker. The product (``graph-kernel-injection_amd/``) never imports it.

Each function restates one piece of the reference algorithm and cites it.
How each is pinned (by the tests in ``tests/test_oracle_pins.py``):

* ``block_mask``          -- sparse_triton_kernel.py:154-181. Pinned by brute
  force over token pairs (for W >= 1 a block is kept iff some token pair of its
  unclipped ranges is visible; W = 0 keeps the documented quirk), by the
  superset / ceil-div shape / decode S+W checks of the reference's tests, and
  by the kept counts 81 / 8143 / 2151 / 34 / 67519 of the five configs.
* ``token_mask``          -- sparse_triton_kernel.py:905-932. Pinned against
  the position-by-position ``visible`` loop (tests/test_streaming_definition.py:45-67
  restated) on the reference's 13 shapes.
* ``dense_block_mask``    -- sparse_triton_kernel.py:184-210. Pinned by brute force.
* ``kept_lists``          -- build-only (CSR/CSC). Pinned by ``np.nonzero``.
* ``dkdv_items``          -- build-only dK/dV work list. Pinned by its
  invariants: every kv tile's iterations covered once, in order, by items of
  at most ``chunk`` iterations whose lengths differ by at most one; slots
  numbered consecutively per split tile; the unsplit case one item per tile.
* ``tile_classes``        -- build-only tile classification. Pinned per tile
  against ``effective_mask`` (visited iff some effective element; class 1 iff
  the effective mask equals the token rule there).
* ``expand_kv_heads`` / ``reduce_kv_grad`` -- build-only grouped-query
  extension. Pinned against torch's repeat_interleave and its autograd
  adjoint, and (through ``attention_fwd``) against torch's SDPA with
  ``enable_gqa=True``, which fixes the head mapping h -> h // group.
* ``attention_fwd/bwd``   -- sparse_triton_kernel.py:845-902 (eager oracle) with
  the kernel's LSE sentinel (:341-352). Pinned against a pure-Python loop on
  tiny inputs, torch's math SDPA with an explicit mask, torch autograd
  through the reference formulation, finite differences, and the identities
  sum_k dS = 0 and Delta = rowsum(dO*O) = rowsum(P*dP).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np


# ---------------------------------------------------------------------------
# Masks
# ---------------------------------------------------------------------------


def visible(q_abs: int, k_abs: int, sink: int, window: int) -> bool:
    """Token rule (k <= q) and (k < S or q - k < W)."""
    if k_abs > q_abs:
        return False
    return k_abs < sink or q_abs - k_abs < window


def token_mask(n_q: int, n_kv: int, sink: int, window: int) -> np.ndarray:
    """Bool [n_q, n_kv]; query row r sits at absolute position n_kv - n_q + r
    (sparse_triton_kernel.py:905-932)."""
    q = np.arange(n_kv - n_q, n_kv, dtype=np.int64)[:, None]
    k = np.arange(n_kv, dtype=np.int64)[None, :]
    return (k <= q) & ((k < sink) | (k >= q - window + 1))


def block_mask(n_q: int, n_kv: int, sink: int, window: int, bm: int, bn: int) -> np.ndarray:
    """int32 [ceil(n_q/bm), ceil(n_kv/bn)] (sparse_triton_kernel.py:154-181).

    q_lo = i*bm + (n_kv - n_q), q_hi = q_lo + bm, k_lo = j*bn, k_hi = k_lo + bn;
    keep iff q_hi > k_lo and (k_lo < S or k_hi - 1 >= q_lo - W + 1).
    """
    if n_q <= 0 or n_kv <= 0:
        raise ValueError("n_q and n_kv must be positive")
    n_qb = -(-n_q // bm)
    n_kb = -(-n_kv // bn)
    q_lo = np.arange(n_qb, dtype=np.int64)[:, None] * bm + (n_kv - n_q)
    q_hi = q_lo + bm
    k_lo = np.arange(n_kb, dtype=np.int64)[None, :] * bn
    k_hi = k_lo + bn
    keep = (q_hi > k_lo) & ((k_lo < sink) | (k_hi - 1 >= q_lo - window + 1))
    return keep.astype(np.int32)


def dense_block_mask(n_q: int, n_kv: int, bm: int, bn: int, causal: bool) -> np.ndarray:
    """sparse_triton_kernel.py:184-210 (requires divisibility)."""
    if n_q % bm or n_kv % bn:
        raise ValueError("block_m / block_n must divide n_q / n_kv")
    n_qb, n_kb = n_q // bm, n_kv // bn
    if not causal:
        return np.ones((n_qb, n_kb), np.int32)
    i = np.arange(n_qb)[:, None]
    j = np.arange(n_kb)[None, :]
    return (j * bn < (i + 1) * bm).astype(np.int32)


def lift(mask: np.ndarray, bm: int, bn: int, n_q: int, n_kv: int) -> np.ndarray:
    """Block mask -> token mask by repetition, clipped (sparse_triton_kernel.py:877-879)."""
    return np.repeat(np.repeat(mask.astype(bool), bm, axis=0), bn, axis=1)[:n_q, :n_kv]


def effective_mask(mask: np.ndarray, n_q: int, n_kv: int, bm: int, bn: int, causal: bool,
                   sink: int, window: int) -> np.ndarray:
    """lift(mask) & token_mask when causal, else lift(mask) (sparse_triton_kernel.py:881-894)."""
    eff = lift(mask, bm, bn, n_q, n_kv)
    if causal:
        eff = eff & token_mask(n_q, n_kv, sink, window)
    return eff


# ---------------------------------------------------------------------------
# Kept-block lists and the kernels' tile classification (build-only)
# ---------------------------------------------------------------------------


def kept_lists(m: np.ndarray) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """CSR (row -> ascending cols) and CSC (col -> ascending rows), int32.
    Entries carry ``<< 30`` flags for value 2 (partially kept tiles)."""
    m = np.asarray(m)
    flag = (m == 2).astype(np.int64) << 30
    rows, cols = np.nonzero(m)
    row_ptr = np.concatenate([[0], np.cumsum((m != 0).sum(axis=1))]).astype(np.int32)
    row_idx = (cols + flag[rows, cols]).astype(np.int32)
    cols_t, rows_t = np.nonzero(m.T)
    col_ptr = np.concatenate([[0], np.cumsum((m != 0).sum(axis=0))]).astype(np.int32)
    col_idx = (rows_t + flag[rows_t, cols_t]).astype(np.int32)
    return row_ptr, row_idx, col_ptr, col_idx


def tile_classes(mask: np.ndarray, n_q: int, n_kv: int, bm: int, bn: int, tm: int, tn: int,
                 causal: bool = False, sink: int = 0, window: int = 0) -> np.ndarray:
    """Per tm x tn tile of the kernels: 0 = no in-bounds element is visible
    (kept by lift(mask) and, when causal, allowed by the token rule); 1 = the
    lifted mask keeps every element the token rule allows (all elements when
    not causal), so the kernel needs only the token rule; 2 = otherwise."""
    lifted = lift(mask, bm, bn, n_q, n_kv)
    tok = token_mask(n_q, n_kv, sink, window) if causal else np.ones((n_q, n_kv), bool)
    n_qt, n_kt = -(-n_q // tm), -(-n_kv // tn)
    out = np.zeros((n_qt, n_kt), np.int32)
    for a in range(n_qt):
        for b in range(n_kt):
            sl = (slice(a * tm, (a + 1) * tm), slice(b * tn, (b + 1) * tn))
            allowed, kept = tok[sl], lifted[sl]
            if (allowed & kept).any():
                out[a, b] = 2 if (allowed & ~kept).any() else 1
    return out


def dkdv_items(col_ptr: np.ndarray, group: int, bh_kv: int, chunk: Optional[int] = None,
               min_chunk: int = 32, target_items: int = 8192, max_chunk: int = 0):
    """The dK/dV work list (build-only; the reference runs one program per kv
    tile, sparse_triton_kernel.py:719-777). A kv tile's walk of group x (its
    column length) iterations is one item (slot -1) when it fits the chunk,
    else ``parts = ceil(n_it / chunk)`` items ``[n_it*c/parts, n_it*(c+1)/parts)``
    writing consecutive partial slots. ``chunk`` defaults to
    ``max(min_chunk, ceil(total / target_items))`` with
    ``total = sum(len) * group * bh_kv``, then ``min(chunk, max_chunk)`` when
    ``max_chunk > 0``. Returns (items [n, 4], split [m, 3],
    n_pslots) as int32 arrays: items (kv tile, first, end, slot | -1), split
    (kv tile, first slot, slot count)."""
    cnt = np.diff(col_ptr.astype(np.int64))
    if chunk is None:
        total = int(cnt.sum()) * group * bh_kv
        chunk = max(min_chunk, -(-total // target_items))
        if max_chunk > 0:
            chunk = min(chunk, max_chunk)
    items, split, n_pslots = [], [], 0
    for kt, n in enumerate(cnt):
        n_it = int(n) * group
        parts = max(1, -(-n_it // chunk))
        if parts == 1:
            items.append((kt, 0, n_it, -1))
            continue
        split.append((kt, n_pslots, parts))
        items += [(kt, n_it * c // parts, n_it * (c + 1) // parts, n_pslots + c) for c in range(parts)]
        n_pslots += parts
    return (np.array(items, np.int32).reshape(-1, 4), np.array(split, np.int32).reshape(-1, 3),
            n_pslots)


# ---------------------------------------------------------------------------
# Attention (fp64)
# ---------------------------------------------------------------------------


def _probs(q: np.ndarray, k: np.ndarray, eff: np.ndarray, scale: float):
    s = np.einsum("...qd,...kd->...qk", q, k) * scale
    s = np.where(eff, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(m)
    m = np.where(empty, 0.0, m)
    e = np.where(eff, np.exp(s - m), 0.0)
    l = e.sum(axis=-1, keepdims=True)
    p = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)
    lse = np.where(l[..., 0] > 0, m[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)), 0.0)
    return p, lse


def attention_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, eff: np.ndarray,
                  scale: Optional[float] = None) -> Tuple[np.ndarray, np.ndarray]:
    """O = softmax(masked(Q K^T * scale)) V and LSE (natural log).

    Rows with no visible key give O = 0 and LSE = 0 (the kernel sentinel of
    sparse_triton_kernel.py:341-352; the eager oracle's nan_to_num gives O = 0).
    ``eff`` is a bool [n_q, n_kv] mask shared over the leading dims.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    p, lse = _probs(q, k, eff, scale)
    return p @ v, lse


def attention_bwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, do: np.ndarray, eff: np.ndarray,
                  scale: Optional[float] = None) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Closed-form gradients of ``attention_fwd``'s O w.r.t. (Q, K, V).

    dV = P^T dO; dP = dO V^T; dS = P * (dP - rowsum(P * dP)); dQ = scale dS K;
    dK = scale dS^T Q. Empty rows have P = 0 and contribute nothing.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    do = np.asarray(do, np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    p, _ = _probs(q, k, eff, scale)
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (p * dp).sum(axis=-1, keepdims=True))
    dq = scale * (ds @ k)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    return dq, dk, dv


def expand_kv_heads(t: np.ndarray, group: int) -> np.ndarray:
    """Grouped-query attention: [B, H_kv, N, D] -> [B, H_kv * group, N, D], q head
    h reading kv head h // group (build-only extension; torch SDPA's enable_gqa
    convention, repeat_interleave over the head axis)."""
    return np.repeat(np.asarray(t), group, axis=1)


def reduce_kv_grad(g: np.ndarray, group: int) -> np.ndarray:
    """Adjoint of ``expand_kv_heads``: dK / dV of a kv head = sum of its
    group's per-q-head gradients."""
    g = np.asarray(g)
    B, H, N, D = g.shape
    return g.reshape(B, H // group, group, N, D).sum(axis=2)


def attention_loop(q: np.ndarray, k: np.ndarray, v: np.ndarray, eff: np.ndarray,
                   scale: float) -> np.ndarray:
    """Pure-Python loop restatement for tiny 2-D inputs (brute-force pin)."""
    n_q, d = q.shape
    out = np.zeros((n_q, v.shape[1]))
    for r in range(n_q):
        keys = [c for c in range(k.shape[0]) if eff[r, c]]
        if not keys:
            continue
        logits = [scale * sum(float(q[r, i]) * float(k[c, i]) for i in range(d)) for c in keys]
        mx = max(logits)
        w = [math.exp(x - mx) for x in logits]
        tot = sum(w)
        for c, wi in zip(keys, w):
            out[r] += (wi / tot) * v[c]
    return out
