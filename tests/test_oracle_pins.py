"""Pins of the CPU oracle against brute force, textbook routines and the
reference's own test semantics (tests/test_streaming_definition.py,
tests/test_mask_equivalence.py, tests/test_oracle.py of the reference).

Each check is chosen so a plausible slip in the oracle (dropped term, wrong
sign or offset, transposed operand) fails it; none retypes the oracle's own
formula.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import chunked_reference as cr
from oracle import streaming_oracle as so

# (n_q, n_kv, sink, window) -- the reference's TOKEN_SHAPES
TOKEN_SHAPES = [
    (1, 1000, 4, 256), (1, 1000, 0, 256), (1, 1000, 4, 0), (1, 1000, 4, 2048),
    (16, 16, 4, 8), (64, 64, 4, 16), (2, 10, 4, 4), (1000, 1000, 4, 128),
    (1023, 1023, 4, 128), (1025, 1025, 4, 128), (4, 10, 8, 4), (16, 1000, 4, 128),
    (128, 1024, 4, 128),
]
# (n_q, n_kv, sink, window, bm, bn) -- the reference's BLOCK_SHAPES + SHAPES
BLOCK_SHAPES = [
    (1, 1000, 4, 256, 1, 64), (1, 1023, 4, 256, 1, 64), (1, 1025, 4, 256, 1, 64),
    (16, 1000, 4, 128, 16, 64), (1000, 1000, 4, 128, 64, 64), (1023, 1023, 4, 128, 64, 64),
    (1025, 1025, 4, 128, 64, 64), (4, 10, 8, 4, 2, 2), (16, 16, 4, 8, 8, 8),
    (128, 1024, 4, 128, 16, 64), (32, 32, 4, 8, 8, 8), (64, 64, 4, 16, 16, 16),
    (64, 128, 4, 32, 16, 32), (128, 128, 8, 32, 32, 32), (256, 256, 4, 64, 64, 64),
    (128, 1024, 4, 128, 64, 64), (64, 64, 0, 64, 16, 16), (64, 64, 64, 0, 16, 16),
]


def _hand_token_mask(n_q, n_kv, sink, window):
    out = np.zeros((n_q, n_kv), bool)
    for r in range(n_q):
        q = n_kv - n_q + r
        for k in range(n_kv):
            out[r, k] = so.visible(q, k, sink, window)
    return out


@pytest.mark.parametrize("n_q,n_kv,sink,window", TOKEN_SHAPES)
def test_token_mask_matches_position_loop(n_q, n_kv, sink, window):
    np.testing.assert_array_equal(so.token_mask(n_q, n_kv, sink, window),
                                  _hand_token_mask(n_q, n_kv, sink, window))


def test_visible_rule_by_hand():
    # q=10, S=2, W=3: sees keys 0, 1 (sink) and 8, 9, 10 (window)
    assert [k for k in range(12) if so.visible(10, k, 2, 3)] == [0, 1, 8, 9, 10]


def test_decode_sees_sink_plus_window():
    assert so.token_mask(1, 1000, 4, 256).sum() == 260


def test_sink_does_not_leak_future():
    np.testing.assert_array_equal(so.token_mask(4, 4, 4, 1), np.tril(np.ones((4, 4), bool)))


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", BLOCK_SHAPES)
def test_block_mask_superset_and_shape(n_q, n_kv, sink, window, bm, bn):
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    assert m.shape == (-(-n_q // bm), -(-n_kv // bn))
    assert m.dtype == np.int32
    tok = _hand_token_mask(n_q, n_kv, sink, window)
    assert not (tok & ~so.lift(m, bm, bn, n_q, n_kv)).any()


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", BLOCK_SHAPES)
def test_effective_mask_equals_token_mask(n_q, n_kv, sink, window, bm, bn):
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    eff = so.effective_mask(m, n_q, n_kv, bm, bn, True, sink, window)
    np.testing.assert_array_equal(eff, _hand_token_mask(n_q, n_kv, sink, window))


def _brute_block_mask(n_q, n_kv, sink, window, bm, bn):
    """Keep (i, j) iff some token pair of the unclipped block ranges is visible;
    for window == 0 the reference formula additionally keeps causal blocks with
    k_hi - 1 >= q_lo + 1 (its window term does not vanish at W = 0)."""
    n_qb, n_kb = -(-n_q // bm), -(-n_kv // bn)
    off = n_kv - n_q
    out = np.zeros((n_qb, n_kb), np.int32)
    for i, j in itertools.product(range(n_qb), range(n_kb)):
        qs = range(i * bm + off, i * bm + off + bm)
        ks = range(j * bn, j * bn + bn)
        hit = any(so.visible(q, k, sink, window) for q in qs for k in ks)
        if window == 0 and not hit:
            hit = (max(qs) >= min(ks)) and (max(ks) >= min(qs) + 1)
        out[i, j] = int(hit)
    return out


@pytest.mark.parametrize("seed", range(40))
def test_block_mask_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n_q = int(rng.integers(1, 40))
    n_kv = int(rng.integers(n_q, 80))
    sink = int(rng.integers(0, 6))
    window = int(rng.integers(0, 20)) if seed % 5 else 0
    bm, bn = int(rng.integers(1, 9)), int(rng.integers(1, 9))
    np.testing.assert_array_equal(so.block_mask(n_q, n_kv, sink, window, bm, bn),
                                  _brute_block_mask(n_q, n_kv, sink, window, bm, bn))


# Kept counts of the five BASELINE configs, derived independently in the
# survey from the reference formula (sparse_triton_kernel.py:159-180).
CONFIG_COUNTS = [
    ((1024, 1024, 4, 256, 64, 64), 81),
    ((16384, 16384, 4, 2048, 64, 64), 8143),
    ((8192, 8192, 4, 1024, 64, 64), 2151),
    ((1, 100000, 4, 2048, 1, 64), 34),
    ((131072, 131072, 4, 4096, 128, 64), 67519),
]


@pytest.mark.parametrize("shape,count", CONFIG_COUNTS)
def test_config_kept_counts(shape, count):
    assert int(so.block_mask(*shape).sum()) == count


def test_decode_config_kept_tiles():
    m = so.block_mask(1, 100000, 4, 2048, 1, 64)
    assert list(np.nonzero(m[0])[0]) == [0] + list(range(1530, 1563))


def test_dense_block_mask_brute_force():
    for n_q, n_kv, bm, bn in [(64, 128, 16, 32), (32, 32, 8, 8), (48, 96, 16, 16)]:
        full = so.dense_block_mask(n_q, n_kv, bm, bn, False)
        assert full.shape == (n_q // bm, n_kv // bn) and full.all()
        causal = so.dense_block_mask(n_q, n_kv, bm, bn, True)
        for i, j in itertools.product(range(n_q // bm), range(n_kv // bn)):
            # some key of block j precedes the end of row block i (no offset)
            assert causal[i, j] == int(any(k < (i + 1) * bm for k in range(j * bn, (j + 1) * bn)))
    with pytest.raises(ValueError):
        so.dense_block_mask(10, 16, 4, 4, False)


def test_kept_lists_against_nonzero():
    rng = np.random.default_rng(0)
    m = (rng.random((13, 21)) < 0.3).astype(np.int32)
    m[3] = 0
    row_ptr, row_idx, col_ptr, col_idx = so.kept_lists(m)
    for r in range(13):
        assert list(row_idx[row_ptr[r]:row_ptr[r + 1]]) == [c for c in range(21) if m[r, c]]
    for c in range(21):
        assert list(col_idx[col_ptr[c]:col_ptr[c + 1]]) == [r for r in range(13) if m[r, c]]
    nz = np.argwhere(m)
    np.testing.assert_array_equal(row_idx, nz[:, 1])
    # partial flag
    m2 = m.copy()
    m2[0, 0] = 2
    _, ri2, _, ci2 = so.kept_lists(m2)
    assert ri2[0] == (1 << 30) | 0 and ci2[0] == (1 << 30) | 0


def test_tile_classes_aligned_and_unaligned():
    m = so.block_mask(300, 300, 4, 64, 64, 64)
    t = so.tile_classes(m, 300, 300, 64, 64, 64, 64)
    np.testing.assert_array_equal(t, m)            # same granularity: 0/1 only
    m16 = so.block_mask(300, 300, 4, 64, 16, 16)
    t16 = so.tile_classes(m16, 300, 300, 16, 16, 64, 64)
    lifted = so.lift(m16, 16, 16, 300, 300)
    for a, b in itertools.product(range(t16.shape[0]), range(t16.shape[1])):
        blk = lifted[64 * a:64 * a + 64, 64 * b:64 * b + 64]
        assert t16[a, b] == (0 if blk.sum() == 0 else (1 if blk.sum() == blk.size else 2))
    assert (t16 == 2).any()


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn,tm,tn",
                         [(300, 300, 4, 64, 16, 16, 64, 64), (300, 300, 4, 64, 16, 16, 128, 64),
                          (200, 333, 2, 50, 8, 128, 128, 64), (130, 260, 0, 1, 32, 32, 64, 64),
                          (1, 700, 4, 100, 1, 64, 16, 64), (257, 257, 3, 0, 64, 64, 128, 64),
                          (300, 300, 4, 64, 64, 64, 64, 64)])
def test_tile_classes_causal_against_effective_mask(n_q, n_kv, sink, window, bm, bn, tm, tn):
    """Each tile's class follows from the effective (kernel-visible) mask:
    visited iff some element is visible; class 1 iff, inside the tile, the
    effective mask equals the token rule alone (so the kernel may skip the
    mask lookup); class 2 otherwise. A random mask with holes exercises 2."""
    rng = np.random.default_rng(n_q * 7 + n_kv)
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    m_holes = m * (rng.random(m.shape) < 0.7)
    for mm in (m, m_holes):
        t = so.tile_classes(mm, n_q, n_kv, bm, bn, tm, tn, True, sink, window)
        eff = so.effective_mask(mm, n_q, n_kv, bm, bn, True, sink, window)
        tok = np.array([[so.visible(n_kv - n_q + i, j, sink, window) for j in range(n_kv)]
                        for i in range(n_q)])
        for a, b in itertools.product(range(t.shape[0]), range(t.shape[1])):
            sl = (slice(tm * a, tm * a + tm), slice(tn * b, tn * b + tn))
            if not eff[sl].any():
                assert t[a, b] == 0
            else:
                assert t[a, b] == (1 if (eff[sl] == tok[sl]).all() else 2)
        # the streaming mask itself never needs a per-element lookup when the
        # tile and block grids coincide
        if mm is m and (bm, bn) == (tm, tn):
            assert not (t == 2).any()


def _check_work_list(col_ptr, group, items, split, n_pslots, chunk):
    """Invariants of a dK/dV work list over CSC column pointers."""
    cnt = np.diff(col_ptr.astype(np.int64)) * group
    assert items.shape[1] == 4 and split.shape[1] == 3
    assert sorted(set(items[:, 0].tolist())) == list(range(len(cnt)))
    assert (np.diff(items[:, 0]) >= 0).all()               # tiles in order
    splits = {int(kt): (int(p0), int(n)) for kt, p0, n in split}
    next_slot = 0
    for kt, n_it in enumerate(cnt):
        it = items[items[:, 0] == kt]
        assert it[0, 1] == 0 and it[-1, 2] == n_it         # covers [0, n_it)
        assert (it[1:, 1] == it[:-1, 2]).all()             # contiguous, no overlap
        lens = it[:, 2] - it[:, 1]
        if len(it) == 1:
            assert it[0, 3] == -1 and kt not in splits and n_it <= chunk
            continue
        assert lens.max() <= chunk and lens.max() - lens.min() <= 1
        assert len(it) == -(-n_it // chunk)
        p0, n = splits[kt]
        assert p0 == next_slot and n == len(it)
        assert it[:, 3].tolist() == list(range(p0, p0 + n))
        next_slot += n
    assert n_pslots == next_slot


def test_dkdv_work_list_invariants():
    rng = np.random.default_rng(5)
    for _ in range(60):
        n_kt = int(rng.integers(1, 40))
        cnt = rng.integers(0, 90, n_kt)
        cnt[rng.random(n_kt) < 0.2] = 0
        col_ptr = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
        group, bh_kv = int(rng.choice([1, 2, 4, 8])), int(rng.integers(1, 64))
        for chunk in (None, 1, int(rng.integers(2, 50))):
            items, split, n_pslots = so.dkdv_items(col_ptr, group, bh_kv, chunk=chunk)
            c = chunk or max(32, -(-int(cnt.sum()) * group * bh_kv // 8192))
            _check_work_list(col_ptr, group, items, split, n_pslots, c)
        # a cap below the default chunk (the fp32 work list) bounds every item
        items, split, n_pslots = so.dkdv_items(col_ptr, group, bh_kv, max_chunk=4)
        _check_work_list(col_ptr, group, items, split, n_pslots, 4)


def test_dkdv_work_list_splits_only_long_columns():
    """Config 5's mask (S 4, W 4096, 64x64 tiles, N 131072): the sink column
    (all 2048 q tiles) is cut; window columns (<= 65 q tiles) are not. A huge
    chunk gives one item per tile and no split."""
    m = so.block_mask(131072, 131072, 4, 4096, 64, 64)
    _, _, col_ptr, _ = so.kept_lists(m)
    items, split, n_pslots = so.dkdv_items(col_ptr, 1, 16)
    assert split[:, 0].tolist() == [0]
    assert split[0, 2] == n_pslots == -(-2048 // max(32, -(-int(col_ptr[-1]) * 16 // 8192)))
    items, split, n_pslots = so.dkdv_items(col_ptr, 1, 16, chunk=1 << 20)
    assert len(items) == len(col_ptr) - 1 and len(split) == 0 and n_pslots == 0
    assert (items[:, 3] == -1).all()


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def _torch_reference(q, k, v, eff, scale):
    """The reference's eager formulation (sparse_triton_kernel.py:898-902) in torch."""
    s = torch.matmul(q, k.transpose(-2, -1)) * scale
    s = s.masked_fill(~eff, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    return torch.matmul(p, v)


def test_attention_fwd_matches_python_loop():
    q, k, v = _rand((5, 3), 1), _rand((9, 3), 2), _rand((9, 4), 3)
    eff = so.token_mask(5, 9, 1, 3)
    eff[2] = False                                 # an empty row
    o, lse = so.attention_fwd(q, k, v, eff, 0.7)
    np.testing.assert_allclose(o, so.attention_loop(q, k, v, eff, 0.7), atol=1e-12)
    assert np.all(o[2] == 0) and lse[2] == 0


def test_attention_fwd_matches_sdpa_and_logsumexp():
    from scipy.special import logsumexp

    B, H, n_q, n_kv, D = 2, 3, 40, 70, 16
    q, k, v = _rand((B, H, n_q, D), 4), _rand((B, H, n_kv, D), 5), _rand((B, H, n_kv, D), 6)
    eff = so.token_mask(n_q, n_kv, 4, 12)
    scale = 1 / math.sqrt(D)
    o, lse = so.attention_fwd(q, k, v, eff, scale)
    sdpa = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
        attn_mask=torch.from_numpy(eff), scale=scale)
    np.testing.assert_allclose(o, sdpa.numpy(), atol=1e-12, rtol=1e-12)
    logits = np.where(eff, np.einsum("bhqd,bhkd->bhqk", q, k) * scale, -np.inf)
    np.testing.assert_allclose(lse, logsumexp(logits, axis=-1), atol=1e-12)


@pytest.mark.parametrize("empty_row", [False, True])
def test_attention_bwd_matches_autograd(empty_row):
    B, H, n_q, n_kv, D = 1, 2, 24, 40, 8
    q, k, v = _rand((B, H, n_q, D), 7), _rand((B, H, n_kv, D), 8), _rand((B, H, n_kv, D), 9)
    do = _rand((B, H, n_q, D), 10)
    eff = so.token_mask(n_q, n_kv, 2, 6)
    if empty_row:
        eff[5] = False
    scale = 0.37
    dq, dk, dv = so.attention_bwd(q, k, v, do, eff, scale)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    out = _torch_reference(tq, tk, tv, torch.from_numpy(eff), scale)
    out.backward(torch.from_numpy(do))
    for ours, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(ours, ref.numpy(), atol=1e-12, rtol=1e-10)
    if empty_row:
        assert np.all(dq[..., 5, :] == 0)


def test_attention_reference_gradcheck():
    """Finite differences pin the torch formulation the backward is checked against."""
    eff = torch.from_numpy(so.token_mask(6, 9, 1, 3))
    args = [torch.randn(1, 1, n, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(s),
                        requires_grad=True) for n, s in ((6, 0), (9, 1), (9, 2))]
    assert torch.autograd.gradcheck(lambda a, b, c: _torch_reference(a, b, c, eff, 0.5), args)


def test_attention_bwd_identities():
    B, H, n_q, n_kv, D = 1, 1, 30, 30, 8
    q, k, v = _rand((B, H, n_q, D), 11), _rand((B, H, n_kv, D), 12), _rand((B, H, n_kv, D), 13)
    do = _rand((B, H, n_q, D), 14)
    eff = so.token_mask(n_q, n_kv, 3, 5)
    scale = 0.3
    o, _ = so.attention_fwd(q, k, v, eff, scale)
    dq, dk, dv = so.attention_bwd(q, k, v, do, eff, scale)
    # sum over keys of dS is zero  =>  sum_k dK = scale * dS^T Q summed = 0 along rows of Q
    # equivalently sum of dK over all keys equals scale * sum_q (sum_k dS[q,k]) Q[q] = 0
    np.testing.assert_allclose(dk.sum(axis=-2), 0.0, atol=1e-10)
    # dV sums: sum_k dV[k] = sum_q dO[q] for rows that see at least one key
    np.testing.assert_allclose(dv.sum(axis=-2), do.sum(axis=-2), atol=1e-10)
    # Delta = rowsum(dO * O) equals rowsum(P * dP)
    p, _ = so._probs(q, k, eff, scale)
    dp = do @ np.swapaxes(v, -1, -2)
    np.testing.assert_allclose((do * o).sum(-1), (p * dp).sum(-1), atol=1e-12)


def test_prefix_regressions_of_the_reference():
    # lifted block mask alone is strictly looser than the token mask (H-1)
    m = so.block_mask(32, 32, 4, 8, 8, 8)
    assert (so.lift(m, 8, 8, 32, 32) & ~so.token_mask(32, 32, 4, 8)).any()
    # is_causal=False differs from the fixed path (H-2)
    q, k, v = _rand((1, 1, 32, 8), 0), _rand((1, 1, 32, 8), 1), _rand((1, 1, 32, 8), 2)
    fixed, _ = so.attention_fwd(q, k, v, so.effective_mask(m, 32, 32, 8, 8, True, 4, 8))
    loose, _ = so.attention_fwd(q, k, v, so.effective_mask(m, 32, 32, 8, 8, False, 4, 8))
    assert not np.allclose(fixed, loose, atol=1e-10)


@pytest.mark.parametrize("causal", [True, False])
def test_chunked_reference_matches_dense_oracle(causal):
    B, H, n_q, n_kv, D, bm, bn, S, W = 2, 2, 150, 170, 16, 16, 32, 3, 40
    m = so.block_mask(n_q, n_kv, S, W, bm, bn)
    if not causal:
        m = (np.random.default_rng(3).random(m.shape) < 0.4).astype(np.int32)
        m[1] = 0                                        # empty rows 16..31
    q, k, v = _rand((B, H, n_q, D), 20), _rand((B, H, n_kv, D), 21), _rand((B, H, n_kv, D), 22)
    do = _rand((B, H, n_q, D), 23)
    eff = so.effective_mask(m, n_q, n_kv, bm, bn, causal, S, W)
    o, lse = so.attention_fwd(q, k, v, eff)
    grads = so.attention_bwd(q, k, v, do, eff)
    t = [torch.from_numpy(x) for x in (q, k, v, do)]
    res = cr.chunked_attention(t[0], t[1], t[2], torch.from_numpy(m), bm, bn, causal, S, W,
                               do=t[3], chunk=37)
    np.testing.assert_allclose(res[0].numpy(), o, atol=1e-12)
    np.testing.assert_allclose(res[1].numpy(), lse, atol=1e-12)
    for ours, ref in zip(res[2:], grads):
        np.testing.assert_allclose(ours.numpy(), ref, atol=1e-11)


def test_eager_cpu_baseline_matches_oracle():
    from oracle import eager_cpu

    B, H, n_q, n_kv, D, bm, bn, S, W = 1, 2, 150, 200, 16, 32, 16, 3, 40
    m = so.block_mask(n_q, n_kv, S, W, bm, bn)
    q, k, v = _rand((B, H, n_q, D), 30), _rand((B, H, n_kv, D), 31), _rand((B, H, n_kv, D), 32)
    got = eager_cpu.eager_masked_attention(*(torch.from_numpy(x) for x in (q, k, v)),
                                           torch.from_numpy(m), bm, bn, True, S, W, chunk=64)
    ref, _ = so.attention_fwd(q, k, v, so.effective_mask(m, n_q, n_kv, bm, bn, True, S, W))
    np.testing.assert_allclose(got.numpy(), ref, atol=1e-12)
