"""CPU tests of the product's host side: mask API, validation errors, C ABI.

No kernel is launched here (there is no GPU in this tier): the library is only
loaded, its exported symbols checked against ``include/gki_bsa.h``, and its
host-side argument validation exercised.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import sparse_triton_kernel as stk
from gki import _lib
from oracle import streaming_oracle as so

from test_oracle_pins import BLOCK_SHAPES, TOKEN_SHAPES

HEADER = Path(__file__).resolve().parents[1] / "include" / "gki_bsa.h"


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", BLOCK_SHAPES)
def test_cpu_streaming_mask_matches_oracle(n_q, n_kv, sink, window, bm, bn):
    m = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), bm, bn, device="cpu")
    assert m.dtype == torch.int32 and m.is_contiguous()
    np.testing.assert_array_equal(m.numpy(), so.block_mask(n_q, n_kv, sink, window, bm, bn))


@pytest.mark.parametrize("n_q,n_kv,sink,window", TOKEN_SHAPES)
def test_token_mask_matches_oracle(n_q, n_kv, sink, window):
    np.testing.assert_array_equal(stk.streaming_token_mask(n_q, n_kv, sink, window).numpy(),
                                  so.token_mask(n_q, n_kv, sink, window))


def test_dense_mask_cpu():
    np.testing.assert_array_equal(stk.make_dense_mask(64, 128, 16, 32, causal=True, device="cpu").numpy(),
                                  so.dense_block_mask(64, 128, 16, 32, True))
    assert stk.make_dense_mask(64, 128, 16, 32, device="cpu").all()
    with pytest.raises(ValueError, match="must divide"):
        stk.make_dense_mask(65, 128, 16, 32, device="cpu")


def test_drop_in_module_names():
    """The reference module's public names and its backend flag: True here,
    where the kernel library loads (the op itself needs a GPU)."""
    for name in ("StreamingMaskSpec", "make_streaming_mask", "make_dense_mask", "streaming_token_mask",
                 "block_sparse_attention", "reference_block_sparse_attention",
                 "_BlockSparseFlashAttention"):
        assert hasattr(stk, name), name
    assert stk._TRITON_AVAILABLE is True and stk._TRITON_AVAILABLE == _lib.available()


def test_spec_and_mask_argument_errors():
    with pytest.raises(ValueError, match="non-negative"):
        stk.StreamingMaskSpec(-1, 4)
    with pytest.raises(ValueError, match="non-negative"):
        stk.StreamingMaskSpec(4, -4)
    with pytest.raises(ValueError, match="positive"):
        stk.make_streaming_mask(0, 10, stk.StreamingMaskSpec(1, 1), 4, 4, device="cpu")
    with pytest.raises(ValueError, match="positive"):
        stk.make_streaming_mask(10, 10, stk.StreamingMaskSpec(1, 1), 0, 4, device="cpu")


def test_reference_eager_api_matches_oracle():
    n_q, n_kv, D, S, W, bm, bn = 48, 80, 16, 2, 20, 16, 16
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 2, n, D, generator=g, dtype=torch.float64) for n in (n_q, n_kv, n_kv))
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), bm, bn, device="cpu")
    out = stk.reference_block_sparse_attention(q, k, v, mask, block_m=bm, block_n=bn,
                                               is_causal=True, sink_size=S, window_size=W)
    eff = so.effective_mask(mask.numpy(), n_q, n_kv, bm, bn, True, S, W)
    np.testing.assert_allclose(out.numpy(), so.attention_fwd(q.numpy(), k.numpy(), v.numpy(), eff)[0],
                               atol=1e-12)


def _qkv(device="cpu", dtype=torch.float32, shape=(1, 2, 32, 16)):
    return [torch.zeros(shape, dtype=dtype, device=device) for _ in range(3)]


def test_op_validation_errors_on_cpu():
    q, k, v = _qkv()
    mask = torch.ones(1, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="4-D"):
        stk.block_sparse_attention(q[0], k, v, mask)
    with pytest.raises(ValueError, match="CUDA device"):
        stk.block_sparse_attention(q, k, v, mask, block_m=32, block_n=32)


def _declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(gki_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_symbols()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), f"{name} declared in gki_bsa.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.gki_abi_version() == _lib.ABI_VERSION == 8


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """Without the built gfx950 library the binding raises, naming the build
    command and that there is no CPU fallback; nothing is bound."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_load_error", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libgki_bsa.so")
    with pytest.raises(RuntimeError, match=r"unavailable \(OSError.*no CPU fallback"):
        _lib.load()
    assert not _lib.available()


def test_load_refuses_other_abi_version(monkeypatch):
    """A library whose gki_abi_version differs from the binding's table (a stale
    build exporting the same names with other argument lists) is refused with a
    RuntimeError naming both versions, as the reference raises when its backend
    is unusable (sparse_triton_kernel.py:626-630); nothing is bound from it."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_load_error", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", 7)
    with pytest.raises(RuntimeError, match=r"C ABI version 8, this binding needs version 7"):
        _lib.load()
    assert not _lib.available()
    # the real binding loads again once the expected version matches
    monkeypatch.setattr(_lib, "_load_error", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", 8)
    assert _lib.load().gki_abi_version() == 8


def test_dkdv_work_list_matches_oracle():
    """gki_dkdv_items (host code) equals the oracle's plan bit for bit, including
    empty columns, a single tile and sizes that split many columns."""
    from gki.lists import dkdv_items

    rng = np.random.default_rng(9)
    cases = [(np.array([0, 0]), 1, 1), (np.array([0, 5]), 4, 1)]
    for _ in range(40):
        n_kt = int(rng.integers(1, 300))
        cnt = rng.integers(0, 200, n_kt)
        cnt[rng.random(n_kt) < 0.1] = 0
        cases.append((np.concatenate([[0], np.cumsum(cnt)]), int(rng.choice([1, 2, 4, 8])),
                      int(rng.integers(1, 128))))
    m = so.block_mask(131072, 131072, 4, 4096, 64, 64)
    cases.append((so.kept_lists(m)[2], 1, 16))
    for i, (col_ptr, group, bh_kv) in enumerate(cases):
        col_ptr = col_ptr.astype(np.int32)
        # uncapped (16-bit inputs), the fp32 cap, and caps above the default chunk
        for max_chunk in (0, 4, 1 + i % 50):
            items, split, n_items, n_split, n_pslots = dkdv_items(torch.from_numpy(col_ptr), group,
                                                                  bh_kv, max_chunk)
            want_items, want_split, want_np = so.dkdv_items(col_ptr, group, bh_kv,
                                                            max_chunk=max_chunk)
            np.testing.assert_array_equal(items.numpy(), want_items)
            assert n_items == len(want_items) and n_split == len(want_split) and n_pslots == want_np
            np.testing.assert_array_equal(split.numpy()[:n_split], want_split)
            if max_chunk > 0:
                assert (want_items[:, 2] - want_items[:, 1]).max(initial=0) <= max_chunk


def test_fwd_order_sorts_each_xcd_share_heaviest_first():
    """gki_fwd_order (host code): a permutation of the n_qt * bh work units that
    keeps each XCD's share (the hardware hands workgroup b to XCD b % 8, so XCD
    x runs n // 8 units, one more for x < n % 8, as one contiguous range of
    logical ids in XCD order) and sorts every share by descending kept-tile
    count, ties in unit order -- which fixes the table uniquely."""
    lib = _lib.load()
    rng = np.random.default_rng(5)
    cases = [(np.array([0, 3]), 1), (np.array([0, 0, 0]), 5)]
    # the c2 forward schedule's row lengths (sink + window tiles, light first rows)
    lens = np.minimum(np.arange(128) * 2 + 2, 34)
    cases.append((np.concatenate([[0], np.cumsum(lens)]), 32))
    for _ in range(30):
        n_qt = int(rng.integers(1, 300))
        cnt = rng.integers(0, 6, n_qt) * int(rng.choice([1, 7]))
        cases.append((np.concatenate([[0], np.cumsum(cnt)]), int(rng.choice([1, 3, 8, 13, 64]))))
    for row_ptr, bh in cases:
        row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int32)
        n_qt = len(row_ptr) - 1
        n = n_qt * bh
        order = np.full(n, -1, dtype=np.int32)
        assert lib.gki_fwd_order(row_ptr.ctypes.data, n_qt, bh, order.ctypes.data) == 0
        assert np.array_equal(np.sort(order), np.arange(n))
        length = np.diff(row_ptr)[order % n_qt]
        lo = 0
        for x in range(8):
            hi = lo + n // 8 + (x < n % 8)
            share = order[lo:hi]
            assert np.array_equal(np.sort(share), np.arange(lo, hi)), "a unit left its XCD"
            d_len, d_id = np.diff(length[lo:hi]), np.diff(share)
            assert (d_len <= 0).all() and (d_id[d_len == 0] > 0).all()
            lo = hi
        assert lo == n
    bad = np.array([0, 4, 2], dtype=np.int32)
    out = np.zeros(4, dtype=np.int32)
    assert lib.gki_fwd_order(bad.ctypes.data, 2, 2, out.ctypes.data) == 1
    assert b"non-decreasing" in lib.gki_last_error()
    assert lib.gki_fwd_order(bad.ctypes.data, 0, 2, out.ctypes.data) == 1
    assert lib.gki_fwd_order(None, 2, 2, out.ctypes.data) == 1


def test_decode_routing_rules():
    """The op's decode plan mirrors the library: 2..32 query rows per K / V
    stream of a 16-bit computed-stream step run on the matrix cores with one
    slot per stream; otherwise a group shares a workgroup only within the 4-row
    kernel's limit."""
    from gki import ops

    tile_m = 16
    assert ops._decode_on_mfma(2, 128, 4, 1, tile_m)            # grouped-query, one position
    assert ops._decode_on_mfma(1, 64, 1, 4, tile_m)             # multi-head, 4 positions
    assert ops._decode_on_mfma(2, 128, 32, 1, tile_m)           # 32 rows: two column blocks
    assert not ops._decode_on_mfma(2, 128, 1, 1, tile_m)        # one row: the vector kernel
    assert not ops._decode_on_mfma(2, 128, 64, 1, tile_m)       # 64 rows
    assert not ops._decode_on_mfma(0, 128, 4, 1, tile_m)        # fp32
    assert not ops._decode_on_mfma(2, 32, 4, 1, tile_m)         # head_dim 32
    assert ops._decode_slots(8, 32, 8, 1, 4, mfma=True) == 64
    assert ops._decode_slots(8, 32, 8, 1, 4) == 64              # group 4 fits the 4-row kernel
    assert ops._decode_slots(8, 32, 2, 1, 4) == 256             # group 16: one q head each
    assert ops._decode_slots(8, 32, 32, 2, 4) == 256
    # about one workgroup per CU, at least ~256 tokens each
    assert ops._decode_splits(2052, 64) == 4 and ops._decode_splits(2052, 256) == 1
    assert ops._decode_splits(2052, 8) == 8 and ops._decode_splits(100, 1) == 1


def test_decode_plan_is_memoized_and_matches_the_rules(monkeypatch):
    """The per-call decode plan (matrix cores?, splits, workspace floats) equals
    the rules above plus the library's workspace size, and a second call with
    the same key asks the library nothing."""
    from gki import ops

    lib = _lib.load()
    ops._DECODE_PLANS.clear()
    ts = _lib.tile_sizes()
    for (dt, B, H, H_kv, n_q, D, n_tok, ring) in [(2, 8, 32, 8, 1, 128, 2052, True),
                                                  (2, 8, 32, 32, 1, 128, 2052, True),
                                                  (2, 8, 32, 1, 1, 128, 2052, True),
                                                  (1, 1, 4, 4, 4, 64, 600, False),
                                                  (0, 2, 8, 8, 1, 64, 5000, True)]:
        mfma = ring and ops._decode_on_mfma(dt, D, H // H_kv, n_q, ts["decode_tile_m"])
        splits = ops._decode_splits(n_tok, ops._decode_slots(B, H, H_kv, n_q, ts["decode_max_q"], mfma))
        ws = int(lib.gki_bsa_decode_workspace_floats(B, H, n_q, D, splits)) if splits > 1 else 0
        assert ops._decode_plan(lib, dt, B, H, H_kv, n_q, D, n_tok, ring) == (mfma, splits, ws)

    class _NoLib:
        def __getattr__(self, name):
            raise AssertionError("memoized plan must not call the library")

    assert ops._decode_plan(_NoLib(), 2, 8, 32, 8, 1, 128, 2052, True)[1] == 4


def test_dkdv_work_list_rejects_bad_columns():
    lib = _lib.load()
    out = [ctypes.c_int32() for _ in range(3)]
    refs = [ctypes.addressof(c) for c in out]
    bad = np.array([0, 5, 3], np.int32)                         # decreasing pointer
    assert lib.gki_dkdv_items(bad.ctypes.data, 2, 1, 1, 0, None, refs[0], None, refs[1], refs[2]) == 1
    assert b"column" in lib.gki_last_error()
    ok = np.array([0, 5], np.int32)
    assert lib.gki_dkdv_items(ok.ctypes.data, 1, 0, 1, 0, None, refs[0], None, refs[1], refs[2]) == 1


def test_tile_sizes():
    ts = _lib.tile_sizes()
    assert ts == {"fwd_tile_m_16": 128, "fwd_tile_m_32": 64, "bwd_tile_m": 64, "tile_n": 64,
                  "decode_tile_m": 16, "decode_max_q": 4}


def test_capi_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    # unsupported head_dim: code 2, nothing launched
    rc = lib.gki_bsa_fwd(1, 1, 1, 1, 1, 2, 1, 1, 1, 64, 64, 48, 1, 1, 1, 0, 1, 1, 1, 64, 64, 0.1, 1, 4, 8,
                         null)
    assert rc == 2 and b"head_dim" in lib.gki_last_error()
    # bad dtype code
    rc = lib.gki_bsa_fwd(1, 1, 1, 1, 1, 7, 1, 1, 1, 64, 64, 64, 1, 1, 1, 0, 1, 1, 1, 64, 64, 0.1, 1, 4, 8,
                         null)
    assert rc == 2 and b"dtype" in lib.gki_last_error()
    # mask shape mismatch
    rc = lib.gki_bsa_fwd(1, 1, 1, 1, 1, 0, 1, 1, 1, 64, 64, 64, 1, 1, 1, 0, 1, 2, 1, 64, 64, 0.1, 1, 4, 8,
                         null)
    assert rc == 1 and b"mask shape" in lib.gki_last_error()
    # schedule row count mismatch
    rc = lib.gki_bsa_fwd(16, 16, 16, 16, 16, 0, 1, 1, 1, 200, 64, 64, 16, 16, 2, 0, 1, 4, 1, 64, 64,
                         0.1, 1, 4, 8, null)
    assert rc == 1 and b"schedule" in lib.gki_last_error()
    # decode: too many rows
    rc = lib.gki_bsa_decode(16, 16, 16, 16, 16, 2, 1, 1, 1, 8, 64, 64, 1, 1, 1, 1, 1, 64, 64, 0.1,
                            1, 4, 8, 1, 1, null)
    assert rc == 2 and b"decode" in lib.gki_last_error()
    # masks
    assert lib.gki_streaming_mask(1, 0, 10, 4, 4, 64, 64, null) == 1
    assert lib.gki_dense_mask(1, 60, 64, 16, 16, 0, null) == 1
    assert b"divide" in lib.gki_last_error()
    assert lib.gki_bsa_decode_workspace_floats(2, 3, 1, 128, 5) == 2 * 3 * 5 * 130
    # decode: several splits need a workspace
    rc = lib.gki_bsa_decode(16, 16, 16, 16, 16, 2, 1, 1, 1, 1, 1000, 64, 1, 300, 1, 1, 16, 1, 64,
                            0.1, 1, 4, 8, 0, 2, null)
    assert rc == 1 and b"workspace" in lib.gki_last_error()
    # misaligned tensor pointers are rejected before any launch
    rc = lib.gki_bsa_fwd(16, 18, 16, 16, 16, 2, 1, 1, 1, 64, 64, 64, 16, 16, 1, 0, 16, 1, 1, 64, 64,
                         0.1, 1, 4, 8, null)
    assert rc == 1 and b"aligned" in lib.gki_last_error()
    # grouped-query attention: H_kv must divide H
    rc = lib.gki_bsa_fwd(1, 1, 1, 1, 1, 2, 1, 6, 4, 64, 64, 64, 1, 1, 1, 0, 1, 1, 1, 64, 64, 0.1, 1, 4,
                         8, null)
    assert rc == 1 and b"H_kv" in lib.gki_last_error()
    # a block mask of 2^31 or more entries (kernels index it with 32-bit offsets)
    n = 1 << 20
    rc = lib.gki_bsa_fwd(16, 16, 16, 16, 16, 2, 1, 1, 1, n, n, 64, 16, 16, 1, 0, 16, n // 16, n // 16, 16,
                         16, 0.1, 1, 4, 8, null)
    assert rc == 1 and b"block mask too large" in lib.gki_last_error()


def test_fp32_dkdv_spread_chunk():
    """Short fp32 grids: the dK/dV column walks are cut so that about ``target``
    items result, at least two iterations each; grids with enough columns keep
    the library's own chunk (0)."""
    from gki.lists import spread_chunk

    def ptr(lens):
        return torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)

    assert spread_chunk(ptr([6] * 16), 1, 4, 512) == 2           # c1: 64 columns of ~6
    assert spread_chunk(ptr([18] * 64), 1, 4, 512) == 9          # 256 columns of 18
    assert spread_chunk(ptr([18] * 64), 2, 4, 512) == 18         # q heads per kv head count
    assert spread_chunk(ptr([18] * 128), 1, 4, 512) == 0         # 512 columns fill the grid
    assert spread_chunk(ptr([6] * 16), 1, 4, 0) == 0             # not asked for
