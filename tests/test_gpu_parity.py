"""GPU parity of the gfx950 kernels against the oracle.

* masks and kept-block lists: bit-exact against ``oracle.streaming_oracle``;
* forward / backward / decode: against the fp64 oracle on small shapes and
  against the chunked exact reference (``oracle.chunked_reference``, fp64 on
  the GPU) at the full sizes of the five BASELINE configs.

Tolerances: fp32 atol 1e-5; fp16/bf16 atol 2e-2 and
rtol 1e-2, i.e. |ours - ref| <= atol + rtol * |ref| elementwise.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fx_compiler_pass as fxp
import sparse_triton_kernel as stk
from gki import _lib, build_block_lists
from gki.ops import _FP32_DKDV_TARGET_ITEMS
from gki.lists import bwd_schedule, decode_schedule, fwd_order, fwd_schedule
from oracle import chunked_reference as cr
from oracle import streaming_oracle as so

from test_oracle_pins import BLOCK_SHAPES

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: (1e-5, 0.0), torch.float16: (2e-2, 1e-2), torch.bfloat16: (2e-2, 1e-2)}


def _close(ours: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, what: str) -> None:
    atol, rtol = TOL[dtype]
    o = ours.detach().to(torch.float64).cpu()
    r = ref.detach().to(torch.float64).cpu()
    err = (o - r).abs()
    bound = atol + rtol * r.abs()
    bad = err > bound
    assert torch.isfinite(o).all(), f"{what}: non-finite values"
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements out of tolerance, max|d|="
                           f"{float(err.max()):.3e}, worst excess={float((err - bound).max()):.3e}")


def _inputs(shape_q, shape_kv, dtype, seed, scale=1.0, chunked=False, grad_out=False):
    """q, k, v (and dO) ~ N(0, scale^2) from a CPU generator seeded per case,
    then moved to the GPU: the same bits on every host. ``chunked`` draws
    through ``benchmark.seeded_normal`` (per-chunk CPU generators on a thread
    pool), for the full-size decode and layer configs, as bench.py does."""
    shapes = [shape_q, shape_kv, shape_kv] + ([shape_q] if grad_out else [])
    if chunked:
        from benchmark import seeded_normal

        ts = seeded_normal(shapes, seed, dtype, DEV, scale=scale)
    else:
        g = torch.Generator().manual_seed(seed)
        ts = [(torch.randn(s, generator=g, dtype=torch.float32) * scale).to(dtype).to(DEV) for s in shapes]
    return ts[0], ts[1], ts[2], (ts[3] if grad_out else None)


# ---------------------------------------------------------------------------
# masks and lists: bit-exact
# ---------------------------------------------------------------------------

CONFIG_MASKS = [
    (1024, 1024, 4, 256, 64, 64), (16384, 16384, 4, 2048, 64, 64), (8192, 8192, 4, 1024, 64, 64),
    (1, 100000, 4, 2048, 1, 64), (131072, 131072, 4, 4096, 128, 64),
]


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", BLOCK_SHAPES + CONFIG_MASKS)
def test_device_streaming_mask_bit_exact(n_q, n_kv, sink, window, bm, bn):
    m = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), bm, bn, device=DEV)
    assert m.dtype == torch.int32 and m.is_cuda
    np.testing.assert_array_equal(m.cpu().numpy(), so.block_mask(n_q, n_kv, sink, window, bm, bn))


def test_device_dense_mask_bit_exact():
    for causal in (False, True):
        m = stk.make_dense_mask(256, 512, 32, 64, causal=causal, device=DEV)
        np.testing.assert_array_equal(m.cpu().numpy(), so.dense_block_mask(256, 512, 32, 64, causal))


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", CONFIG_MASKS + [(1000, 1000, 4, 128, 64, 64)])
def test_kept_block_lists_bit_exact(n_q, n_kv, sink, window, bm, bn):
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    lists = build_block_lists(torch.from_numpy(m).to(DEV))
    ref = so.kept_lists(m)
    for got, want in zip((lists.row_ptr, lists.row_idx, lists.col_ptr, lists.col_idx), ref):
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    assert lists.nnz == int(m.sum())


def test_kept_block_lists_random_and_empty():
    rng = np.random.default_rng(5)
    for shape, p in (((37, 1500), 0.2), ((1, 1), 1.0), ((5, 7), 0.0), ((300, 2), 0.5)):
        m = (rng.random(shape) < p).astype(np.int32)
        lists = build_block_lists(torch.from_numpy(m).to(DEV))
        for got, want in zip((lists.row_ptr, lists.row_idx, lists.col_ptr, lists.col_idx),
                             so.kept_lists(m)):
            np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn",
                         [(300, 300, 4, 64, 16, 16), (1000, 1000, 4, 128, 128, 32),
                          (8192, 8192, 4, 1024, 64, 64), (200, 333, 2, 50, 8, 128)])
def test_schedules_match_oracle(n_q, n_kv, sink, window, bm, bn, causal):
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    dm = torch.from_numpy(m).to(DEV)
    ts = _lib.tile_sizes()
    # backward: CSR + CSC over 64x64 tiles and the dK/dV work list
    sched = bwd_schedule(dm, n_q, n_kv, bm, bn, causal, sink, window, group=2, bh_kv=3)
    tiles = so.tile_classes(m, n_q, n_kv, bm, bn, ts["bwd_tile_m"], ts["tile_n"], causal, sink,
                            window)
    ref = so.kept_lists(tiles)
    L = sched.lists
    for got, want in zip((L.row_ptr, L.row_idx, L.col_ptr, L.col_idx), ref):
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    items, split, n_pslots = so.dkdv_items(ref[2], 2, 3)
    np.testing.assert_array_equal(sched.items.cpu().numpy(), items)
    np.testing.assert_array_equal(sched.split.cpu().numpy()[:sched.n_split], split)
    assert (sched.n_items, sched.n_split, sched.n_pslots) == (len(items), len(split), n_pslots)
    # forward: CSR over the per-dtype q tiles
    for fp32, key in ((False, "fwd_tile_m_16"), (True, "fwd_tile_m_32")):
        fs = fwd_schedule(dm, n_q, n_kv, bm, bn, causal, sink, window, fp32)
        tiles = so.tile_classes(m, n_q, n_kv, bm, bn, ts[key], ts["tile_n"], causal, sink, window)
        ref = so.kept_lists(tiles)
        assert fs.n_qt == tiles.shape[0]
        np.testing.assert_array_equal(fs.lists.row_ptr.cpu().numpy(), ref[0])
        np.testing.assert_array_equal(fs.lists.row_idx.cpu().numpy(), ref[1])


def test_decode_schedule_matches_oracle():
    m = so.block_mask(1, 100000, 4, 2048, 1, 64)
    sched = decode_schedule(torch.from_numpy(m).to(DEV), 1, 100000, 1, 64, True, 4, 2048)
    assert sched.n_tiles == 34
    np.testing.assert_array_equal(sched.tiles.cpu().numpy(), [0] + list(range(1530, 1563)))
    # token-exact stream: the 4 sink tokens and the 2048-token window
    assert sched.n_tokens == 4 + 2048
    np.testing.assert_array_equal(sched.tokens.cpu().numpy(),
                                  list(range(4)) + list(range(100000 - 2048, 100000)))


@pytest.mark.parametrize("n_q,n_kv,sink,window,bm,bn", [
    (1, 100, 4, 64, 1, 64),      # window starts inside tile 0, past the sinks
    (1, 90, 4, 50, 1, 64),
    (3, 500, 4, 100, 1, 64),
    (4, 129, 2, 32, 2, 32),
    (1, 1000, 0, 64, 1, 64),
    (2, 300, 4, 0, 1, 64),       # W = 0: sinks only
    (1, 3000, 4, 256, 1, 16),
])
def test_decode_stream_is_the_visible_union(n_q, n_kv, sink, window, bm, bn):
    """The decode token stream is exactly the positions some query row can see
    (ascending), except that for W = 0 and several rows it may keep the rows'
    own positions, which the per-row token rule then drops."""
    m = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    sched = decode_schedule(torch.from_numpy(m).to(DEV), n_q, n_kv, bm, bn, True, sink, window)
    got = (sched.tokens.cpu().numpy() & ((1 << 30) - 1)).tolist()
    assert got == sorted(got) and len(set(got)) == len(got)
    vis = np.nonzero(so.token_mask(n_q, n_kv, sink, window).any(axis=0))[0].tolist()
    if window >= 1 or n_q == 1:
        assert got == vis
    else:
        assert set(vis) <= set(got) and set(got) - set(vis) <= set(range(n_kv - n_q + 1, n_kv))


# ---------------------------------------------------------------------------
# small shapes vs the fp64 oracle
# ---------------------------------------------------------------------------


def _oracle(q, k, v, mask, bm, bn, causal, sink, window, scale, do=None):
    n_q, n_kv = q.shape[-2], k.shape[-2]
    eff = so.effective_mask(mask.cpu().numpy(), n_q, n_kv, bm, bn, causal, sink, window)
    qn, kn, vn = (t.detach().to(torch.float64).cpu().numpy() for t in (q, k, v))
    o, lse = so.attention_fwd(qn, kn, vn, eff, scale)
    grads = None
    if do is not None:
        grads = so.attention_bwd(qn, kn, vn, do.detach().to(torch.float64).cpu().numpy(), eff, scale)
    return torch.from_numpy(o), torch.from_numpy(lse), grads


def _run_case(B, H, n_q, n_kv, D, dtype, bm, bn, causal, sink, window, seed, mask=None,
              backward=True, softmax_scale=None, H_kv=None):
    H_kv = H if H_kv is None else H_kv
    group = H // H_kv
    q, k, v, do = _inputs((B, H, n_q, D), (B, H_kv, n_kv, D), dtype, seed, grad_out=True)
    if mask is None:
        mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), bm, bn, device=DEV)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    leaves = [t.clone().requires_grad_(backward) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, softmax_scale=softmax_scale, block_m=bm,
                                     block_n=bn, is_causal=causal, sink_size=sink,
                                     window_size=window, enable_gqa=group > 1)
    kx = torch.from_numpy(so.expand_kv_heads(k.double().cpu().numpy(), group))
    vx = torch.from_numpy(so.expand_kv_heads(v.double().cpu().numpy(), group))
    o_ref, lse_ref, grads = _oracle(q, kx, vx, mask, bm, bn, causal, sink, window, scale,
                                    do if backward else None)
    tag = (f"B{B} H{H}/{H_kv} nq{n_q} nkv{n_kv} D{D} {dtype} bm{bm} bn{bn} causal{causal} S{sink} "
           f"W{window} scale {scale:.4g}")
    _close(out, o_ref, dtype, "O " + tag)
    if backward:
        out.backward(do)
        grads = (grads[0], so.reduce_kv_grad(grads[1], group), so.reduce_kv_grad(grads[2], group))
        for name, t, ref in zip(("dQ", "dK", "dV"), leaves, grads):
            _close(t.grad, torch.from_numpy(ref), dtype, f"{name} {tag}")
    return out


SMALL = [
    # (B, H, n_q, n_kv, D, bm, bn, S, W)
    (1, 2, 64, 64, 64, 64, 64, 4, 16),
    (1, 2, 200, 200, 64, 64, 64, 4, 50),
    (2, 1, 130, 333, 32, 64, 64, 3, 90),
    (1, 2, 1000, 1000, 128, 64, 64, 4, 128),
    (1, 1, 1025, 1025, 64, 64, 64, 4, 128),
    (1, 2, 1023, 1023, 16, 64, 64, 4, 128),
    (1, 2, 256, 256, 64, 128, 64, 4, 64),
    (1, 2, 300, 300, 64, 16, 16, 4, 64),
    (1, 1, 257, 700, 128, 32, 128, 2, 100),
    (1, 2, 48, 1000, 64, 16, 64, 4, 128),
    (1, 2, 128, 128, 64, 64, 64, 0, 64),
    (1, 2, 128, 128, 64, 64, 64, 4, 0),
    (1, 2, 64, 64, 64, 16, 16, 64, 0),
    # more queries than keys: q_offset = n_kv - n_q < 0, the first rows see nothing
    (1, 2, 300, 200, 64, 64, 64, 4, 64),
    (2, 1, 200, 64, 128, 32, 64, 2, 16),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n_kv", [64, 100, 128, 192, 256, 300, 320, 384])
def test_fwd_d128_kept_tile_counts(n_kv, dtype):
    """head_dim 128 runs the 16-bit forward skewed by one kv tile and unrolled
    by two (the next tile's S while the current one's softmax runs, a peeled
    last step for odd counts). One 128-row q tile that sees every key (a
    window past n_kv) keeps ceil(n_kv / 64) kv tiles: 1 .. 6 here, even and
    odd, with a ragged last tile at 100 and 300 keys."""
    _run_case(1, 2, 128, n_kv, 128, dtype, 64, 64, True, 4, 4096, seed=n_kv, backward=False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", SMALL, ids=lambda c: "x".join(map(str, c)))
def test_small_causal_vs_oracle(case, dtype):
    B, H, n_q, n_kv, D, bm, bn, S, W = case
    _run_case(B, H, n_q, n_kv, D, dtype, bm, bn, True, S, W, seed=hash(case) % 1000)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_q,n_kv,D,bm,bn", [(1, 700, 64, 1, 64), (1, 1000, 128, 1, 64),
                                               (3, 500, 128, 1, 64), (4, 129, 64, 2, 32),
                                               (1, 64, 128, 1, 64), (2, 2000, 64, 1, 16),
                                               (4, 3, 64, 1, 64)])
def test_decode_vs_oracle(n_q, n_kv, D, bm, bn, dtype):
    _run_case(2, 3, n_q, n_kv, D, dtype, bm, bn, True, 4, 256, seed=n_kv + D, backward=dtype == torch.float32)


@pytest.mark.parametrize("softmax_scale", [0.0, -0.3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("path", ["prefill", "decode", "decode_gqa"])
def test_zero_and_negative_softmax_scale_vs_oracle(path, dtype, softmax_scale):
    """The reference takes any float softmax_scale (sparse_triton_kernel.py:831-837):
    scale 0 (uniform weights over the visible keys) and a negative scale,
    forward and backward, through the prefill kernels, the vector decode and
    (16-bit, grouped-query) the matrix-core decode."""
    print(f"[case] scale {softmax_scale} {dtype} {path}", flush=True)
    if path == "prefill":
        _run_case(1, 2, 300, 300, 64, dtype, 64, 64, True, 4, 64, seed=51, softmax_scale=softmax_scale)
    elif path == "decode":
        _run_case(2, 3, 1, 700, 128, dtype, 1, 64, True, 4, 256, seed=52, softmax_scale=softmax_scale)
    else:
        _run_case(1, 8, 1, 900, 64, dtype, 1, 64, True, 4, 256, seed=53, softmax_scale=softmax_scale,
                  H_kv=2)


def test_decode_more_queries_than_keys_without_window():
    """n_q > n_kv with S = W = 0 on the decode path: no query sees a key, so the
    output is zero (the reference's nan_to_num), through the list path; the
    backward then walks empty lists and gives zero gradients."""
    _run_case(1, 2, 3, 2, 64, torch.bfloat16, 1, 64, True, 0, 0, seed=54, backward=False)
    _run_case(1, 2, 4, 3, 128, torch.float32, 1, 64, True, 0, 0, seed=55)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_all_zero_mask_gives_zeros(dtype):
    """A block mask that keeps nothing: empty kept-block lists, zero output and
    zero gradients (prefill and decode), as the reference's eager path gives."""
    for n_q, n_kv in ((200, 300), (2, 300)):
        mask = torch.zeros((-(-n_q // 64), -(-n_kv // 64)), dtype=torch.int32, device=DEV)
        out = _run_case(1, 2, n_q, n_kv, 64, dtype, 64, 64, False, 0, 0, seed=56, mask=mask)
        assert torch.equal(out, torch.zeros_like(out))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_custom_noncausal_mask_vs_oracle(dtype):
    rng = np.random.default_rng(11)
    n_q, n_kv, bm, bn = 200, 260, 32, 16
    m = (rng.random((-(-n_q // bm), -(-n_kv // bn))) < 0.35).astype(np.int32)
    m[2] = 0                                            # rows 64..95 see nothing
    _run_case(1, 2, n_q, n_kv, 64, dtype, bm, bn, False, 0, 0, seed=3,
              mask=torch.from_numpy(m).to(DEV))


def test_fully_masked_row_outputs_zero_and_no_nan():
    """The reference's GPU test (tests/test_fully_masked_row.py:28-69)."""
    B, H, N_Q, N_KV, D, bm = 1, 2, 32, 32, 16, 16
    q, k, v = (torch.randn(B, H, n, D, device=DEV, requires_grad=True) for n in (N_Q, N_KV, N_KV))
    mask = torch.zeros((2, 2), dtype=torch.int32, device=DEV)
    mask[1, 1] = 1
    out = stk.block_sparse_attention(q, k, v, mask, block_m=bm, block_n=bm, is_causal=False)
    assert torch.isfinite(out).all()
    assert torch.equal(out[:, :, :bm], torch.zeros_like(out[:, :, :bm]))
    out.backward(torch.randn_like(out))
    for g in (q.grad, k.grad, v.grad):
        assert g is not None and torch.isfinite(g).all()
    assert torch.equal(q.grad[:, :, :bm], torch.zeros_like(q.grad[:, :, :bm]))
    assert torch.equal(k.grad[:, :, :bm], torch.zeros_like(k.grad[:, :, :bm]))


def test_decode_and_prefill_paths_agree():
    """n_q <= 4 goes through the split-KV decode kernel; n_q = 5 through prefill."""
    B, H, n_kv, D = 2, 4, 3000, 128
    k = torch.randn(B, H, n_kv, D, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, H, n_kv, D, device=DEV, dtype=torch.bfloat16)
    q5 = torch.randn(B, H, 5, D, device=DEV, dtype=torch.bfloat16)
    spec = stk.StreamingMaskSpec(4, 512)
    o5 = stk.block_sparse_attention(q5, k, v, stk.make_streaming_mask(5, n_kv, spec, 1, 64, DEV),
                                    block_m=1, block_n=64, is_causal=True, sink_size=4, window_size=512)
    o4 = stk.block_sparse_attention(q5[:, :, 1:].contiguous(), k, v,
                                    stk.make_streaming_mask(4, n_kv, spec, 1, 64, DEV),
                                    block_m=1, block_n=64, is_causal=True, sink_size=4, window_size=512)
    _close(o4, o5[:, :, 1:].float(), torch.bfloat16, "decode vs prefill")


# ---------------------------------------------------------------------------
# config 1: FX-rewritten StandardAttention, fp32 fwd + bwd
# ---------------------------------------------------------------------------


def test_config1_fx_rewrite_fp32_fwd_bwd():
    B, H, N, D, S, W = 1, 4, 1024, 64, 4, 256
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, generator=g) for _ in range(3))
    cfg = fxp.InjectionConfig(seq_len_q=N, seq_len_kv=N, head_dim=D,
                              streaming=stk.StreamingMaskSpec(S, W), block_m=64, block_n=64)
    fused = fxp.BlockSparseAttentionInjector(cfg).transform(fxp.StandardAttention(D)).to(DEV)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = fused(*leaves)
    do = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)).to(DEV)
    out.backward(do)
    mask = so.block_mask(N, N, S, W, 64, 64)
    eff = so.effective_mask(mask, N, N, 64, 64, True, S, W)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do.cpu()))
    o_ref, _ = so.attention_fwd(qn, kn, vn, eff, 1 / 8)
    grads = so.attention_bwd(qn, kn, vn, dn, eff, 1 / 8)
    _close(out, torch.from_numpy(o_ref), torch.float32, "c1 O")
    for name, t, ref in zip(("dQ", "dK", "dV"), leaves, grads):
        _close(t.grad, torch.from_numpy(ref), torch.float32, f"c1 {name}")


# ---------------------------------------------------------------------------
# full-size configs vs the chunked exact reference (fp64 on the GPU)
# ---------------------------------------------------------------------------


def test_config2_prefill_bf16_full():
    B, H, N, D, S, W, bm = 1, 32, 16384, 128, 4, 2048, 64
    q, k, v, _ = _inputs((B, H, N, D), (B, H, N, D), torch.bfloat16, seed=1, scale=0.5)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    out = stk.block_sparse_attention(q, k, v, mask, block_m=bm, block_n=bm, is_causal=True,
                                     sink_size=S, window_size=W)
    lse = _forward_lse(q, k, v, mask, bm, bm, S, W)
    o_ref, lse_ref = cr.chunked_attention(q, k, v, mask, bm, bm, True, S, W)
    _close(out, o_ref, torch.bfloat16, "c2 O")
    # LSE is an fp32 result the backward consumes, held to an absolute bar set
    # by the kernel's one rounding step instead of the bf16 output bar: the
    # 16-bit forward's row sum l adds the same bf16-rounded P that multiplies V
    # (the reference sums the fp32 P), each term within 2^-8 of its fp32 value,
    # so |LSE - ref| <= ln(1 + 2^-8 p_max / l) < 2e-3 (largest in the first
    # rows, which see two or three keys). fp16 and fp32 LSE are pinned tighter
    # in test_lse_vs_oracle.
    err = (lse.double().cpu() - lse_ref.double().cpu()).abs()
    assert torch.isfinite(lse).all() and float(err.max()) <= 2.5e-3, f"c2 LSE max err {float(err.max()):.3e}"
    print(f"[c2] LSE max abs error {float(err.max()):.3e}", flush=True)


@pytest.mark.parametrize("dtype,bar", [(torch.float32, 1e-5), (torch.float16, 5e-4),
                                       (torch.bfloat16, 2.5e-3)])
@pytest.mark.parametrize("case", [(1, 2, 1000, 1000, 128, 64, 64, 4, 128),
                                  (2, 1, 130, 333, 32, 64, 64, 3, 90),
                                  (1, 2, 300, 300, 64, 16, 16, 4, 64),
                                  (1, 2, 128, 128, 64, 64, 64, 0, 64)],
                         ids=lambda c: "x".join(map(str, c)))
def test_lse_vs_oracle(case, dtype, bar):
    """The saved log-sum-exp against the fp64 oracle's, absolute: fp32 sums fp32
    P (1e-5); the 16-bit kernels sum the 16-bit-rounded P that multiplies V,
    within 2^-11 (fp16) / 2^-8 (bf16) of each fp32 term, bounding the LSE error
    by ln(1 + 2^-11) < 5e-4 and ln(1 + 2^-8) < 2.5e-3. Rows that see no key
    keep the sentinel 0."""
    B, H, n_q, n_kv, D, bm, bn, S, W = case
    q, k, v, _ = _inputs((B, H, n_q, D), (B, H, n_kv, D), dtype, seed=57)
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), bm, bn, device=DEV)
    lse = _forward_lse(q, k, v, mask, bm, bn, S, W).cpu()
    _, lse_ref, _ = _oracle(q, k, v, mask, bm, bn, True, S, W, 1.0 / math.sqrt(D))
    err = (lse - lse_ref).abs()
    assert torch.isfinite(lse).all() and float(err.max()) <= bar, f"LSE max err {float(err.max()):.3e}"


def _forward_lse(q, k, v, mask, bm, bn, S, W):
    """LSE saved for backward by the autograd Function: the reference's natural
    m + ln(l) (sparse_triton_kernel.py:351, saved at :684), as the kernels
    store it."""
    leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=bm, block_n=bn, is_causal=True,
                                     sink_size=S, window_size=W)
    return out.grad_fn.saved_tensors[4].double()


@pytest.mark.parametrize("dtype,chunk", [(torch.float32, 1), (torch.float32, 5),
                                         (torch.float32, None), (torch.float32, 1 << 20),
                                         (torch.bfloat16, 1), (torch.bfloat16, 5),
                                         (torch.bfloat16, None), (torch.bfloat16, 1 << 20)])
def test_dkdv_any_cut_of_the_work_list_matches_oracle(chunk, dtype):
    """gki_bsa_bwd through the C ABI with the dK/dV work list cut at any chunk
    (1 iteration per item, 5, the library's default list -- the op's own for
    16-bit inputs; fp32 ones spread short grids into 2+ iteration items --,
    never): every cut gives the
    oracle's gradients, grouped-query (4 q heads per kv head) so items also
    split inside a group. Inputs N(0, 1): the sink keys' walk covers 44
    iterations (2816 q rows, |dV| up to ~9). The fp32 kernels add each
    iteration's 64 rows into the running sums with a compensated (TwoSum)
    addition and the reduce sums fp32 partials with Kahan summation: one fp32
    accumulator over the whole walk reached 1.08e-5 of dV against the 1e-5 bar."""
    B, H_kv, group, N, D, S, W, bm = 1, 2, 4, 700, 64, 4, 128, 64
    H = H_kv * group
    print(f"[case] work list chunk {chunk} {dtype}", flush=True)
    q, k, v, do = _inputs((B, H, N, D), (B, H_kv, N, D), dtype, seed=31, scale=1.0, grad_out=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=bm, block_n=bm, is_causal=True,
                                     sink_size=S, window_size=W, enable_gqa=True)
    lse = out.grad_fn.saved_tensors[4]
    sched = bwd_schedule(mask, N, N, bm, bm, True, S, W, group=group, bh_kv=B * H_kv)
    L = sched.lists
    items, split, n_pslots = so.dkdv_items(L.col_ptr.cpu().numpy(), group, B * H_kv, chunk=chunk)
    if chunk is None:        # the op's own work list
        np.testing.assert_array_equal(sched.items.cpu().numpy(), items)
    assert (len(split) > 0) == (chunk is None or chunk < 1 << 20)
    items_d = torch.from_numpy(items).to(DEV)
    split_d = torch.from_numpy(split if len(split) else np.zeros((1, 3), np.int32)).to(DEV)
    partials = torch.empty(max(B * H_kv * n_pslots * 2 * 64 * D, 1), dtype=torch.float32, device=DEV)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((2, B, H, N), dtype=torch.float32, device=DEV)   # row-term workspace
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    n_b = (N + bm - 1) // bm
    lib = _lib.load()
    rc = lib.gki_bsa_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(), lse.data_ptr(),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), code, B, H, H_kv, N, N, D,
        L.row_ptr.data_ptr(), L.row_idx.data_ptr(), sched.n_qt, L.col_ptr.data_ptr(),
        L.col_idx.data_ptr(), sched.n_kt, items_d.data_ptr(), len(items), split_d.data_ptr(),
        len(split), n_pslots, partials.data_ptr(), None, mask.data_ptr(), n_b, n_b, bm, bm,
        1.0 / math.sqrt(D), 1, S, W, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gki_last_error()
    torch.cuda.synchronize()
    eff = so.effective_mask(mask.cpu().numpy(), N, N, bm, bm, True, S, W)
    qn, kn, vn, don = (t.to(torch.float64).cpu().numpy() for t in (q, k, v, do))
    grads = so.attention_bwd(qn, so.expand_kv_heads(kn, group), so.expand_kv_heads(vn, group), don,
                             eff, 1.0 / math.sqrt(D))
    _close(dq, torch.from_numpy(grads[0]), dtype, f"dQ chunk {chunk}")
    _close(dk, torch.from_numpy(so.reduce_kv_grad(grads[1], group)), dtype, f"dK chunk {chunk}")
    _close(dv, torch.from_numpy(so.reduce_kv_grad(grads[2], group)), dtype, f"dV chunk {chunk}")


def test_config3_train_fp16_full():
    B, H, N, D, S, W, bm = 4, 16, 8192, 64, 4, 1024, 64
    q, k, v, do = _inputs((B, H, N, D), (B, H, N, D), torch.float16, seed=2, grad_out=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=bm, block_n=bm, is_causal=True,
                                     sink_size=S, window_size=W)
    out.backward(do)
    ref = cr.chunked_attention(q, k, v, mask, bm, bm, True, S, W, do=do)
    _close(out, ref[0], torch.float16, "c3 O")
    for name, t, r in zip(("dQ", "dK", "dV"), leaves, ref[2:]):
        _close(t.grad, r, torch.float16, f"c3 {name}")


def test_config4_decode_bf16_full():
    B, H, NKV, D, S, W = 8, 32, 100000, 128, 4, 2048
    q, k, v, _ = _inputs((B, H, 1, D), (B, H, NKV, D), torch.bfloat16, seed=3, chunked=True)
    mask = stk.make_streaming_mask(1, NKV, stk.StreamingMaskSpec(S, W), 1, 64, device=DEV)
    out = stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                     sink_size=S, window_size=W)
    o_ref, _ = cr.chunked_attention(q, k, v, mask, 1, 64, True, S, W)
    _close(out, o_ref, torch.bfloat16, "c4 O")


def test_config5_layer_bf16_full():
    """One c5 attention layer (1x16x131072x64, S4 W4096, 128x64 blocks), fwd+bwd."""
    B, H, N, D, S, W, bm, bn = 1, 16, 131072, 64, 4, 4096, 128, 64
    q, k, v, do = _inputs((B, H, N, D), (B, H, N, D), torch.bfloat16, seed=4, chunked=True,
                          grad_out=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bn, device=DEV)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=bm, block_n=bn, is_causal=True,
                                     sink_size=S, window_size=W)
    out.backward(do)
    ref = cr.chunked_attention(q, k, v, mask, bm, bn, True, S, W, do=do, chunk=2048)
    _close(out, ref[0], torch.bfloat16, "c5 O")
    for name, t, r in zip(("dQ", "dK", "dV"), leaves, ref[2:]):
        _close(t.grad, r, torch.bfloat16, f"c5 {name}")


@pytest.mark.parametrize("B,H,H_kv,N,D,dtype", [
    (1, 3, 3, 300, 64, torch.bfloat16),       # 9 units: XCD shares of 2 and 1
    (2, 8, 2, 1000, 128, torch.float16),      # grouped-query, ragged last tile
    (1, 4, 4, 700, 32, torch.float32),        # the fp32 kernel's 64-row tiles
    (4, 16, 16, 2048, 64, torch.bfloat16)])
def test_fwd_order_gives_the_index_order_bits(B, H, H_kv, N, D, dtype):
    """gki_bsa_fwd with the gki_fwd_order table (what the op passes) and with
    no table (index order) write the same O and LSE bits: each workgroup's
    q tile is computed independently of when it runs."""
    print(f"[case] fwd order {B}x{H}/{H_kv}x{N}x{D} {dtype}", flush=True)
    S, W, bm = 4, 256, 64
    q, k, v, _ = _inputs((B, H, N, D), (B, H_kv, N, D), dtype, seed=17)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    fp32 = dtype == torch.float32
    sched = fwd_schedule(mask, N, N, bm, bm, True, S, W, fp32)
    order = fwd_order(mask, sched, B * H)
    assert sorted(order.cpu().tolist()) == list(range(sched.n_qt * B * H))
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    n_b = (N + bm - 1) // bm
    lib = _lib.load()
    outs = []
    for table in (order.data_ptr(), None):
        o, lse = torch.empty_like(q), torch.empty((B, H, N), dtype=torch.float32, device=DEV)
        rc = lib.gki_bsa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                             code, B, H, H_kv, N, N, D, sched.lists.row_ptr.data_ptr(),
                             sched.lists.row_buf.data_ptr(), sched.n_qt, table, mask.data_ptr(),
                             n_b, n_b, bm, bm, 1.0 / math.sqrt(D), 1, S, W,
                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.gki_last_error()
        outs.append((o, lse))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    if B * H * N * N > 2e7:          # bits only: the dense fp64 oracle would hold GBs of scores
        return
    eff = so.effective_mask(mask.cpu().numpy(), N, N, bm, bm, True, S, W)
    group = H // H_kv
    qn, kn, vn = (t.to(torch.float64).cpu().numpy() for t in (q, k, v))
    o_ref, _ = so.attention_fwd(qn, so.expand_kv_heads(kn, group), so.expand_kv_heads(vn, group), eff,
                                1.0 / math.sqrt(D))
    _close(outs[0][0], torch.from_numpy(o_ref), dtype, "O with the order table")


def test_fwd_order_entries_out_of_range_do_nothing():
    """A workgroup whose order-table entry is outside 0 .. n-1 exits without
    touching memory (the table is caller data): with every other entry
    replaced by -5 or n, the units still listed get the bits of a full launch
    and the rest of O / LSE keeps its sentinel."""
    print("[case] fwd order with out-of-range entries", flush=True)
    B, H, N, D, S, W, bm = 2, 4, 1000, 64, 4, 256, 64
    q, k, v, _ = _inputs((B, H, N, D), (B, H, N, D), torch.bfloat16, seed=23)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    sched = fwd_schedule(mask, N, N, bm, bm, True, S, W, False)
    n = sched.n_qt * B * H
    full = fwd_order(mask, sched, B * H)
    holed = full.clone()
    holed[0::2] = torch.tensor([-5, n], dtype=torch.int32, device=DEV).repeat(n)[: holed[0::2].numel()]
    lib = _lib.load()
    n_b = (N + bm - 1) // bm

    def run(table):
        o = torch.full_like(q, 0).view(torch.int16).fill_(0x7E7E).view(torch.bfloat16)
        lse = torch.full((B, H, N), -7.0, dtype=torch.float32, device=DEV)
        rc = lib.gki_bsa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                             2, B, H, H, N, N, D, sched.lists.row_ptr.data_ptr(),
                             sched.lists.row_buf.data_ptr(), sched.n_qt, table.data_ptr(),
                             mask.data_ptr(), n_b, n_b, bm, bm, 1.0 / math.sqrt(D), 1, S, W,
                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.gki_last_error()
        return o, lse

    o_full, l_full = run(full)
    o_hole, l_hole = run(holed)
    torch.cuda.synchronize()
    kept = set(full[1::2].tolist())
    tm = _lib.tile_sizes()["fwd_tile_m_16"]
    for unit in range(n):
        bh, qt = divmod(unit, sched.n_qt)
        b, h = divmod(bh, H)
        rows = slice(qt * tm, min(N, (qt + 1) * tm))
        if unit in kept:
            assert torch.equal(o_hole[b, h, rows], o_full[b, h, rows]), unit
            assert torch.equal(l_hole[b, h, rows], l_full[b, h, rows]), unit
        else:
            assert (o_hole[b, h, rows].view(torch.int16) == 0x7E7E).all(), unit
            assert (l_hole[b, h, rows] == -7.0).all(), unit


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dq_order_gives_the_index_order_bits(dtype):
    """gki_bsa_bwd with the schedule's dQ order table (what the op passes) and
    with none (index order) writes the same dQ, dK, dV bits."""
    print(f"[case] dQ order {dtype}", flush=True)
    B, H, N, D, S, W, bm = 2, 4, 1000, 64, 4, 256, 64
    q, k, v, do = _inputs((B, H, N, D), (B, H, N, D), dtype, seed=29, grad_out=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=DEV)
    leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, block_m=bm, block_n=bm, is_causal=True,
                                     sink_size=S, window_size=W)
    lse = out.grad_fn.saved_tensors[4]
    out.backward(do)
    spread = _FP32_DKDV_TARGET_ITEMS if dtype == torch.float32 else 0
    sched = bwd_schedule(mask, N, N, bm, bm, True, S, W, group=1, bh_kv=B * H,
                         spread_to=spread)   # the op's own
    assert sorted(sched.dq_order.cpu().tolist()) == list(range(sched.n_qt * B * H))
    L = sched.lists
    partials = torch.empty(max(B * H * sched.n_pslots * 2 * 64 * D, 1), dtype=torch.float32, device=DEV)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((2, B, H, N), dtype=torch.float32, device=DEV)   # row-term workspace
    n_b = (N + bm - 1) // bm
    lib = _lib.load()
    rc = lib.gki_bsa_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(), lse.data_ptr(),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(),
        {torch.float32: 0, torch.bfloat16: 2}[dtype], B, H, H, N, N, D,
        L.row_ptr.data_ptr(), L.row_buf.data_ptr(), sched.n_qt, L.col_ptr.data_ptr(),
        L.col_buf.data_ptr(), sched.n_kt, sched.items.data_ptr(), sched.n_items,
        sched.split.data_ptr(), sched.n_split, sched.n_pslots, partials.data_ptr(), None,
        mask.data_ptr(), n_b, n_b, bm, bm, 1.0 / math.sqrt(D), 1, S, W,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gki_last_error()
    torch.cuda.synchronize()
    for name, got, ref in zip(("dQ", "dK", "dV"), (dq, dk, dv), [t.grad for t in leaves]):
        assert torch.equal(got, ref), name


def test_fwd_bwd_deterministic():
    B, H, N, D, S, W = 2, 4, 2048, 64, 4, 256
    q, k, v, do = _inputs((B, H, N, D), (B, H, N, D), torch.bfloat16, seed=9, grad_out=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), 64, 64, device=DEV)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
        out = stk.block_sparse_attention(*leaves, mask, is_causal=True, sink_size=S, window_size=W)
        out.backward(do)
        runs.append([out.detach()] + [t.grad for t in leaves])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("n_q", [1, 300])
def test_inference_path_equals_the_autograd_forward(n_q):
    """Without any input requiring a gradient (or under no_grad) the op runs the
    forward without an autograd node: the same bits as the differentiable call,
    and an output that does not require grad. Decode (n_q 1, grouped-query) and
    prefill."""
    B, H, H_kv, N, D = 1, 8, 2, 2000, 128
    q, k, v, _ = _inputs((B, H, n_q, D), (B, H_kv, N, D), torch.bfloat16, seed=41)
    mask = stk.make_streaming_mask(n_q, N, stk.StreamingMaskSpec(4, 256), 64, 64, device=DEV)
    kw = dict(block_m=64, block_n=64, is_causal=True, sink_size=4, window_size=256, enable_gqa=True)
    o_fast = stk.block_sparse_attention(q, k, v, mask, **kw)
    with torch.no_grad():
        o_nograd = stk.block_sparse_attention(q, k, v, mask, **kw)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o_grad = stk.block_sparse_attention(*leaves, mask, **kw)
    assert o_grad.requires_grad and o_grad.grad_fn is not None
    assert not o_fast.requires_grad and o_fast.grad_fn is None
    assert torch.equal(o_fast, o_grad.detach()) and torch.equal(o_nograd, o_fast)


def test_misaligned_views_are_copied_not_faulted():
    """Contiguous views at an odd storage offset (2 bytes off a 16-byte
    boundary) give exactly the aligned result, forward and backward."""
    B, H, N, D = 1, 2, 300, 64
    n = B * H * N * D
    g = torch.Generator().manual_seed(21)
    base = [torch.randn(n + 8, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]
    q, k, v, do = (b[1:1 + n].view(B, H, N, D) for b in base)
    assert q.is_contiguous() and q.data_ptr() % 16 != 0
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(4, 64), 64, 64, device=DEV)
    outs = []
    for qq, kk, vv in ((q, k, v), (q.clone(), k.clone(), v.clone())):
        leaves = [t.detach().requires_grad_(True) for t in (qq, kk, vv)]
        o = stk.block_sparse_attention(*leaves, mask, is_causal=True, sink_size=4, window_size=64)
        o.backward(do)
        outs.append([o] + [t.grad for t in leaves])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
