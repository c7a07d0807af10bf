"""Rolling StreamingLLM KV cache (sink slots + ring) feeding the decode kernel.

CPU (no marker): the slot layout against a brute-force simulation of the ring,
the library's visible-token stream against the oracle's token rule, and the
C-ABI argument checks.
GPU (``gpu``): the cache contents after appends (bit-exact), and decode over the
rolling cache against (a) the full-cache decode of ``block_sparse_attention`` --
bit-identical whenever both walk the same token stream -- and (b) the fp64
oracle over the full K/V with the token rule (BASELINE tolerances).
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

import sparse_triton_kernel as stk
from gki import _lib
from gki.kv_cache import StreamingKVCache, ring_slot, rolling_stream
from gki.lists import decode_schedule
from oracle import streaming_oracle as so

DEV = "cuda"
TOL = {torch.float32: (1e-5, 0.0), torch.float16: (2e-2, 1e-2), torch.bfloat16: (2e-2, 1e-2)}


# ---------------------------------------------------------------------------
# host side (CPU)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("sink,window,max_q", [(4, 16, 4), (0, 7, 1), (3, 1, 2), (5, 0, 4), (1, 33, 3)])
def test_ring_layout_keeps_every_visible_position(sink, window, max_q):
    """Simulate appends slot by slot (last writer wins) and check that after
    every length, each position some decode row can see is still in its slot."""
    ring = max(1, window + max_q - 1)
    slots = {}
    for length in range(1, 3 * (sink + ring) + 20):
        p = length - 1
        slots[ring_slot(p, sink, ring)] = p
        assert all(0 <= s < sink + ring for s in slots)
        for n_q in range(1, min(max_q, length) + 1):
            vis = so.token_mask(n_q, length, sink, window).any(axis=0)
            for k in np.nonzero(vis)[0]:
                assert slots.get(ring_slot(int(k), sink, ring)) == k, (length, n_q, k)


def test_rolling_stream_is_the_union_of_visible_positions():
    rng = np.random.default_rng(0)
    for _ in range(400):
        sink, window = int(rng.integers(0, 9)), int(rng.integers(0, 40))
        n_q = int(rng.integers(1, 5))
        length = int(rng.integers(n_q, 120))
        ring = window + n_q - 1 + int(rng.integers(0, 3))
        if ring < 1:
            continue
        n_sink, w_lo, n_tok = rolling_stream(length, n_q, sink, window, ring)
        stream = list(range(n_sink)) + list(range(w_lo, length))
        assert n_tok == len(stream) and len(set(stream)) == len(stream)
        assert stream == sorted(stream)
        vis = set(np.nonzero(so.token_mask(n_q, length, sink, window).any(axis=0))[0].tolist())
        assert vis <= set(stream)
        if window >= 1:
            assert set(stream) == vis, (sink, window, n_q, length)
        else:
            # W = 0 sees only sinks; the stream keeps the rows' own hull, masked per element
            assert set(stream) - vis <= set(range(length - n_q + 1, length))


def test_rolling_stream_matches_full_cache_stream_c4():
    """c4 (n_q = 1, KV 100000, S4 W2048): the stream the full-cache decode walks
    (positions 0-3 and 97952-99999, pinned in test_gpu_parity) is the rolling one."""
    n_sink, w_lo, n_tok = rolling_stream(100000, 1, 4, 2048, 2048)
    assert (n_sink, w_lo, n_tok) == (4, 100000 - 2048, 2052)


def test_rolling_capi_rejects_bad_arguments():
    lib = _lib.load()
    out = ctypes.c_int32()
    # ring too small for the window and the decode rows
    assert lib.gki_rolling_stream(100, 2, 4, 16, 16, None, None, ctypes.byref(out)) == 1
    assert b"ring_size" in lib.gki_last_error()
    # too many decode rows / length shorter than the rows
    assert lib.gki_rolling_stream(100, 5, 4, 16, 32, None, None, None) == 2
    assert lib.gki_rolling_stream(2, 3, 4, 16, 32, None, None, None) == 1
    # decode head_dim limited to 64 / 128; checked before any launch
    null = ctypes.c_void_p(0)
    rc = lib.gki_rolling_decode(1, 1, 1, 1, 1, 2, 1, 1, 1, 1, 32, 4, 16, 16, 100, 0.1, null, 1, null)
    assert rc == 2 and b"head_dim" in lib.gki_last_error()
    rc = lib.gki_rolling_decode(None, 1, 1, 1, 1, 2, 1, 1, 1, 1, 64, 4, 16, 16, 100, 0.1, null, 1, null)
    assert rc == 1 and b"null" in lib.gki_last_error()
    rc = lib.gki_rolling_append(1, 1, 1, 1, 2, 1, 1, 64, 4, 16, -1, 1, null)
    assert rc == 1 and b"positions" in lib.gki_last_error()
    assert lib.gki_rolling_append(None, None, None, None, 2, 1, 1, 64, 4, 16, 0, 0, null) == 0


def test_cache_rejects_bad_configuration():
    with pytest.raises(ValueError, match="head_dim"):
        StreamingKVCache(1, 1, 32, stk.StreamingMaskSpec(4, 16), device=DEV)
    with pytest.raises(ValueError, match="max_query"):
        StreamingKVCache(1, 1, 64, stk.StreamingMaskSpec(4, 16), device=DEV, max_query=5)
    with pytest.raises(ValueError, match="CUDA"):
        StreamingKVCache(1, 1, 64, stk.StreamingMaskSpec(4, 16), device="cpu")


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------


def _close(ours, ref, dtype, what):
    atol, rtol = TOL[dtype]
    o = ours.detach().to(torch.float64).cpu()
    r = ref.detach().to(torch.float64).cpu() if isinstance(ref, torch.Tensor) else torch.from_numpy(ref)
    bad = (o - r).abs() > atol + rtol * r.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of tolerance, max err {(o - r).abs().max():.3e}"


def _on_matrix_cores(dtype, D, group, n_q):
    """The library's rule for the matrix-core decode of a computed stream
    (16-bit, head_dim 64 / 128, 2..32 query rows per K / V stream)."""
    return dtype != torch.float32 and D in (64, 128) and 2 <= group * n_q <= 32


def _full_cache_decode(q, k, v, sink, window):
    """The full-cache decode path (block_m = 1, block_n = 64, token rule) and
    the length of the token stream it walks."""
    n_q, n_kv = q.shape[2], k.shape[2]
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), 1, 64, device=DEV)
    o = stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                   sink_size=sink, window_size=window)
    n_tok = decode_schedule(mask, n_q, n_kv, 1, 64, True, sink, window).n_tokens
    return o, n_tok


def _oracle(q, k, v, sink, window):
    n_q, n_kv = q.shape[2], k.shape[2]
    eff = so.token_mask(n_q, n_kv, sink, window)
    qn, kn, vn = (t.to(torch.float64).cpu().numpy() for t in (q, k, v))
    return so.attention_fwd(qn, kn, vn, eff, 1.0 / math.sqrt(q.shape[-1]))


def _randn(shape, dtype, gen):
    return torch.randn(shape, generator=gen).to(dtype).to(DEV)


@pytest.mark.gpu
def test_append_places_tokens_in_their_slots():
    sink, window, max_q, B, H, D = 3, 37, 4, 2, 3, 64
    cache = StreamingKVCache(B, H, D, stk.StreamingMaskSpec(sink, window), torch.float16, DEV, max_q)
    ring = cache.ring_size
    gen = torch.Generator().manual_seed(7)
    k_all = _randn((B, H, 400, D), torch.float16, gen)
    v_all = _randn((B, H, 400, D), torch.float16, gen)
    pos = 0
    for n in (1, 2, 5, 60, 1, 100, 7, 224):          # includes chunks longer than the ring
        print(f"[append] {pos}..{pos + n}", flush=True)
        cache.append(k_all[:, :, pos:pos + n], v_all[:, :, pos:pos + n])
        pos += n
        torch.cuda.synchronize()
        live = list(range(min(sink, pos))) + list(range(max(sink, pos - ring), pos))
        for p in live:
            s = ring_slot(p, sink, ring)
            assert torch.equal(cache.k_cache[:, :, s], k_all[:, :, p]), (pos, p)
            assert torch.equal(cache.v_cache[:, :, s], v_all[:, :, p]), (pos, p)
    assert cache.length == 400


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,D,dtype,sink,window,length,n_q", [
    (2, 4, 128, torch.bfloat16, 4, 2048, 10000, 1),      # c4 shape per head, shorter cache
    (1, 8, 64, torch.float16, 4, 256, 3000, 1),
    (2, 2, 64, torch.bfloat16, 4, 256, 3001, 4),
    (1, 3, 128, torch.float32, 4, 100, 1000, 2),
    (1, 2, 64, torch.float16, 4, 256, 200, 1),           # cache shorter than S + W
    (1, 2, 128, torch.bfloat16, 4, 64, 3, 3),            # length < sink
    (1, 2, 64, torch.float32, 0, 50, 500, 3),            # no sink
    (2, 2, 64, torch.float16, 4, 0, 300, 2),             # sinks only
])
def test_rolling_decode_matches_full_cache_and_oracle(B, H, D, dtype, sink, window, length, n_q):
    tag = f"B{B} H{H} D{D} {dtype} S{sink} W{window} L{length} nq{n_q}"
    print(f"[case] {tag}", flush=True)
    gen = torch.Generator().manual_seed(length + D)
    k = _randn((B, H, length, D), dtype, gen)
    v = _randn((B, H, length, D), dtype, gen)
    q = _randn((B, H, n_q, D), dtype, gen)
    cache = StreamingKVCache(B, H, D, stk.StreamingMaskSpec(sink, window), dtype, DEV)
    cache.append(k, v)                                   # whole prefill in one call
    o, lse = cache.attend(q, return_lse=True)
    o_full, n_full = _full_cache_decode(q, k, v, sink, window)
    n_roll = rolling_stream(length, n_q, sink, window, cache.ring_size)[2]
    listed = decode_schedule(stk.make_streaming_mask(n_q, length, stk.StreamingMaskSpec(sink, window), 1,
                                                     64, device=DEV), n_q, length, 1, 64, True, sink,
                             window).ring == 0
    if n_roll == n_full and listed and _on_matrix_cores(dtype, D, 1, n_q):
        # a full cache too short for the computed stream decodes its list with
        # the 4-row kernel, the rolling cache on the matrix cores
        _close(o, o_full.float(), dtype, "rolling vs full cache " + tag)
    elif n_roll == n_full:
        assert torch.equal(o, o_full), tag
    o_ref, lse_ref = _oracle(q, k, v, sink, window)
    _close(o, o_ref, dtype, "O " + tag)
    np.testing.assert_allclose(lse.cpu().numpy(), lse_ref, atol=1e-4, rtol=1e-5, err_msg="LSE " + tag)


@pytest.mark.gpu
def test_rolling_decode_steps_across_the_ring_wrap():
    """Token-by-token decode (append one K/V row, attend) past several wraps of
    the ring; every step equals the full-cache decode over the same prefix."""
    B, H, D, dtype, sink, window = 1, 2, 64, torch.float16, 4, 96
    steps, prefill = 260, 40
    gen = torch.Generator().manual_seed(5)
    k = _randn((B, H, prefill + steps, D), dtype, gen)
    v = _randn((B, H, prefill + steps, D), dtype, gen)
    q = _randn((B, H, prefill + steps, D), dtype, gen)
    cache = StreamingKVCache(B, H, D, stk.StreamingMaskSpec(sink, window), dtype, DEV, max_query=1)
    cache.append(k[:, :, :prefill], v[:, :, :prefill])
    n_exact = 0
    for t in range(prefill, prefill + steps):
        o = cache.step(q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1])
        o_full, n_full = _full_cache_decode(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], sink, window)
        if rolling_stream(t + 1, 1, sink, window, cache.ring_size)[2] == n_full:
            assert torch.equal(o, o_full), f"step {t}"
            n_exact += 1
        else:
            _close(o, o_full.float(), dtype, f"step {t}")
    assert n_exact > steps // 2
    o_ref, _ = _oracle(q[:, :, -1:], k, v, sink, window)
    _close(o, o_ref, dtype, "last step vs oracle")


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,H_kv,n_q,n_kv,D,S,W,dtype", [
    (2, 4, 4, 1, 3000, 128, 4, 512, torch.bfloat16),
    (1, 8, 2, 1, 5000, 128, 4, 1024, torch.bfloat16),   # grouped-query, 4 heads per stream
    (2, 3, 3, 3, 700, 64, 2, 100, torch.float16),
    (1, 4, 1, 2, 900, 64, 0, 200, torch.float32),
])
def test_full_cache_decode_computes_the_stream(B, H, H_kv, n_q, n_kv, D, S, W, dtype):
    """A StreamingLLM mask's decode stream is computed in the kernel (the full
    cache decoded as a sink + ring cache, slot = position) instead of read from
    the token list; both give the same bits where both run the same kernel. A
    custom mask keeps the list."""
    print(f"[case] B{B} H{H}/{H_kv} nq{n_q} nkv{n_kv} D{D} S{S} W{W} {dtype}", flush=True)
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), 1, 64, device=DEV)
    sched = decode_schedule(mask, n_q, n_kv, 1, 64, True, S, W)
    assert sched.ring == n_kv - S
    g = torch.Generator().manual_seed(n_kv + n_q)
    mk = lambda *s: torch.randn(*s, generator=g).to(dtype).to(DEV)  # noqa: E731
    q, k, v = mk(B, H, n_q, D), mk(B, H_kv, n_kv, D), mk(B, H_kv, n_kv, D)
    o = stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                   sink_size=S, window_size=W, enable_gqa=H != H_kv)
    # the token-list entry on the same schedule
    from gki import ops
    lib = _lib.load()
    n_splits = ops._decode_splits(sched.n_tokens, ops._decode_slots(B, H, H_kv, n_q, 4))
    ws = torch.empty(max(1, int(lib.gki_bsa_decode_workspace_floats(B, H, n_q, D, n_splits))),
                     device=DEV)
    o_list = torch.empty_like(q)
    lse = torch.empty(B, H, n_q, device=DEV)
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    _lib.check(lib.gki_bsa_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), o_list.data_ptr(),
                                  lse.data_ptr(), code, B, H, H_kv, n_q, n_kv, D,
                                  sched.tokens.data_ptr(), sched.n_tokens, mask.data_ptr(),
                                  mask.shape[0], mask.shape[1], 1, 64, 1.0 / math.sqrt(D), 1, S, W,
                                  ws.data_ptr() if n_splits > 1 else 0, n_splits,
                                  torch.cuda.current_stream().cuda_stream), "gki_bsa_decode")
    torch.cuda.synchronize()
    if _on_matrix_cores(dtype, D, H // H_kv, n_q):
        # 2..16 query rows per K / V stream on the computed stream run the
        # matrix-core kernel, the list the 4-row kernel: the same stream (pinned
        # bit for bit by the single-row and fp32 cases, which share the token
        # source), other arithmetic
        _close(o, o_list.float(), dtype, "computed vs listed stream")
    else:
        assert torch.equal(o, o_list)
    # a custom mask (one window block dropped) keeps the token list
    m2 = mask.clone()
    m2[0, -2] = 0
    assert decode_schedule(m2, n_q, n_kv, 1, 64, True, S, W).ring == 0


@pytest.mark.gpu
@pytest.mark.parametrize("bh,n_kv,D,dtype,sink,window", [
    (3, 1000, 128, torch.bfloat16, 4, 300),
    (2, 50, 64, torch.float16, 8, 100),          # the window reaches the sinks: every row once
    (1, 5, 64, torch.float32, 10, 0),            # more sinks than rows, no window
    (4, 4099, 128, torch.float16, 0, 2048),
])
def test_read_probe_reads_exactly_the_decode_rows(bh, n_kv, D, dtype, sink, window):
    """gki_read_probe (bench.py's read ceiling of the decode step) folds exactly
    the sink rows and the window rows of every slice: the XOR of its output
    words is the XOR of those rows' 32-bit words."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(n_kv)
    k = torch.randn(bh, n_kv, D, generator=gen).to(dtype)
    v = torch.randn(bh, n_kv, D, generator=gen).to(dtype)
    words = int(lib.gki_read_probe_words(bh))
    out = torch.full((words,), -1, dtype=torch.int32, device=DEV)
    kd, vd = k.to(DEV), v.to(DEV)
    _lib.check(lib.gki_read_probe(kd.data_ptr(), vd.data_ptr(), bh, n_kv, D * k.element_size(), sink, window,
                                  out.data_ptr(), words, torch.cuda.current_stream().cuda_stream),
               "gki_read_probe")
    n_sink = min(sink, n_kv)
    w_lo = max(n_sink, n_kv - window)
    rows = [t[:, :n_sink] for t in (k, v)] + [t[:, w_lo:] for t in (k, v)]
    want = np.bitwise_xor.reduce(np.concatenate([r.contiguous().view(torch.int32).numpy().ravel()
                                                 for r in rows] + [np.zeros(1, np.int32)]))
    assert np.bitwise_xor.reduce(out.cpu().numpy()) == want
