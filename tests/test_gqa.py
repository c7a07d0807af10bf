"""Grouped-query / multi-query attention (K/V with H_kv heads, H_kv | H).

The reference rejects any head mismatch (sparse_triton_kernel.py:640-641) and
its SDPA matcher ignores ``enable_gqa`` (fx_compiler_pass.py:295-308); this
build accepts it behind ``enable_gqa=True`` (default off: the reference's error
stays).

CPU: the oracle's head expansion against torch (repeat_interleave, its autograd
adjoint, SDPA ``enable_gqa=True``), and the FX matcher's handling of
``enable_gqa``.
GPU: prefill forward and dQ bit-identical to the multi-head op on expanded K/V;
dK/dV, decode and the rolling cache against the fp64 oracle (BASELINE
tolerances); the argument checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812

import fx_compiler_pass as fxp
import sparse_triton_kernel as stk
from gki.kv_cache import StreamingKVCache
from oracle import streaming_oracle as so

DEV = "cuda"
TOL = {torch.float32: (1e-5, 0.0), torch.float16: (2e-2, 1e-2), torch.bfloat16: (2e-2, 1e-2)}


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------


def test_expand_kv_heads_is_repeat_interleave_and_reduce_is_its_adjoint():
    k = _rand((2, 3, 5, 4), 1)
    np.testing.assert_array_equal(so.expand_kv_heads(k, 4),
                                  torch.from_numpy(k).repeat_interleave(4, dim=1).numpy())
    t = torch.from_numpy(k).requires_grad_(True)
    g = _rand((2, 12, 5, 4), 2)
    t.repeat_interleave(4, dim=1).backward(torch.from_numpy(g))
    np.testing.assert_allclose(so.reduce_kv_grad(g, 4), t.grad.numpy(), atol=1e-14)


@pytest.mark.parametrize("H,H_kv", [(8, 2), (6, 1), (4, 4)])
def test_oracle_gqa_matches_torch_sdpa_enable_gqa(H, H_kv):
    """torch's SDPA with enable_gqa fixes the head mapping h -> h // group."""
    B, n_q, n_kv, D = 2, 30, 50, 8
    q, k, v = _rand((B, H, n_q, D), 3), _rand((B, H_kv, n_kv, D), 4), _rand((B, H_kv, n_kv, D), 5)
    eff = so.token_mask(n_q, n_kv, 3, 9)
    g = H // H_kv
    o, _ = so.attention_fwd(q, so.expand_kv_heads(k, g), so.expand_kv_heads(v, g), eff, 0.4)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                         attn_mask=torch.from_numpy(eff), scale=0.4, enable_gqa=True)
    np.testing.assert_allclose(o, ref.numpy(), atol=1e-12)


class _GQASdpa(torch.nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)


class _MHASdpa(torch.nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def test_fx_sdpa_enable_gqa_is_carried_to_the_module():
    cfg = fxp.InjectionConfig(seq_len_q=128, seq_len_kv=128, head_dim=64,
                              streaming=stk.StreamingMaskSpec(4, 32))
    gm = fxp.BlockSparseAttentionInjector(cfg).transform(_GQASdpa())
    assert gm._triton_attn_0.enable_gqa is True
    gm = fxp.BlockSparseAttentionInjector(cfg).transform(_MHASdpa())
    assert gm._triton_attn_0.enable_gqa is False


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------


def _close(ours, ref, dtype, what):
    atol, rtol = TOL[dtype]
    o = ours.detach().to(torch.float64).cpu()
    r = torch.as_tensor(ref).to(torch.float64)
    bad = (o - r).abs() > atol + rtol * r.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} out of tolerance, max err {(o - r).abs().max():.3e}"


def _inputs(B, H, H_kv, n_q, n_kv, D, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=gen).to(dtype).to(DEV)  # noqa: E731
    return mk(B, H, n_q, D), mk(B, H_kv, n_kv, D), mk(B, H_kv, n_kv, D), mk(B, H, n_q, D)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,H,H_kv,n_q,n_kv,D,bm,bn,S,W", [
    (1, 8, 2, 300, 300, 64, 64, 64, 4, 64),
    (2, 6, 1, 257, 400, 128, 32, 64, 4, 100),     # MQA, ragged, prefill offset
    (1, 4, 2, 200, 200, 32, 16, 16, 2, 50),
])
def test_gqa_prefill_fwd_bwd(B, H, H_kv, n_q, n_kv, D, bm, bn, S, W, dtype):
    tag = f"B{B} H{H}/{H_kv} nq{n_q} nkv{n_kv} D{D} {dtype} bm{bm} bn{bn} S{S} W{W}"
    print(f"[case] {tag}", flush=True)
    g = H // H_kv
    q, k, v, do = _inputs(B, H, H_kv, n_q, n_kv, D, dtype, n_q + D)
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), bm, bn, device=DEV)
    lq, lk, lv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = stk.block_sparse_attention(lq, lk, lv, mask, block_m=bm, block_n=bn, is_causal=True,
                                     sink_size=S, window_size=W, enable_gqa=True)
    out.backward(do)
    # the same op on K/V expanded to H heads: same kernels, same bits for O and dQ
    eq, ek, ev = q.clone().requires_grad_(True), k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
    ek.requires_grad_(True)
    ev.requires_grad_(True)
    out_e = stk.block_sparse_attention(eq, ek, ev, mask, block_m=bm, block_n=bn, is_causal=True,
                                       sink_size=S, window_size=W)
    out_e.backward(do)
    assert torch.equal(out, out_e), tag
    assert torch.equal(lq.grad, eq.grad), tag
    # dK / dV (summed over each group in fp32) against the fp64 oracle
    eff = so.effective_mask(mask.cpu().numpy(), n_q, n_kv, bm, bn, True, S, W)
    qn, kn, vn, don = (t.to(torch.float64).cpu().numpy() for t in (q, k, v, do))
    kx, vx = so.expand_kv_heads(kn, g), so.expand_kv_heads(vn, g)
    o_ref, _ = so.attention_fwd(qn, kx, vx, eff, 1 / math.sqrt(D))
    dq_ref, dk_ref, dv_ref = so.attention_bwd(qn, kx, vx, don, eff, 1 / math.sqrt(D))
    _close(out, o_ref, dtype, "O " + tag)
    _close(lq.grad, dq_ref, dtype, "dQ " + tag)
    _close(lk.grad, so.reduce_kv_grad(dk_ref, g), dtype, "dK " + tag)
    _close(lv.grad, so.reduce_kv_grad(dv_ref, g), dtype, "dV " + tag)


@pytest.mark.gpu
@pytest.mark.parametrize("H,H_kv,n_q,D,dtype,W", [
    (8, 2, 1, 128, torch.bfloat16, 1024),   # 4 heads share one K/V stream (matrix cores, 4 splits)
    (8, 4, 1, 64, torch.float16, 1024),     # group 2, head_dim 64 (matrix cores)
    (4, 1, 1, 128, torch.float16, 1024),    # MQA, group 4 (matrix cores)
    (8, 2, 1, 64, torch.bfloat16, 200),     # 204 tokens: one split, one ragged chunk
    (8, 2, 1, 128, torch.float16, 100),     # 104 tokens: last chunk one wave partly, one fully masked
    (8, 2, 2, 64, torch.float16, 1024),     # 4 x 2 rows > 4: one head per workgroup
    (4, 1, 1, 64, torch.float32, 1024),     # MQA, 4 heads per stream (fp32: 4-row kernel)
    (6, 3, 2, 128, torch.bfloat16, 1024),   # 2 heads x 2 rows
    (16, 2, 1, 128, torch.bfloat16, 1024),  # group 8 (matrix cores: 8 of 16 columns)
    (32, 2, 1, 64, torch.float16, 1024),    # group 16: all 16 columns
    (32, 1, 1, 128, torch.bfloat16, 1024),  # group 32: two 16-column blocks
    (32, 2, 2, 64, torch.float16, 1024),    # 16 heads x 2 positions: two blocks, token rule per row
    (64, 1, 1, 64, torch.bfloat16, 1024),   # group 64 > 32 rows: one head per workgroup, shared L2
])
def test_gqa_decode_and_rolling_cache(H, H_kv, n_q, D, dtype, W):
    B, n_kv, S = 2, 5000, 4
    tag = f"B{B} H{H}/{H_kv} nq{n_q} D{D} {dtype} W{W}"
    print(f"[case] {tag}", flush=True)
    g = H // H_kv
    q, k, v, _ = _inputs(B, H, H_kv, n_q, n_kv, D, dtype, H + n_q)
    mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(S, W), 1, 64, device=DEV)
    o = stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                   sink_size=S, window_size=W, enable_gqa=True)
    eff = so.token_mask(n_q, n_kv, S, W)
    qn, kn, vn = (t.to(torch.float64).cpu().numpy() for t in (q, k, v))
    o_ref, lse_ref = so.attention_fwd(qn, so.expand_kv_heads(kn, g), so.expand_kv_heads(vn, g), eff,
                                      1 / math.sqrt(D))
    _close(o, o_ref, dtype, "decode O " + tag)
    cache = StreamingKVCache(B, H_kv, D, stk.StreamingMaskSpec(S, W), dtype, DEV)
    cache.append(k, v)
    o_roll, lse = cache.attend(q, return_lse=True)
    assert torch.equal(o_roll, o), "rolling vs full cache " + tag
    np.testing.assert_allclose(lse.cpu().numpy(), lse_ref, atol=1e-4, rtol=1e-5)


@pytest.mark.gpu
def test_head_mismatch_needs_enable_gqa():
    q, k, v, _ = _inputs(1, 8, 2, 64, 64, 64, torch.float16, 0)
    mask = stk.make_streaming_mask(64, 64, stk.StreamingMaskSpec(4, 16), 64, 64, device=DEV)
    with pytest.raises(ValueError, match="batch/head/dim mismatch"):
        stk.block_sparse_attention(q, k, v, mask, is_causal=True, sink_size=4, window_size=16)
    q3 = q[:, :3].contiguous()
    with pytest.raises(ValueError, match="batch/head/dim mismatch"):
        stk.block_sparse_attention(q3, k, v, mask, is_causal=True, sink_size=4, window_size=16,
                                   enable_gqa=True)


@pytest.mark.gpu
def test_fx_gqa_model_runs_injected_kernel():
    cfg = fxp.InjectionConfig(seq_len_q=256, seq_len_kv=256, head_dim=64,
                              streaming=stk.StreamingMaskSpec(4, 64))
    gm = fxp.BlockSparseAttentionInjector(cfg).transform(_GQASdpa()).to(DEV)
    q, k, v, _ = _inputs(1, 8, 2, 256, 256, 64, torch.float32, 9)
    out = gm(q, k, v)
    eff = so.token_mask(256, 256, 4, 64)
    qn, kn, vn = (t.to(torch.float64).cpu().numpy() for t in (q, k, v))
    o_ref, _ = so.attention_fwd(qn, so.expand_kv_heads(kn, 4), so.expand_kv_heads(vn, 4), eff,
                                1 / 8.0)
    _close(out, o_ref, torch.float32, "FX GQA")
