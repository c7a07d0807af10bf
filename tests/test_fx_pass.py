"""FX rewrite tests (CPU): graph structure only, no kernel launch.

Restates the reference's tests/test_fx_sdpa.py (causal SDPA -> one
``_triton_attn_*`` call_module, two chained -> two, non-causal refused with
the same message, StreamingLLM params carried) and adds the eager
``StandardAttention`` motif (config 1's input module).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F  # noqa: N812

import fx_compiler_pass as fxp
from sparse_triton_kernel import StreamingMaskSpec
from oracle import streaming_oracle as so


class _CausalSDPA(nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)


class _NonCausalSDPA(nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v)


class _TwoSDPA(nn.Module):
    def forward(self, q, k, v):
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return F.scaled_dot_product_attention(a, k, v, is_causal=True)


class _DropoutSDPA(nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v, dropout_p=0.1, is_causal=True)


class _ScaledSDPA(nn.Module):
    def forward(self, q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.25)


class _DivAttention(nn.Module):
    def forward(self, q, k, v):
        s = torch.matmul(q, k.transpose(-2, -1)) / 8.0
        return torch.matmul(torch.softmax(s, dim=-1), v)


class _MixedModule(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = fxp.StandardAttention(16)

    def forward(self, q, k, v):
        a = self.attn(q, k, v)
        return F.scaled_dot_product_attention(a, k, v, is_causal=True)


def _cfg(**kw) -> fxp.InjectionConfig:
    base = dict(seq_len_q=64, seq_len_kv=64, head_dim=16,
                streaming=StreamingMaskSpec(sink_size=4, window_size=16),
                block_m=16, block_n=16, device="cpu")
    base.update(kw)
    return fxp.InjectionConfig(**base)


def _count(gm, pred):
    return sum(1 for n in gm.graph.nodes if pred(n))


def _sdpa_calls(gm):
    return _count(gm, lambda n: n.op == "call_function" and n.target is F.scaled_dot_product_attention)


def _injected(gm):
    return _count(gm, lambda n: n.op == "call_module" and str(n.target).startswith("_triton_attn_"))


def test_single_causal_sdpa_rewritten():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(_CausalSDPA())
    assert _sdpa_calls(gm) == 0 and _injected(gm) == 1


def test_two_chained_sdpa_rewritten():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(_TwoSDPA())
    assert _sdpa_calls(gm) == 0 and _injected(gm) == 2
    # the second call consumes the first call's output
    mods = [n for n in gm.graph.nodes if n.op == "call_module"]
    assert mods[1].args[0] is mods[0]


def test_non_causal_sdpa_refused():
    with pytest.raises(RuntimeError, match="No scaled-dot-product-attention"):
        fxp.BlockSparseAttentionInjector(_cfg()).transform(_NonCausalSDPA())


def test_dropout_sdpa_refused():
    with pytest.raises(RuntimeError, match="No scaled-dot-product-attention"):
        fxp.BlockSparseAttentionInjector(_cfg()).transform(_DropoutSDPA())


def test_injected_module_carries_streaming_params():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(_CausalSDPA())
    mod = gm.get_submodule("_triton_attn_0")
    assert mod.is_causal is True and mod.sink_size == 4 and mod.window_size == 16
    assert mod.softmax_scale == pytest.approx(1 / math.sqrt(16))
    assert (mod.block_m, mod.block_n) == (16, 16)
    np.testing.assert_array_equal(mod.block_mask.numpy(), so.block_mask(64, 64, 4, 16, 16, 16))
    assert "block_mask" not in gm.state_dict() and "_triton_attn_0.block_mask" not in gm.state_dict()


def test_sdpa_static_scale_and_plain_causal_window():
    gm = fxp.BlockSparseAttentionInjector(_cfg(streaming=None,
                                               custom_mask=torch.ones(4, 4))).transform(_ScaledSDPA())
    mod = gm.get_submodule("_triton_attn_0")
    assert mod.softmax_scale == 0.25
    assert mod.sink_size == 0 and mod.window_size == 64 and mod.is_causal is True


def test_standard_attention_eager_motif_rewritten():
    cfg = fxp.InjectionConfig(seq_len_q=1024, seq_len_kv=1024, head_dim=64,
                              streaming=StreamingMaskSpec(4, 256), device="cpu")
    gm = fxp.BlockSparseAttentionInjector(cfg).transform(fxp.StandardAttention(64))
    ops = [n.target for n in gm.graph.nodes if n.op == "call_function"]
    assert torch.softmax not in ops and torch.matmul not in ops
    assert _injected(gm) == 1
    mod = gm.get_submodule("_triton_attn_0")
    assert mod.softmax_scale == pytest.approx(0.125)
    assert mod.is_causal and (mod.sink_size, mod.window_size) == (4, 256)
    assert int(mod.block_mask.sum()) == 81
    # the transpose is gone too
    assert _count(gm, lambda n: n.op == "call_method" and n.target == "transpose") == 0


def test_single_layer_transformer_rewritten_keeps_projections():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(fxp.SingleLayerTransformer(16, 64))
    assert _injected(gm) == 1
    assert _count(gm, lambda n: n.op == "call_module" and "proj" in str(n.target)) == 4


def test_truediv_scale_inverted():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(_DivAttention())
    assert gm.get_submodule("_triton_attn_0").softmax_scale == pytest.approx(1 / 8.0)


def test_eager_without_streaming_is_not_causal():
    gm = fxp.BlockSparseAttentionInjector(_cfg(streaming=None, custom_mask=torch.ones(4, 4))).transform(
        fxp.StandardAttention(16))
    mod = gm.get_submodule("_triton_attn_0")
    assert mod.is_causal is False and mod.sink_size == 0 and mod.window_size == 0


def test_numbering_eager_first_then_sdpa():
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(_MixedModule())
    targets = [n.target for n in gm.graph.nodes if n.op == "call_module"]
    assert targets == ["_triton_attn_0", "_triton_attn_1"]
    assert gm.get_submodule("_triton_attn_1").softmax_scale == pytest.approx(0.25)


def test_custom_mask_wins_and_missing_config_raises():
    custom = torch.eye(4, dtype=torch.int64)
    inj = fxp.BlockSparseAttentionInjector(_cfg(custom_mask=custom))
    assert inj._mask.dtype == torch.int32 and torch.equal(inj._mask, custom.to(torch.int32))
    with pytest.raises(ValueError, match="streaming"):
        fxp.BlockSparseAttentionInjector(_cfg(streaming=None))


def test_original_model_untouched_and_pretty_print():
    model = fxp.StandardAttention(16)
    gm = fxp.BlockSparseAttentionInjector(_cfg()).transform(model)
    assert not hasattr(model, "_triton_attn_0")
    text = fxp.pretty_print_graph(gm, header="fused")
    assert text.startswith("=== fused ===") and "_triton_attn_0" in text and "# node tally:" in text
