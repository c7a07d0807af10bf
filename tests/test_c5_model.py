"""Config 5: the long-context GPT model, FX-rewritten, against the eager-masked model.

a 12-layer GPT-style decoder (d_model 1024, 16 heads, D 64,
MLP 4x, pre-LN RMSNorm), random-init weights from seed 4, B 1, N 131072 token
ids ~ U[0, 32000), bf16, causal ``F.scaled_dot_product_attention`` rewritten
by the FX pass (fx_compiler_pass.py:295-308 matcher) with the StreamingLLM
mask S 4, W 4096 on 128x64 blocks; fwd+bwd loss equivalence against the same
model with the eager masked attention (sparse_triton_kernel.py:845-902).

The eager reference needs Theta(N^2) memory (about 1.1 TB per layer at N
131072), so the reference model runs the oracle's memory-bounded exact
restatement (``oracle/chunked_reference.py``: the same softmax over
lift(mask) & token rule, chunk by chunk, fp32 math, output cast to bf16)
behind an autograd function. Both models share every weight; the rewritten
one runs this build's HIP kernels through ``_InjectedTritonAttention``.

Bars (bf16 model; the attention kernels round P to bf16 before P V, the
reference does not): the scalar loss within 2e-3 relative, every parameter
gradient within 3e-2 relative Frobenius error and cosine >= 0.999 against the
reference model's. A smaller two-layer case at N 8192 runs first; there a
reference model that ignores the window (plain causal attention) must fail
the same gradient bars, so the comparison can tell a wrong mask.
"""

from __future__ import annotations

import math
import time

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F  # noqa: N812

import fx_compiler_pass as fxp
import sparse_triton_kernel as stk
from oracle import chunked_reference as cr

DEV = "cuda"
VOCAB, D_MODEL, HEADS, HEAD_DIM = 32000, 1024, 16, 64
SINK, WINDOW, BM, BN = 4, 4096, 128, 64


def _sdpa_causal(q, k, v):
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


class _EagerMaskedAttention(torch.autograd.Function):
    """Exact masked attention (chunked oracle, fp32 math) with its closed-form backward."""

    @staticmethod
    def forward(ctx, q, k, v, mask, window):  # type: ignore[override]
        o, _ = cr.chunked_attention(q, k, v, mask, BM, BN, True, SINK, window, chunk=2048,
                                    dtype=torch.float32)
        ctx.save_for_backward(q, k, v, mask)
        ctx.window = window
        return o.to(q.dtype)

    @staticmethod
    def backward(ctx, do):  # type: ignore[override]
        q, k, v, mask = ctx.saved_tensors
        _, _, dq, dk, dv = cr.chunked_attention(q, k, v, mask, BM, BN, True, SINK, ctx.window,
                                                do=do.contiguous(), chunk=2048, dtype=torch.float32)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None


class Block(nn.Module):
    def __init__(self, attn):
        super().__init__()
        self.attn = attn
        self.n1 = nn.RMSNorm(D_MODEL)
        self.qkv = nn.Linear(D_MODEL, 3 * D_MODEL, bias=False)
        self.proj = nn.Linear(D_MODEL, D_MODEL, bias=False)
        self.n2 = nn.RMSNorm(D_MODEL)
        self.fc1 = nn.Linear(D_MODEL, 4 * D_MODEL, bias=False)
        self.fc2 = nn.Linear(4 * D_MODEL, D_MODEL, bias=False)

    def forward(self, x):
        b, n = x.size(0), x.size(1)
        qkv = self.qkv(self.n1(x)).view(b, n, 3, HEADS, HEAD_DIM).permute(2, 0, 3, 1, 4)
        a = self.attn(qkv[0], qkv[1], qkv[2])
        x = x + self.proj(a.transpose(1, 2).reshape(b, n, D_MODEL))
        return x + self.fc2(F.gelu(self.fc1(self.n2(x))))


class GPT(nn.Module):
    def __init__(self, n_layers, attn=_sdpa_causal):
        super().__init__()
        self.emb = nn.Embedding(VOCAB, D_MODEL)
        self.blocks = nn.ModuleList([Block(attn) for _ in range(n_layers)])
        self.norm = nn.RMSNorm(D_MODEL)
        self.head = nn.Linear(D_MODEL, VOCAB, bias=False)

    def forward(self, tokens):
        x = self.emb(tokens)
        for blk in self.blocks:
            x = blk(x)
        logits = self.head(self.norm(x))
        return F.cross_entropy(logits[0, :-1].float(), tokens[0, 1:])


def _loss_and_grads(model, tokens):
    model.zero_grad(set_to_none=True)
    loss = model(tokens)
    loss.backward()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters()}
    return loss.item(), grads


def _reference(base, n_layers, mask, window, tokens):
    ref = GPT(n_layers, attn=lambda q, k, v: _EagerMaskedAttention.apply(q, k, v, mask, window))
    ref = ref.to(torch.bfloat16)
    ref.load_state_dict(base.state_dict())
    return _loss_and_grads(ref.to(DEV), tokens)


def _grad_errors(grads_i, grads_r):
    """(name, relative Frobenius error, cosine) per parameter."""
    out = []
    for name, gr in grads_r.items():
        gi = grads_i[name]
        rel = ((gi - gr).norm() / gr.norm().clamp_min(1e-30)).item()
        out.append((name, rel, F.cosine_similarity(gi.flatten(), gr.flatten(), dim=0).item()))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n_layers,n", [(2, 8192), (12, 131072)])
def test_c5_model_loss_equivalence(n_layers, n):
    print(f"[case] c5 model: {n_layers} layers, N {n}", flush=True)
    torch.manual_seed(4)
    base = GPT(n_layers).to(torch.bfloat16)
    gen = torch.Generator().manual_seed(4)
    tokens = torch.randint(0, VOCAB, (1, n), generator=gen).to(DEV)
    mask = stk.make_streaming_mask(n, n, stk.StreamingMaskSpec(SINK, WINDOW), BM, BN, device=DEV)

    cfg = fxp.InjectionConfig(seq_len_q=n, seq_len_kv=n, head_dim=HEAD_DIM,
                              streaming=stk.StreamingMaskSpec(SINK, WINDOW), block_m=BM, block_n=BN)
    injected = fxp.BlockSparseAttentionInjector(cfg).transform(base).to(DEV)
    n_injected = sum(1 for m in injected.modules() if isinstance(m, fxp._InjectedTritonAttention))
    assert n_injected == n_layers

    t0 = time.perf_counter()
    loss_i, grads_i = _loss_and_grads(injected, tokens)
    torch.cuda.synchronize()
    print(f"[c5] injected fwd+bwd {time.perf_counter() - t0:.1f} s, loss {loss_i:.6f}", flush=True)
    del injected

    t0 = time.perf_counter()
    loss_r, grads_r = _reference(base, n_layers, mask, WINDOW, tokens)
    torch.cuda.synchronize()
    print(f"[c5] reference fwd+bwd {time.perf_counter() - t0:.1f} s, loss {loss_r:.6f}", flush=True)

    assert math.isfinite(loss_i) and abs(loss_i - loss_r) <= 2e-3 * abs(loss_r), (loss_i, loss_r)
    errs = _grad_errors(grads_i, grads_r)
    for name, rel, cos in errs:
        assert rel <= 3e-2 and cos >= 0.999, (name, rel, cos)
    worst = max(errs, key=lambda e: e[1])
    print(f"[c5] loss {loss_i:.6f} vs {loss_r:.6f}; worst grad rel err {worst[1]:.2e} ({worst[0]})", flush=True)

    if n <= 8192:
        # negative control: the same comparison against a model without the window
        dense = stk.make_streaming_mask(n, n, stk.StreamingMaskSpec(SINK, n), BM, BN, device=DEV)
        _, grads_d = _reference(base, n_layers, dense, n, tokens)
        bad = [(name, rel) for name, rel, cos in _grad_errors(grads_i, grads_d) if rel > 3e-2 or cos < 0.999]
        print(f"[c5] window-free reference: {len(bad)} of {len(errs)} gradients outside the bars", flush=True)
        assert bad, "the gradient bars do not distinguish a model without the window"
