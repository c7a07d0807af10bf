"""Schedule cache: identity hits, sharing between equal-content masks (one list
build per model, not per layer), and no sharing after an in-place change."""

from __future__ import annotations

import torch

from gki.lists import _ScheduleCache


def _builder(calls, tag):
    def build():
        calls.append(tag)
        return tag
    return build


def test_identity_hit_and_equal_content_sharing():
    c, calls = _ScheduleCache(), []
    a = torch.randint(0, 2, (8, 16), dtype=torch.int32)
    assert c.get(a, ("fwd", 1), _builder(calls, "A")) == "A"
    assert c.get(a, ("fwd", 1), _builder(calls, "X")) == "A"          # identity hit
    b = a.clone()                                                       # e.g. another layer's copy
    assert c.get(b, ("fwd", 1), _builder(calls, "B")) == "A"          # equal content: shared
    assert calls == ["A"]
    assert c.get(b, ("bwd", 1), _builder(calls, "C")) == "C"          # other schedule key
    d = a.clone()
    d[0, 0] ^= 1
    assert c.get(d, ("fwd", 1), _builder(calls, "D")) == "D"          # other content
    assert calls == ["A", "C", "D"]


def test_in_place_change_is_not_shared():
    c, calls = _ScheduleCache(), []
    a = torch.zeros((4, 4), dtype=torch.int32)
    assert c.get(a, ("k",), _builder(calls, "A")) == "A"
    a[1, 1] = 1                                                         # version bump: stale entry
    assert c.get(a, ("k",), _builder(calls, "A2")) == "A2"
    z = torch.zeros((4, 4), dtype=torch.int32)                          # old content of a
    assert c.get(z, ("k",), _builder(calls, "Z")) == "Z"              # a's first entry is stale
    assert calls == ["A", "A2", "Z"]
    e = a.clone()
    assert c.get(e, ("k",), _builder(calls, "E")) == "A2"


class _ThreeLayers(torch.nn.Module):
    def forward(self, q, k, v):
        F = torch.nn.functional
        x = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = F.scaled_dot_product_attention(x, k, v, is_causal=True)
        return F.scaled_dot_product_attention(x, k, v, is_causal=True)


import pytest  # noqa: E402


@pytest.mark.gpu
def test_injected_layers_build_one_schedule(monkeypatch):
    import fx_compiler_pass as fxp
    import gki.lists as lists
    import sparse_triton_kernel as stk

    lists.clear_schedule_cache()
    builds = []
    orig = lists._lists_of

    def counting(*a, **kw):
        builds.append(1)
        return orig(*a, **kw)

    monkeypatch.setattr(lists, "_lists_of", counting)
    cfg = fxp.InjectionConfig(seq_len_q=512, seq_len_kv=512, head_dim=64,
                              streaming=stk.StreamingMaskSpec(4, 128))
    gm = fxp.BlockSparseAttentionInjector(cfg).transform(_ThreeLayers()).to("cuda")
    masks = [getattr(gm, f"_triton_attn_{i}").block_mask for i in range(3)]
    assert masks[0] is not masks[1] and masks[1] is not masks[2]        # one copy per layer
    q, k, v = (torch.randn(1, 2, 512, 64, device="cuda", dtype=torch.float16) for _ in range(3))
    out = gm(q, k, v)
    torch.cuda.synchronize()
    assert len(builds) == 1                                             # one forward list build
    ref = q
    for _ in range(3):
        ref = stk.block_sparse_attention(ref, k, v, masks[0], is_causal=True, sink_size=4,
                                         window_size=128)
    assert torch.equal(out, ref)


def test_many_layers_steady_state_makes_no_comparison_and_no_build(monkeypatch):
    """24 layers, each with its own copy of one mask, fwd + bwd schedules per
    step: the first step resolves every copy once (one comparison each) and
    builds two schedules; later steps neither compare nor build."""
    import gki.lists as lists

    c, calls = _ScheduleCache(), []
    base = torch.randint(0, 2, (32, 32), dtype=torch.int32)
    layers = [base.clone() for _ in range(24)]
    compares = []
    orig_equal = torch.equal

    def counting_equal(a, b):
        compares.append(1)
        return orig_equal(a, b)

    monkeypatch.setattr(lists.torch, "equal", counting_equal)

    def step():
        for m in layers:
            assert c.get(m, ("fwd",), _builder(calls, "F")) == "F"
        for m in reversed(layers):
            assert c.get(m, ("bwd",), _builder(calls, "B")) == "B"

    step()
    assert calls == ["F", "B"] and len(compares) == 23
    for _ in range(3):
        step()
    assert calls == ["F", "B"] and len(compares) == 23


def test_dead_masks_leave_the_alias_table():
    """50 short-lived masks of 3 contents: 3 classes (their first tensors are
    the representatives, held by the class table), 3 builds, and only the
    representatives' aliases left."""
    c, calls = _ScheduleCache(), []
    for i in range(50):
        m = torch.full((4, 4), i % 3, dtype=torch.int32)
        assert c.get(m, ("k",), _builder(calls, i)) == i % 3
        del m
    assert calls == [0, 1, 2] and len(c._classes) == 3 and len(c._alias) == 3
