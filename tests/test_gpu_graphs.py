"""HIP graph replay of the op's launch paths (``gpu``).

A serving loop captures its steps once and replays them. Every launch path of
the op is capturable once its schedule is cached (the first call builds it,
with a host read of the list length): the launches go onto the caller's
current stream, the op's own tensors come from torch's allocator (the graph's
pool during capture), and no path issues a memset. Each test captures one
step, then replays it several times with new contents in the static inputs,
with eager work and a device synchronisation between replays, and checks
every replay against an eager call on the same inputs: bit-identical, since
the replay runs the same kernels on the same data.
"""

from __future__ import annotations

import pytest
import torch

import sparse_triton_kernel as stk
from gki.kv_cache import StreamingKVCache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn, warmups: int = 3) -> tuple:
    """Warm `fn` up on a side stream (schedules built and cached there), then
    capture one call into a graph; returns (graph, static outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmups):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _replay_and_check(g, static_inputs, out, eager, seeds, make_inputs):
    """For each seed: eager work, new input contents, replay, compare."""
    for seed in seeds:
        new = make_inputs(seed)
        junk = torch.randn(1 << 20, device=DEV).sum()       # the program's own eager work
        for dst, src in zip(static_inputs, new):
            dst.copy_(src)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = eager(*new)
        got = out if isinstance(out, (tuple, list)) else (out,)
        want = want if isinstance(want, (tuple, list)) else (want,)
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay with seed {seed} differs from the eager call"
        del junk


@pytest.mark.parametrize("H_kv", [8, 2])
def test_decode_step_replays_in_a_graph(H_kv):
    """A c4-like decode step (n_q 1, StreamingLLM mask, matrix-core grouped-query
    path with its split merge for H_kv 2, the vector kernel for H_kv 8)."""
    B, H, N, D, S, W = 2, 8, 4096, 128, 4, 512
    mask = stk.make_streaming_mask(1, N, stk.StreamingMaskSpec(S, W), 1, 64, device=DEV)

    def make(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        return tuple(torch.randn(*shape, generator=g, device=DEV).to(torch.bfloat16)
                     for shape in ((B, H, 1, D), (B, H_kv, N, D), (B, H_kv, N, D)))

    q, k, v = make(0)

    def eager(q_, k_, v_):
        return stk.block_sparse_attention(q_, k_, v_, mask, block_m=1, block_n=64, is_causal=True,
                                          sink_size=S, window_size=W, enable_gqa=H_kv != H)

    graph, out = _capture(lambda: eager(q, k, v))
    _replay_and_check(graph, (q, k, v), out, eager, (1, 2, 3), make)


def test_prefill_forward_and_backward_replay_in_a_graph():
    """Forward and backward of a prefill step (fp16, D 64, causal streaming
    mask) captured together through torch.autograd.grad."""
    B, H, N, D, S, W = 1, 2, 1024, 64, 4, 256
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), 64, 64, device=DEV)

    def make(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        return tuple(torch.randn(B, H, N, D, generator=g, device=DEV).to(torch.float16)
                     for _ in range(4))

    q, k, v, do = make(0)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]

    def step_on(q_, k_, v_, do_, lv):
        for dst, src in zip(lv, (q_, k_, v_)):
            dst.data.copy_(src)
        o = stk.block_sparse_attention(*lv, mask, is_causal=True, sink_size=S, window_size=W)
        return (o,) + tuple(torch.autograd.grad(o, lv, do_))

    graph, out = _capture(lambda: step_on(q, k, v, do, leaves))

    fresh = [t.clone().requires_grad_(True) for t in (q, k, v)]

    def eager(q_, k_, v_, do_):
        return tuple(t.detach() for t in step_on(q_, k_, v_, do_, fresh))

    _replay_and_check(graph, (q, k, v, do), out, eager, (1, 2), make)


def test_rolling_cache_attend_replays_in_a_graph():
    """The rolling-cache decode at a fixed cache length (the append moves the
    position and stays outside the graph)."""
    B, H, D, S, W = 2, 4, 128, 4, 256
    cache = StreamingKVCache(B, H, D, stk.StreamingMaskSpec(S, W), torch.bfloat16, DEV, max_query=1)
    g0 = torch.Generator(device=DEV).manual_seed(7)
    k0, v0 = (torch.randn(B, H, 3000, D, generator=g0, device=DEV).to(torch.bfloat16) for _ in range(2))
    cache.append(k0, v0)

    def make(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        return (torch.randn(B, H, 1, D, generator=g, device=DEV).to(torch.bfloat16),)

    (q,) = make(0)
    graph, out = _capture(lambda: cache.attend(q))
    _replay_and_check(graph, (q,), out, lambda q_: cache.attend(q_), (1, 2, 3), make)
