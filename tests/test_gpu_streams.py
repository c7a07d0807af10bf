"""Streams and threads at the boundary: every entry point launches on the
calling thread's current stream and keeps no state between calls, and a
schedule is complete on the device before the cache hands it to another
stream. The op on a side stream, and two host threads each on its own
stream sharing one mask (and its cached schedules), must give the bits of
the sequential default-stream run (the kernels are deterministic)."""

from __future__ import annotations

import threading

import pytest
import torch

import sparse_triton_kernel as stk
from gki import clear_schedule_cache

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
B, H, N, D, S, W = 1, 4, 1024, 64, 4, 256


def _inputs(seed: int):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]


def _step(q, k, v, do, mask):
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    out = stk.block_sparse_attention(*leaves, mask, is_causal=True, sink_size=S, window_size=W)
    out.backward(do)
    return [out.detach()] + [t.grad for t in leaves]


def _same(a, b, what):
    for name, x, y in zip(("O", "dQ", "dK", "dV"), a, b):
        assert torch.equal(x, y), f"{what}: {name} differs from the sequential run"


def test_op_on_a_side_stream_matches_the_default_stream():
    print("[case] side stream, bf16 1x4x1024x64", flush=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), 64, 64, device=DEV)
    q, k, v, do = _inputs(11)
    ref = _step(q, k, v, do, mask)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = _step(q, k, v, do, mask)
    side.synchronize()
    _same(ref, got, "side stream")


def test_two_threads_on_their_own_streams_share_one_schedule():
    print("[case] two threads, two streams, one mask, cold schedule cache", flush=True)
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), 64, 64, device=DEV)
    inputs = [_inputs(21 + i) for i in range(2)]
    refs = [_step(*x, mask) for x in inputs]
    torch.cuda.synchronize()
    clear_schedule_cache()           # both threads meet the cold cache
    start = threading.Barrier(2)
    results, errors = [None, None], []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            start.wait()
            with torch.cuda.stream(stream):
                outs = [_step(*inputs[i], mask) for _ in range(4)]
            stream.synchronize()
            results[i] = outs
        except Exception as exc:     # surfaced on the main thread below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for i in range(2):
        for j, got in enumerate(results[i]):
            _same(refs[i], got, f"thread {i} call {j}")
