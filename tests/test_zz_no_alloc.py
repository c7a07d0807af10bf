"""gki_rolling_decode_noalloc (the allocation-free decode entry point) against
gki_rolling_decode with a caller workspace, through the C ABI: bit-identical
O and LSE on two calls in a row, the second smaller, on both decode kernels
(grouped-query rows on the matrix cores, single rows on the vector decode);
no change of the device's free memory over repeated calls; and a clear error,
before any launch, for a request beyond the 16 MiB scratch."""

from __future__ import annotations

import math

import pytest
import torch

from gki import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, H, H_kv, n_q, D, length, S, W, n_splits, seed, dtype=torch.bfloat16):
    print(f"[case] no-alloc decode B{B} H{H}/{H_kv} n_q{n_q} D{D} len{length} splits{n_splits}",
          flush=True)
    lib = _lib.load()
    ring = W + n_q - 1
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, H, n_q, D, generator=g, device=DEV).to(dtype)
    kc = torch.randn(B, H_kv, S + ring, D, generator=g, device=DEV).to(dtype)
    vc = torch.randn(B, H_kv, S + ring, D, generator=g, device=DEV).to(dtype)
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for noalloc in (False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, H, n_q), float("nan"), dtype=torch.float32, device=DEV)
        args = (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), lse.data_ptr(), code, B, H,
                H_kv, n_q, D, S, W, ring, length, 1.0 / math.sqrt(D))
        if noalloc:
            rc = lib.gki_rolling_decode_noalloc(*args, n_splits, stream)
        else:
            ws = torch.empty(max(1, int(lib.gki_bsa_decode_workspace_floats(B, H, n_q, D, n_splits))),
                             dtype=torch.float32, device=DEV)
            rc = lib.gki_rolling_decode(*args, ws.data_ptr(), n_splits, stream)
        assert rc == 0, lib.gki_last_error()
        torch.cuda.synchronize()
        outs.append((o, lse))
    (o_ws, lse_ws), (o_na, lse_na) = outs
    assert torch.isfinite(o_na).all() and torch.isfinite(lse_na).all()
    assert torch.equal(o_na, o_ws) and torch.equal(lse_na, lse_ws)


def test_noalloc_decode_equals_the_workspace_decode_twice():
    # large first call: grouped-query rows on the matrix cores, 6 splits
    _case(4, 32, 8, 1, 128, 6000, 4, 2048, 6, seed=61)
    # smaller second call on the same scratch: one row per K / V stream (vector decode)
    _case(1, 4, 4, 1, 64, 3000, 4, 512, 3, seed=62)


def test_noalloc_decode_single_split_and_positions():
    _case(2, 8, 8, 3, 128, 900, 4, 256, 1, seed=63, dtype=torch.float16)
    _case(2, 8, 2, 2, 64, 900, 4, 256, 2, seed=64, dtype=torch.float16)


def test_noalloc_decode_allocates_nothing():
    """The entry point's defining contract: after a warm-up call (which loads the
    code object holding the scratch array), further calls with preallocated
    outputs leave the device's free memory unchanged -- no hipMalloc, no
    allocating library routine, on the split path (4 splits, the scratch) and
    on the single-split path."""
    lib = _lib.load()
    B, H, H_kv, n_q, D, length, S, W = 2, 16, 4, 1, 128, 5000, 4, 1024
    ring = W + n_q - 1
    g = torch.Generator().manual_seed(65)
    q = torch.randn(B, H, n_q, D, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.randn(B, H_kv, S + ring, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, H_kv, S + ring, D, generator=g).to(torch.bfloat16).to(DEV)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, n_q, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream

    def call(n_splits):
        rc = lib.gki_rolling_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(),
                                            lse.data_ptr(), 2, B, H, H_kv, n_q, D, S, W, ring, length,
                                            1.0 / math.sqrt(D), n_splits, stream)
        assert rc == 0, lib.gki_last_error()

    for n_splits in (4, 1):          # warm-up: code objects loaded, scratch address looked up
        call(n_splits)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(20):
        for n_splits in (4, 1):
            call(n_splits)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()


def test_noalloc_decode_rejects_requests_beyond_the_scratch():
    lib = _lib.load()
    B, H, n_q, D, n_splits = 64, 64, 1, 128, 8          # 4,259,840 floats > 4,194,304
    assert lib.gki_bsa_decode_workspace_floats(B, H, n_q, D, n_splits) > (4 << 20)
    q = torch.zeros(B, H, n_q, D, device=DEV, dtype=torch.bfloat16)
    kc = torch.zeros(B, H, 4 + 2048, D, device=DEV, dtype=torch.bfloat16)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, n_q, device=DEV)
    rc = lib.gki_rolling_decode_noalloc(q.data_ptr(), kc.data_ptr(), kc.data_ptr(), o.data_ptr(),
                                        lse.data_ptr(), 2, B, H, H, n_q, D, 4, 2048, 2048, 5000,
                                        0.1, n_splits, torch.cuda.current_stream().cuda_stream)
    assert rc == 1
    assert b"exceeds the library scratch" in lib.gki_last_error()
