"""Seeded random sweep of the mask and schedule builders against the oracle (GPU).

Each case draws a geometry (1-3000 query and key positions, the reference's
block sizes 1-128, sink 0-8, window 0-1500, causal or not, 1-4 q heads per kv
head over 1-4 kv heads) and either the StreamingLLM block mask or a random one
of random density (empty rows and columns included). Checked bit for bit: the
device StreamingLLM mask against the closed form (sparse_triton_kernel.py:154-181),
the kept-block lists against ``np.nonzero`` order, the forward CSR over the
16-bit and fp32 q tiles, and the backward CSR / CSC and dK/dV work list over
the kernels' 64 x 64 tiles against the oracle's tile classification.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import sparse_triton_kernel as stk
from gki import _lib, build_block_lists
from gki.lists import bwd_schedule, fwd_schedule
from oracle import streaming_oracle as so

DEV = "cuda"
BLOCKS = [1, 2, 8, 16, 32, 64, 128]
N_CASES = 48


def _case(seed):
    rng = np.random.default_rng(7000 + seed)
    n_kv = int(np.exp(rng.uniform(0, np.log(3000))))
    n_q = n_kv if rng.random() < 0.5 else int(np.exp(rng.uniform(0, np.log(3000))))
    return dict(n_q=max(1, n_q), n_kv=max(1, n_kv), bm=int(rng.choice(BLOCKS)), bn=int(rng.choice(BLOCKS)),
                sink=int(rng.integers(0, 9)), window=0 if rng.random() < 0.1 else int(rng.integers(1, 1501)),
                causal=bool(rng.random() < 0.7), streaming=bool(rng.random() < 0.67),
                density=float(rng.uniform(0, 1)), group=int(rng.choice([1, 2, 4])),
                bh_kv=int(rng.integers(1, 5)), mask_seed=int(rng.integers(0, 1 << 30)))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_schedules_match_oracle(seed):
    c = _case(seed)
    print(f"[case] seed {seed}: {c}", flush=True)
    n_q, n_kv, bm, bn, sink, window, causal = (c[k] for k in ("n_q", "n_kv", "bm", "bn", "sink", "window",
                                                              "causal"))
    ref_mask = so.block_mask(n_q, n_kv, sink, window, bm, bn)
    dev_mask = stk.make_streaming_mask(n_q, n_kv, stk.StreamingMaskSpec(sink, window), bm, bn, device=DEV)
    np.testing.assert_array_equal(dev_mask.cpu().numpy(), ref_mask)
    if c["streaming"]:
        m = ref_mask
    else:
        mrng = np.random.default_rng(c["mask_seed"])
        m = (mrng.random(ref_mask.shape) < c["density"]).astype(np.int32)
    dm = torch.from_numpy(m).to(DEV)

    lists = build_block_lists(dm)
    for got, want in zip((lists.row_ptr, lists.row_idx, lists.col_ptr, lists.col_idx), so.kept_lists(m)):
        np.testing.assert_array_equal(got.cpu().numpy(), want)

    ts = _lib.tile_sizes()
    for fp32, key in ((False, "fwd_tile_m_16"), (True, "fwd_tile_m_32")):
        fs = fwd_schedule(dm, n_q, n_kv, bm, bn, causal, sink, window, fp32)
        tiles = so.tile_classes(m, n_q, n_kv, bm, bn, ts[key], ts["tile_n"], causal, sink, window)
        ref = so.kept_lists(tiles)
        assert fs.n_qt == tiles.shape[0]
        np.testing.assert_array_equal(fs.lists.row_ptr.cpu().numpy(), ref[0])
        np.testing.assert_array_equal(fs.lists.row_idx.cpu().numpy(), ref[1])

    sched = bwd_schedule(dm, n_q, n_kv, bm, bn, causal, sink, window, group=c["group"], bh_kv=c["bh_kv"])
    tiles = so.tile_classes(m, n_q, n_kv, bm, bn, ts["bwd_tile_m"], ts["tile_n"], causal, sink, window)
    ref = so.kept_lists(tiles)
    L = sched.lists
    for got, want in zip((L.row_ptr, L.row_idx, L.col_ptr, L.col_idx), ref):
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    items, split, n_pslots = so.dkdv_items(ref[2], c["group"], c["bh_kv"])
    np.testing.assert_array_equal(sched.items.cpu().numpy(), items)
    np.testing.assert_array_equal(sched.split.cpu().numpy()[:sched.n_split], split)
    assert (sched.n_items, sched.n_split, sched.n_pslots) == (len(items), len(split), n_pslots)
