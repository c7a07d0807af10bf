"""The kernels' 64-element visibility words against the oracle (CPU).

The 16-bit attention kernels decide which elements of a tile that needs a mask
are visible through one 64-bit word per lane: `row_valid_bits` (one query row
against the 64 keys of a tile: forward, dQ) and `col_valid_bits` (one key
against the 64 query rows of a tile: dK/dV), both in
graph-kernel-injection_amd/csrc/gki_common.cuh. This test builds those same
functions into a host program (tests/mask_bits_host.hip) and compares every
bit with the oracle:

* partial tiles (the word ANDs in the block mask): the effective mask
  lift(mask) & token rule (sparse_triton_kernel.py:881-894), or lift(mask)
  alone when not causal;
* other masked tiles (the tile class promises the effective mask equals the
  token rule there): the token rule (sparse_triton_kernel.py:905-932) and the
  bounds;
* rows / keys past n_q / n_kv: zero.

Random geometries cover non-divisible lengths, n_q < n_kv (prefill offset),
S = 0, W = 0, windows wider than the sequence, block sizes 1 .. 128 and random
(not streaming) block masks.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import streaming_oracle as so

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "graph-kernel-injection_amd", "csrc")


@pytest.fixture(scope="module")
def mask_bits_exe(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path_factory.mktemp("mask_bits") / "mask_bits_host")
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17", f"-I{CSRC}",
                    f"-I{os.path.join(REPO, 'include')}", os.path.join(HERE, "mask_bits_host.hip"),
                    "-o", exe], check=True, capture_output=True, timeout=600)
    return exe


def _cases(seed, n_geoms):
    rng = np.random.default_rng(seed)
    sizes = [1, 16, 32, 48, 64, 100, 128]
    for _ in range(n_geoms):
        n_kv = int(rng.integers(1, 700))
        n_q = n_kv if rng.random() < 0.3 else int(rng.integers(1, n_kv + 1))
        causal = bool(rng.random() < 0.8)
        sink = 0 if rng.random() < 0.25 else int(rng.integers(0, 70))
        window = 0 if rng.random() < 0.2 else int(rng.integers(1, 900))
        bm, bn = int(rng.choice(sizes)), int(rng.choice(sizes))
        n_qb, n_kb = -(-n_q // bm), -(-n_kv // bn)
        mask = (rng.random((n_qb, n_kb)) < 0.6).astype(np.int32)
        queries = []
        for _ in range(24):
            partial = int(rng.random() < 0.5)
            if rng.random() < 0.5:
                queries.append(("r", int(rng.integers(0, n_q + 20)), 64 * int(rng.integers(0, -(-n_kv // 64))), partial))
            else:
                queries.append(("c", int(rng.integers(0, n_kv + 20)), 64 * int(rng.integers(0, -(-n_q // 64))), partial))
        yield (n_q, n_kv, causal, sink, window, bm, bn, mask, queries)


def _expected(case, query):
    n_q, n_kv, causal, sink, window, bm, bn, mask, _ = case
    kind, a, b, partial = query
    tok = so.token_mask(n_q, n_kv, sink, window) if causal else np.ones((n_q, n_kv), bool)
    ref = so.effective_mask(mask, n_q, n_kv, bm, bn, causal, sink, window) if partial else tok
    bits = 0
    for j in range(64):
        q, k = (a, b + j) if kind == "r" else (b + j, a)
        if q < n_q and k < n_kv and ref[q, k]:
            bits |= 1 << j
    return bits


def test_visibility_words_match_the_oracle(mask_bits_exe):
    cases = list(_cases(seed=11, n_geoms=120))
    lines = []
    for n_q, n_kv, causal, sink, window, bm, bn, mask, queries in cases:
        lines.append(f"G {n_q} {n_kv} {int(causal)} {sink} {window} {bm} {bn} {len(queries)}")
        lines.append(" ".join(str(int(x)) for x in mask.ravel()))
        lines += [f"{k} {a} {b} {p}" for k, a, b, p in queries]
    out = subprocess.run([mask_bits_exe], input="\n".join(lines) + "\n", capture_output=True,
                         text=True, check=True, timeout=120).stdout.split()
    got = iter(int(w, 16) for w in out)
    n = 0
    for case in cases:
        for query in case[-1]:
            want = _expected(case, query)
            word = next(got)
            assert word == want, (case[:7], query, f"{word:016x} != {want:016x}")
            n += 1
    assert n == sum(len(c[-1]) for c in cases)


def test_a_planted_mistake_in_the_oracle_is_caught(mask_bits_exe):
    """The comparison has teeth: an oracle token rule with the window edge off
    by one disagrees with the kernels' words somewhere."""
    n_q = n_kv = 300
    sink, window = 4, 50
    orig = so.token_mask
    try:
        so.token_mask = lambda nq, nk, s, w: orig(nq, nk, s, w + 1)
        case = (n_q, n_kv, True, sink, window, 64, 64, so.block_mask(n_q, n_kv, sink, window, 64, 64), [])
        queries = [("r", q, k0, 0) for q in range(0, n_q, 7) for k0 in range(0, n_kv, 64)]
        inp = f"G {n_q} {n_kv} 1 {sink} {window} 64 64 {len(queries)}\n" + \
            " ".join(str(int(x)) for x in case[7].ravel()) + "\n" + \
            "\n".join(f"{k} {a} {b} {p}" for k, a, b, p in queries) + "\n"
        out = subprocess.run([mask_bits_exe], input=inp, capture_output=True, text=True, check=True,
                             timeout=60).stdout.split()
        assert any(int(w, 16) != _expected(case, q) for w, q in zip(out, queries))
    finally:
        so.token_mask = orig
