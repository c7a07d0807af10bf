#!/usr/bin/env python
"""Benchmark of the gfx950 block-sparse StreamingLLM attention on one MI355X.

Metric: kept-block TFLOP/s for forward / backward and decode-step
KV GB/s, each as a fraction of the MI355X roofline.

* ``value`` -- config 2 (``configs[1]``): prefill forward, B1 H32 N16384 D128
  bf16, S4 W2048, 64x64 blocks, causal. One step = one forward call.
  Kept-block flops = 4 * 64 * 64 * 128 per kept tile per (b, h).
* ``train``  -- config 3: fwd + bwd, B4 H16 N8192 D64 fp16, S4 W1024
  (fwd 4*BM*BN*D, bwd 10*BM*BN*D per kept tile).
* ``decode`` -- config 4: B8 H32, one query, KV 100000, D128 bf16, S4 W2048;
  token-exact kept K/V bytes (S+W)*D*2*2 per (b, h) over the step time; also
  with the memory-side cache evicted, beside a plain read of exactly the same
  rows (``read_ceiling``), and the grouped-query / multi-query /
  four-position variants of the step.
* ``layer_c5`` -- one config-5 attention layer (1x16x131072x64 bf16, S4 W4096,
  128x64 blocks), fwd + bwd.
* ``cpu_baseline`` -- the reference's eager masked attention (restated in
  ``oracle/eager_cpu.py``) in fp32 on the host cores (thread count and CPU
  model recorded), on bounded samples of the same inputs: config 2 forward
  (``value``, same unit as the headline), config 3 forward + backward and
  config 4 decode (whole (b, h) slices until each leg's share of ~24 s).

Inputs are synthetic N(0, 1) (config 2 scaled by 0.5), generated once and
resident in HBM before the timed region. Each section first runs its step
untimed for --warmup calls and at least WARM_SECONDS of wall time (the GPU's
clocks ramp up under sustained load), then times. Kernel durations come from
HIP events recorded on the stream the kernels run on (torch's current stream).
Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Optional

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "graph-kernel-injection_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "kept-block TFLOP/s fwd/bwd + decode-step KV GB/s as % of MI355X roofline"
PEAK_MFMA_16 = 2500.0   # TFLOP/s, dense bf16/fp16 MFMA
PEAK_HBM = 8000.0       # GB/s


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _randn(shape, gen, scale, dtype, device):
    import torch

    return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(dtype).to(device)


# The MI355X ramps its clocks over the first few hundred ms of sustained work:
# steps timed right after a cold start run up to ~15% slow. Every section keeps
# calling its step (untimed) until this much wall time has passed.
WARM_SECONDS = 1.0


def _warm(fn, warmup: int) -> None:
    """``warmup`` untimed calls, then more until WARM_SECONDS have passed."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def _time_calls(fn, steps: int, warmup: int):
    """Warm up, then time ``steps`` back-to-back calls between one pair of HIP
    events (the throughput a caller's loop sees, launch gaps included), then a
    second pass with events around every call for the per-call distribution.
    Returns (ms per step from the first pass, per-call ms list)."""
    import torch

    _warm(fn, warmup)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    per_step = t0.elapsed_time(t1) / steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return per_step, [a.elapsed_time(b) for a, b in evs]


def _time_fwd_bwd(fwd, step, steps: int, warmup: int):
    """Forward and backward time of a training step, each as back-to-back
    work between one pair of HIP events: ``steps`` forwards (``fwd``, its
    output dropped), then ``steps`` full steps (``step``: forward, backward);
    backward = step - forward. An event recorded between the two phases of
    every step would put a queue drain (~10-30 us on this stack) inside each
    phase. Returns (fwd ms, bwd ms, step ms, host wall ms per step)."""
    import torch

    _warm(step, warmup)

    def loop(fn):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps, (time.perf_counter() - w0) * 1e3 / steps

    fwd_ms, _ = loop(fwd)
    step_ms, wall = loop(step)
    return fwd_ms, step_ms - fwd_ms, step_ms, wall


TRAIN_TIMING = ("back-to-back between one pair of HIP events: fwd = --steps forwards, "
                "step = --steps fwd+bwd steps, bwd = step - fwd")


def _time_cold(fn, calls: int = 40):
    """Per-call time of ``fn`` with the device's last-level (Infinity) cache
    evicted first: a 2 GiB read runs before each timed call (outside its
    events, so the call is queued behind it and no host gap is timed). Back-to-
    back decode steps re-read the same rows, which a 256 MB memory-side cache
    can partly hold; this is the same step with HBM serving all of them.
    Returns the median ms per call."""
    import torch

    flush = torch.empty(2 << 30, dtype=torch.uint8, device="cuda:0").view(torch.int64)
    times = []
    for _ in range(calls):
        flush.sum()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    del flush
    return statistics.median(times)


def _traffic(*keys: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled
    by a plain copy of known size), summed over the named kernels; from
    profiles/hbm_traffic.json, which the profiling commands in
    profiles/hbm_traffic_c2_c3_c4_c5.md produce. None when not profiled."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    try:
        table = json.loads(path.read_text())["kernels"]
        return int(sum(table[k]["hbm_bytes"] for k in keys))
    except (OSError, KeyError, ValueError):
        return None


def _roofline(achieved: float, peak: float, unit: str, bound: str, traffic=None) -> dict:
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def section_c2(steps: int, warmup: int, keep_cpu_inputs: bool):
    import torch

    import sparse_triton_kernel as stk

    B, H, N, D, S, W, bm = 1, 32, 16384, 128, 4, 2048, 64
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    q32, k32, v32 = (torch.randn(B, H, N, D, generator=g) * 0.5 for _ in range(3))
    q, k, v = (t.to(torch.bfloat16).to(dev) for t in (q32, k32, v32))
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=dev)
    kept = int(mask.sum().item())
    flops = 4.0 * bm * bm * D * kept * B * H

    def fn():
        return stk.block_sparse_attention(q, k, v, mask, block_m=bm, block_n=bm, is_causal=True,
                                          sink_size=S, window_size=W)

    avg, per = _time_calls(fn, steps, warmup)
    tflops = flops / (avg * 1e-3) / 1e12
    log(f"[c2] fwd step {avg:.4f} ms back-to-back (per call p50 {statistics.median(per):.4f}), "
        f"{tflops:.1f} TFLOP/s")
    cpu_inputs = None
    if keep_cpu_inputs:
        cpu_inputs = tuple(t.to(torch.bfloat16).float() for t in (q32, k32, v32)) + (mask.cpu(),)
    del q, k, v
    return {
        "kept_tiles": kept, "flops_per_step": flops, "avg_ms": avg, "p50_ms": statistics.median(per),
        "ms_per_step": avg, "tflops": tflops,
    }, cpu_inputs


def section_c3(steps: int, warmup: int, cpu_sample: Optional[dict] = None) -> dict:
    import torch

    import sparse_triton_kernel as stk

    B, H, N, D, S, W, bm = 4, 16, 8192, 64, 4, 1024, 64
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(2)
    q, k, v, do = (_randn((B, H, N, D), g, 1.0, torch.float16, dev) for _ in range(4))
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bm, device=dev)
    kept = int(mask.sum().item())
    f_fwd = 4.0 * bm * bm * D * kept * B * H
    f_bwd = 10.0 * bm * bm * D * kept * B * H

    def forward():
        return stk.block_sparse_attention(q, k, v, mask, is_causal=True, sink_size=S, window_size=W)

    def step():
        for t in (q, k, v):
            t.grad = None
        forward().backward(do)

    fwd, bwd, step_ms, wall = _time_fwd_bwd(forward, step, steps, warmup)
    res = {
        "workload": "c3 training fwd+bwd: B4 H16 N8192 D64 fp16, S4 W1024, 64x64 blocks, causal",
        "kept_tiles": kept, "fwd_ms": fwd, "bwd_ms": bwd, "ms_per_step": step_ms,
        "host_wall_ms_per_step": wall, "timing": TRAIN_TIMING,
        "fwd_tflops": f_fwd / (fwd * 1e-3) / 1e12, "bwd_tflops": f_bwd / (bwd * 1e-3) / 1e12,
        "fwdbwd_tflops": (f_fwd + f_bwd) / ((fwd + bwd) * 1e-3) / 1e12,
    }
    res["roofline"] = _roofline(res["fwdbwd_tflops"], PEAK_MFMA_16, "TFLOP/s", "mfma",
                                _traffic("c3_fwd", "c3_dkdv", "c3_dq"))
    log(f"[c3] fwd {fwd:.4f} ms ({res['fwd_tflops']:.1f} TF/s), bwd {bwd:.4f} ms "
        f"({res['bwd_tflops']:.1f} TF/s)")
    if cpu_sample is not None:
        cpu_sample["c3"] = tuple(t.detach().cpu() for t in (q, k, v, do)) + (mask.cpu(), kept)
    return res


def section_c4(steps: int, warmup: int, cpu_sample: Optional[dict] = None) -> dict:
    import torch

    import sparse_triton_kernel as stk

    from benchmark import seeded_normal

    B, H, NKV, D, S, W = 8, 32, 100000, 128, 4, 2048
    dev = torch.device("cuda:0")
    q, k, v = seeded_normal([(B, H, 1, D), (B, H, NKV, D), (B, H, NKV, D)], 3, torch.bfloat16, dev,
                            workers=cpu_threads())
    mask = stk.make_streaming_mask(1, NKV, stk.StreamingMaskSpec(S, W), 1, 64, device=dev)
    kept = int(mask.sum().item())
    exact_bytes = (S + W) * D * 2 * 2 * B * H
    block_bytes = block_granular_tokens(mask[0].cpu(), NKV, 64) * D * 2 * 2 * B * H

    def fn():
        return stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                          sink_size=S, window_size=W)

    avg, per = _time_calls(fn, steps, warmup)
    gbs = exact_bytes / (avg * 1e-3) / 1e9
    res = {
        "workload": "c4 decode step: B8 H32 n_q=1 KV100000 D128 bf16, S4 W2048, BM=1 BN=64",
        "kept_tiles": kept, "kv_bytes_token_exact": exact_bytes, "kv_bytes_block_granular": block_bytes,
        "avg_ms": avg, "p50_ms": statistics.median(per), "ms_per_step": avg,
        "kv_gbs": gbs, "kv_gbs_block_granular": block_bytes / (avg * 1e-3) / 1e9,
    }
    res["roofline"] = _roofline(gbs, PEAK_HBM, "GB/s", "hbm", _traffic("c4_decode"))
    log(f"[c4] decode step {avg * 1e3:.2f} us, {gbs:.0f} GB/s token-exact "
        f"({100 * gbs / PEAK_HBM:.1f}% of HBM peak)")
    cold = _time_cold(fn)
    res["cold_cache"] = {"per_call_ms": cold, "kv_gbs": exact_bytes / (cold * 1e-3) / 1e9,
                         "frac": exact_bytes / (cold * 1e-3) / 1e9 / PEAK_HBM,
                         "protocol": "median of 40 calls, each after a 2 GiB read that evicts "
                                     "the 256 MB memory-side cache"}
    log(f"[c4] decode step after evicting the memory-side cache: {cold * 1e3:.2f} us, "
        f"{res['cold_cache']['kv_gbs']:.0f} GB/s ({100 * res['cold_cache']['frac']:.1f}% of HBM peak)")
    res["rolling_cache"] = _rolling_c4(q, k, v, S, W, fn(), exact_bytes, steps, warmup)
    res["read_ceiling"] = _read_ceiling_c4(k, v, S, W, exact_bytes, avg, cold, steps, warmup)
    if cpu_sample is not None:      # the whole step for the CPU leg (13 GB of bf16 K / V on the host)
        cpu_sample["c4"] = (q.cpu(), k.cpu(), v.cpu(), mask.cpu())
    del k, v
    res["gqa"] = _gqa_c4(B, H, NKV, D, S, W, mask, steps, warmup)
    res["multi_query"] = _gqa_c4(B, H, NKV, D, S, W, mask, steps, warmup, H_kv=1)
    res["four_positions"] = _gqa_c4(B, H, NKV, D, S, W, mask, steps, warmup, H_kv=H, n_q=4)
    return res


def _read_probe(k, v, S, W):
    """A call of ``gki_read_probe`` over the rows a one-position decode step
    reads from K / V ``[B, H_kv, n_kv, D]``: the sink rows and window rows of
    every (b, kv head) slice."""
    import torch

    from gki import _lib

    lib = _lib.load()
    B, H, NKV, D = k.shape
    bh = B * H
    words = int(lib.gki_read_probe_words(bh))
    out = torch.empty(words, dtype=torch.int32, device=k.device)
    row_bytes = D * k.element_size()

    def fn():
        stream = torch.cuda.current_stream(k.device).cuda_stream
        _lib.check(lib.gki_read_probe(k.data_ptr(), v.data_ptr(), bh, NKV, row_bytes, S, W, out.data_ptr(),
                                      words, stream), "gki_read_probe")

    return fn


def _read_ceiling_c4(k, v, S, W, exact_bytes, decode_ms, decode_cold_ms, steps, warmup) -> dict:
    """The read ceiling of the c4 step's own access pattern: ``gki_read_probe``
    streams exactly its token-exact K / V rows (the sink rows and the window
    rows of every (b, h) slice) with 16-byte non-temporal loads and no other
    work, timed like the step: back to back, and after the 2 GiB read that
    evicts the memory-side cache. ``decode_share`` = probe time / step time."""
    fn = _read_probe(k, v, S, W)
    avg, _ = _time_calls(fn, steps, warmup)
    cold = _time_cold(fn)
    res = {"protocol": "gki_read_probe over the same token-exact rows (8 chunks x 256 threads x 4 "
                       "non-temporal 16-byte loads per window, one workgroup for the sink rows); "
                       "warm: back-to-back calls; cold: as decode.cold_cache",
           "warm_ms": avg, "cold_ms": cold,
           "warm_frac_of_hbm": exact_bytes / (avg * 1e-3) / 1e9 / PEAK_HBM,
           "cold_frac_of_hbm": exact_bytes / (cold * 1e-3) / 1e9 / PEAK_HBM,
           "decode_share_warm": avg / decode_ms, "decode_share_cold": cold / decode_cold_ms}
    log(f"[c4] read ceiling of the step's rows: {avg * 1e3:.2f} us warm ({100 * res['warm_frac_of_hbm']:.1f}% "
        f"of HBM peak), {cold * 1e3:.2f} us cold ({100 * res['cold_frac_of_hbm']:.1f}%); the decode step "
        f"reaches {100 * res['decode_share_warm']:.1f}% / {100 * res['decode_share_cold']:.1f}% of it")
    return res


def _gqa_c4(B, H, NKV, D, S, W, mask, steps, warmup, H_kv=8, n_q=1) -> dict:
    """The c4 step with grouped-query K/V (default: 8 kv heads for the 32 q
    heads) and / or n_q query positions: a K/V stream's group x n_q query rows
    are served by one workgroup (on the matrix cores for 2..32 rows), so the
    token-exact K/V bytes are H_kv / H of c4's (positions visible to any row)."""
    import torch

    import sparse_triton_kernel as stk

    from benchmark import seeded_normal

    dev = torch.device("cuda:0")
    q, k, v = seeded_normal([(B, H, n_q, D), (B, H_kv, NKV, D), (B, H_kv, NKV, D)], 5, torch.bfloat16,
                            dev, workers=cpu_threads())
    if n_q != 1:
        mask = stk.make_streaming_mask(n_q, NKV, stk.StreamingMaskSpec(S, W), 1, 64, device=dev)

    def fn():
        return stk.block_sparse_attention(q, k, v, mask, block_m=1, block_n=64, is_causal=True,
                                          sink_size=S, window_size=W, enable_gqa=H_kv != H)

    avg, per = _time_calls(fn, steps, warmup)
    kv_bytes = (S + W + n_q - 1) * D * 2 * 2 * B * H_kv
    gbs = kv_bytes / (avg * 1e-3) / 1e9
    res = {"workload": f"c4 with H {H}, H_kv {H_kv}, n_q {n_q}", "kv_bytes_token_exact": kv_bytes,
           "avg_ms": avg, "p50_ms": statistics.median(per), "kv_gbs": gbs}
    extra = ""
    if n_q == 1:      # the plain read of the same rows, back to back (decode.read_ceiling's probe)
        probe, _ = _time_calls(_read_probe(k, v, S, W), steps, warmup)
        res["read_ceiling_ms"], res["decode_share"] = probe, probe / avg
        extra = f"; a plain read of its rows takes {probe * 1e3:.2f} us ({100 * probe / avg:.0f}% of the step)"
    log(f"[c4] H{H}/H_kv{H_kv} n_q {n_q}: decode step {avg * 1e3:.2f} us, {gbs:.0f} GB/s token-exact "
        f"({kv_bytes / 1e6:.0f} MB of K/V){extra}")
    return res


def _rolling_c4(q, k, v, S, W, o_full, exact_bytes, steps, warmup) -> dict:
    """The same decode from a rolling (sink + ring) cache holding only the
    positions a query can still see: decode alone, and a full step (append the
    new token's K/V, then decode)."""
    import torch

    from gki.kv_cache import StreamingKVCache
    from sparse_triton_kernel import StreamingMaskSpec

    B, H, NKV, D = k.shape
    cache = StreamingKVCache(B, H, D, StreamingMaskSpec(S, W), k.dtype, k.device, max_query=1)
    cache.append(k[:, :, :-1], v[:, :, :-1])
    o_roll = cache.step(q, k[:, :, -1:], v[:, :, -1:])
    identical = bool(torch.equal(o_roll, o_full))
    avg, per = _time_calls(lambda: cache.attend(q), steps, warmup)
    k1, v1 = k[:, :, -1:].contiguous(), v[:, :, -1:].contiguous()
    step_avg, _ = _time_calls(lambda: cache.step(q, k1, v1), steps, warmup)
    gbs = exact_bytes / (avg * 1e-3) / 1e9
    cold = _time_cold(lambda: cache.attend(q))
    cache_bytes = 2 * cache.k_cache.numel() * cache.k_cache.element_size()
    log(f"[c4] rolling cache ({cache.capacity} slots, {cache_bytes / 1e6:.0f} MB vs "
        f"{2 * k.numel() * k.element_size() / 1e9:.2f} GB full): decode {avg * 1e3:.2f} us "
        f"({gbs:.0f} GB/s), append+decode step {step_avg * 1e3:.2f} us, "
        f"bit-identical to the full-cache decode: {identical}; memory-side cache evicted: "
        f"{cold * 1e3:.2f} us ({100 * exact_bytes / (cold * 1e-3) / 1e9 / PEAK_HBM:.1f}% of HBM peak)")
    return {"slots": cache.capacity, "cache_bytes": cache_bytes,
            "full_cache_bytes": 2 * k.numel() * k.element_size(), "decode_ms": avg,
            "decode_p50_ms": statistics.median(per), "kv_gbs": gbs, "step_ms": step_avg,
            "identical_to_full_cache": identical,
            "cold_cache": {"per_call_ms": cold, "kv_gbs": exact_bytes / (cold * 1e-3) / 1e9,
                           "frac": exact_bytes / (cold * 1e-3) / 1e9 / PEAK_HBM}}


def section_c5(steps: int, warmup: int) -> dict:
    import torch

    import sparse_triton_kernel as stk

    from benchmark import seeded_normal

    B, H, N, D, S, W, bm, bn = 1, 16, 131072, 64, 4, 4096, 128, 64
    dev = torch.device("cuda:0")
    q, k, v, do = seeded_normal([(B, H, N, D)] * 4, 4, torch.bfloat16, dev, workers=cpu_threads())
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    mask = stk.make_streaming_mask(N, N, stk.StreamingMaskSpec(S, W), bm, bn, device=dev)
    kept = int(mask.sum().item())
    f_fwd = 4.0 * bm * bn * D * kept * B * H
    f_bwd = 10.0 * bm * bn * D * kept * B * H

    def forward():
        return stk.block_sparse_attention(q, k, v, mask, block_m=bm, block_n=bn, is_causal=True,
                                          sink_size=S, window_size=W)

    def step():
        for t in (q, k, v):
            t.grad = None
        forward().backward(do)

    fwd, bwd, step_ms, wall = _time_fwd_bwd(forward, step, steps, warmup)
    res = {
        "workload": "c5 attention layer fwd+bwd: B1 H16 N131072 D64 bf16, S4 W4096, 128x64 blocks",
        "kept_tiles": kept, "fwd_ms": fwd, "bwd_ms": bwd, "ms_per_step": step_ms,
        "host_wall_ms_per_step": wall, "timing": TRAIN_TIMING,
        "fwd_tflops": f_fwd / (fwd * 1e-3) / 1e12, "bwd_tflops": f_bwd / (bwd * 1e-3) / 1e12,
        "fwdbwd_tflops": (f_fwd + f_bwd) / ((fwd + bwd) * 1e-3) / 1e12,
        "attention_ms_12_layers": 12 * (fwd + bwd),
    }
    res["roofline"] = _roofline(res["fwdbwd_tflops"], PEAK_MFMA_16, "TFLOP/s", "mfma",
                                _traffic("c5_fwd", "c5_dkdv", "c5_dq"))
    log(f"[c5] layer fwd {fwd:.3f} ms, bwd {bwd:.3f} ms ({res['fwdbwd_tflops']:.1f} TF/s)")
    return res


def block_granular_tokens(kept_row, n_kv: int, bn: int) -> int:
    """In-bounds tokens of the kept tiles of a one-row block mask: bn per kept
    tile, the ragged last tile only its n_kv - bn * j in-range tokens (c4: 33
    full tiles + 32 tokens of tile 1562 = 2144 tokens)."""
    cols = [j for j, x in enumerate(kept_row.tolist()) if x]
    return sum(min(bn, n_kv - bn * j) for j in cols)


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the GPU box
    allots each GPU a share of its cores and says so there)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _heads_within(budget_s: float, n_heads: int, one_head) -> tuple:
    """Run one_head(i) for i = 0, 1, ... until the budget is spent (at least
    once, at most n_heads times); returns (heads done, seconds)."""
    heads = 0
    t0 = time.perf_counter()
    while heads < n_heads:
        one_head(heads)
        heads += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return heads, time.perf_counter() - t0


def cpu_baseline(cpu_inputs, kept: int, budget_s: float, extra: Optional[dict] = None) -> dict:
    """The reference's eager path (sparse_triton_kernel.py:845-902, restated in
    oracle/eager_cpu.py) in fp32 on the host cores, on bounded samples of the
    same inputs the GPU sections used (whole (b, h) slices until each leg's
    share of the budget is spent; sums over slices, extrapolation stated):
    config 2 forward (``value``, kept-block TFLOP/s), and from ``extra``
    config 3 forward + backward (autograd; 14 * BM * BN * D per kept tile)
    and the config 4 decode step (token-exact kept K/V GB/s); config 1
    forward + backward runs directly (no GPU input needed)."""
    import torch

    from oracle.eager_cpu import eager_masked_attention

    threads = cpu_threads()
    torch.set_num_threads(threads)
    extra = extra or {}
    legs = 1 + ("c3" in extra) + ("c4" in extra)
    share = budget_s / legs

    q, k, v, mask = cpu_inputs
    H, D = q.shape[1], q.shape[-1]

    def c2_head(h):
        sl = slice(h, h + 1)
        eager_masked_attention(q[:, sl], k[:, sl], v[:, sl], mask, 64, 64, True, 4, 2048)

    heads, elapsed = _heads_within(share, H, c2_head)
    tflops = 4.0 * 64 * 64 * D * kept * heads / elapsed / 1e12
    log(f"[cpu] eager fp32 on {threads} threads: c2 {heads} head(s) in {elapsed:.1f} s, "
        f"{tflops * 1e3:.2f} GFLOP/s kept-block")
    out = {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
           "sample": (f"config 2 forward, {heads} of {H} heads (B1 N16384 D128, fp32 eager "
                      f"masked attention over all keys, 2048-row chunks), {elapsed:.1f} s; "
                      f"full-step extrapolation {elapsed * H / heads:.1f} s")}

    if "c3" in extra:
        q3, k3, v3, do3, m3, kept3 = extra["c3"]
        B3, H3, N3, D3 = q3.shape

        def c3_head(i):
            b, h = divmod(i, H3)
            sl = (slice(b, b + 1), slice(h, h + 1))
            leaves = [t[sl].float().requires_grad_(True) for t in (q3, k3, v3)]
            o = eager_masked_attention(*leaves, m3, 64, 64, True, 4, 1024)
            o.backward(do3[sl].float())

        n3, t3 = _heads_within(share, B3 * H3, c3_head)
        f3 = 14.0 * 64 * 64 * D3 * kept3 * n3
        out["c3"] = {"value": round(f3 / t3 / 1e12, 6), "unit": "TFLOP/s",
                     "sample": (f"config 3 forward + backward (autograd), {n3} of {B3 * H3} (b, h) "
                                f"slices (N8192 D64), {t3:.1f} s; full-step extrapolation "
                                f"{t3 * B3 * H3 / n3:.1f} s")}
        log(f"[cpu] c3 fwd+bwd: {n3} (b, h) slice(s) in {t3:.1f} s, "
            f"{out['c3']['value'] * 1e3:.2f} GFLOP/s kept-block")

    if "c4" in extra:
        q4, k4, v4, m4 = extra["c4"]
        B4, H4, D4 = q4.shape[0], q4.shape[1], q4.shape[-1]

        def c4_head(i):
            sl = (slice(i // H4, i // H4 + 1), slice(i % H4, i % H4 + 1))
            eager_masked_attention(q4[sl].float(), k4[sl].float(), v4[sl].float(), m4, 1, 64, True,
                                   4, 2048)

        n4, t4 = _heads_within(max(share, 60.0), B4 * H4, c4_head)
        kv = (4 + 2048) * D4 * 2 * 2 * n4
        out["c4"] = {"value": round(kv / t4 / 1e9, 4), "unit": "GB/s",
                     "sample": (f"config 4 decode step, {n4} of {B4 * H4} (b, h) slices (n_q 1, KV "
                                f"100000, D128, bf16 cast to fp32 per slice; the eager path reads "
                                f"all 100000 keys), {t4:.2f} s; token-exact kept K/V bytes {kv} "
                                f"over that time")}
        log(f"[cpu] c4 decode: {n4} (b, h) slice(s) in {t4:.2f} s, {out['c4']['value']:.3f} GB/s")

    out["c5"] = {"value": None, "unit": "TFLOP/s",
                 "sample": ("not run: the eager path computes all 131072 x 131072 scores of each of "
                            "a config-5 layer's 16 heads (1.1 TB of fp32 scores; chunked, one head's "
                            "forward is 4.4 TFLOP, minutes of CPU time at the rates above)")}
    # config 1 runs directly: B1 H4 N1024 D64 fp32 (seed 0), forward + backward
    g1 = torch.Generator().manual_seed(0)
    q1, k1, v1 = (torch.randn(1, 4, 1024, 64, generator=g1).requires_grad_(True) for _ in range(3))
    do1 = torch.randn(1, 4, 1024, 64, generator=torch.Generator().manual_seed(1))
    from oracle import streaming_oracle as so
    m1 = torch.from_numpy(so.block_mask(1024, 1024, 4, 256, 64, 64))

    def c1_step(_):
        for t in (q1, k1, v1):
            t.grad = None
        eager_masked_attention(q1, k1, v1, m1, 64, 64, True, 4, 256).backward(do1)

    n1, t1 = _heads_within(min(share, 2.0), 1 << 30, c1_step)
    f1 = 14.0 * 64 * 64 * 64 * int(m1.sum()) * 4 * n1
    out["c1"] = {"value": round(f1 / t1 / 1e12, 6), "unit": "TFLOP/s", "ms_per_step": 1e3 * t1 / n1,
                 "sample": (f"config 1 forward + backward (B1 H4 N1024 D64 fp32, S4 W256), {n1} "
                            f"steps in {t1:.2f} s")}
    log(f"[cpu] c1 fwd+bwd: {1e3 * t1 / n1:.2f} ms per step")
    return out


def copy_calibration() -> None:
    """A plain 1 GiB device-to-device copy, three times: the known-size job that
    FETCH_SIZE / WRITE_SIZE are scaled against (rocprofv3 --pmc)."""
    import torch

    n = 1 << 29                                   # bf16 elements: 1 GiB
    a = torch.empty(n, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"[copy] copied {a.numel() * 2} bytes x3")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sections", default="c2,c3,c4,c5,cpu",
                    help="comma list among c2,c3,c4,c5,cpu (c2 is always run)")
    ap.add_argument("--cpu-budget", type=float, default=24.0,
                    help="seconds of CPU baseline work, shared by its c2 / c3 / c4 legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration), print nothing on stdout")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
              "(the op has no multi-GPU path in this build).", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (none visible)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration()
        return 0
    sections = set(s.strip() for s in args.sections.split(","))
    c2, cpu_in = section_c2(args.steps, args.warmup, "cpu" in sections)
    line = {
        "metric": METRIC,
        "value": round(c2["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: Q/K/V ~ N(0,1)*0.5 from a seed-1 CPU generator (no dataset)",
        "config": {
            "workload": "c2 prefill forward: B1 H32 N16384 D128 bf16, StreamingLLM S4 W2048, "
                        "64x64 blocks, causal",
            "kept_tiles": c2["kept_tiles"], "flops_per_step": c2["flops_per_step"],
            "kernel_avg_ms": round(c2["avg_ms"], 5), "kernel_p50_ms": round(c2["p50_ms"], 5),
        },
        "roofline": _roofline(c2["tflops"], PEAK_MFMA_16, "TFLOP/s", "mfma", _traffic("c2_fwd")),
    }
    torch.cuda.empty_cache()
    cpu_extra = {} if "cpu" in sections else None
    if "c3" in sections:
        line["train"] = section_c3(args.steps, args.warmup, cpu_extra)
        torch.cuda.empty_cache()
    if "c4" in sections:
        # a decode step is ~45 us: time more of them for a stable mean
        line["decode"] = section_c4(max(args.steps, 200), max(args.warmup, 20), cpu_extra)
        torch.cuda.empty_cache()
    if "c5" in sections:
        line["layer_c5"] = section_c5(max(3, args.steps // 4), 2)
        torch.cuda.empty_cache()
    if "cpu" in sections:
        line["cpu_baseline"] = cpu_baseline(cpu_in, c2["kept_tiles"], args.cpu_budget, cpu_extra)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
