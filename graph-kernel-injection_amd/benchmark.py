"""Comparative baselines on one MI355X: this build's kernels vs FlexAttention / SDPA.

Drop-in for the comparison part of the reference's harness (``benchmark.py``:
``HarnessConfig`` :81-97, method factories :512-628, measurement :428-492,
fp64 error at a scaled-down shape :633-680) and its fairness protocol
(``docs/eval_plan.md`` §5: win / tie / loss against FlexAttention). Same
methods, same mask semantics (bottom-right aligned StreamingLLM token rule),
same p50 / p95 per-iteration HIP-event timing and peak-VRAM accounting, same
CLI flags. Deviations, each for fairness on this hardware:

* FlexAttention runs compiled (``torch.compile(flex_attention)``), its intended
  mode; the reference calls the eager function, torch's unfused fallback.
* Every method is first called for ~1 s untimed: the GPU ramps its clocks over
  the first few hundred ms, which would bias whichever method runs first.
* K/V for all methods share one tensor set per mode (as the reference does).

Usage (from ``graph-kernel-injection_amd/``)::

    python benchmark.py bench --seq-q 16384 --seq-len 16384 --heads 32 \\
        --head-dim 128 --dtype bf16 --window 2048          # c2 prefill
    python benchmark.py bench                               # reference default: decode, 131072 keys
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import csv
import dataclasses
import hashlib
import math
import statistics
import sys
import threading
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F  # noqa: N812

from sparse_triton_kernel import (
    StreamingMaskSpec,
    block_sparse_attention,
    make_streaming_mask,
    reference_block_sparse_attention,
    streaming_token_mask,
)

try:
    from torch.nn.attention.flex_attention import create_block_mask as _flex_create_block_mask
    from torch.nn.attention.flex_attention import flex_attention as _flex_attention

    _FLEX_AVAILABLE = True
except ImportError:  # pragma: no cover
    _FLEX_AVAILABLE = False

OURS = "gki-block-sparse"
WARM_SECONDS = 1.0
# eager-dense materialises B*H*N_Q*N_KV fp32 scores: skip it above this many
EAGER_MAX_SCORES = 1 << 28


@dataclass
class HarnessConfig:
    batch: int = 1
    heads: int = 8
    seq_len_q: int = 1
    seq_len_kv: int = 131_072
    head_dim: int = 64
    block_m: int = 64
    block_n: int = 64
    sink_size: int = 4
    window_size: int = 2_048
    device: str = "cuda"
    dtype: torch.dtype = torch.float16
    warmup_iters: int = 25
    measure_iters: int = 100


@dataclass
class BenchResult:
    label: str
    dtype: str
    seq_len_kv: int
    density: float
    fwd_p50_ms: float
    fwd_p95_ms: float
    fwdbwd_p50_ms: Optional[float]
    fwdbwd_p95_ms: Optional[float]
    peak_vram_mib: float
    max_abs_err_vs_fp64: Optional[float]

    def row(self) -> List[str]:
        opt = lambda x, f: "n/a" if x is None else format(x, f)  # noqa: E731
        return [self.label, self.dtype, str(self.seq_len_kv), f"{self.density:.4f}",
                f"{self.fwd_p50_ms:.3f}", f"{self.fwd_p95_ms:.3f}", opt(self.fwdbwd_p50_ms, ".3f"),
                opt(self.fwdbwd_p95_ms, ".3f"), f"{self.peak_vram_mib:.1f}",
                opt(self.max_abs_err_vs_fp64, ".2e")]


HEADERS = ("label", "dtype", "seq_kv", "mask_density", "fwd_p50_ms", "fwd_p95_ms",
           "fwdbwd_p50_ms", "fwdbwd_p95_ms", "peak_vram_MiB", "max_abs_err_vs_fp64")


def percentile(values: Sequence[float], q: float) -> float:
    """Linear-interpolation percentile (the reference's :428-437)."""
    s = sorted(values)
    k = (len(s) - 1) * (q / 100.0)
    lo, hi = math.floor(k), math.ceil(k)
    return s[lo] if lo == hi else s[lo] + (s[hi] - s[lo]) * (k - lo)


# Elements per chunk of seeded_normal: each chunk has its own CPU generator.
SEED_CHUNK = 1 << 24


def _chunk_seed(seed: int, tensor: int, chunk: int) -> int:
    return int.from_bytes(hashlib.blake2b(f"{seed}/{tensor}/{chunk}".encode(), digest_size=8).digest(),
                          "little") >> 1


def seeded_normal(shapes: Sequence[Sequence[int]], seed: int, dtype: torch.dtype,
                  device, scale: float = 1.0, workers: int = 16) -> List[torch.Tensor]:
    """Tensors of N(0, scale^2) values (drawn in fp32, scaled, then rounded to
    ``dtype``) generated on the CPU and moved to ``device``: the same bits on
    every host and GPU, as a CPU ``torch.Generator`` seeded per config gives
    (the protocol of SURVEY's measurement plan; the reference draws q, k, v in
    order from one generator, benchmark.py:128-133). Tensor t's elements come
    in chunks of SEED_CHUNK, chunk c from a generator seeded by a hash of
    (seed, t, c), so the draw of a decode step's 6.5e9 K / V values runs on
    ``workers`` threads instead of one generator's ~40 s."""
    flats = [torch.empty(math.prod(s), dtype=dtype) for s in shapes]
    jobs = [(t, a) for t, f in enumerate(flats) for a in range(0, f.numel(), SEED_CHUNK)]
    local = threading.local()

    def draw(job):
        t, a = job
        n = min(SEED_CHUNK, flats[t].numel() - a)
        if not hasattr(local, "buf"):     # one fp32 chunk buffer per thread
            local.buf = torch.empty(SEED_CHUNK, dtype=torch.float32)
        g = torch.Generator().manual_seed(_chunk_seed(seed, t, a // SEED_CHUNK))
        x = torch.randn(n, generator=g, dtype=torch.float32, out=local.buf[:n])
        if scale != 1.0:
            x.mul_(scale)
        flats[t][a:a + n].copy_(x)

    intra = torch.get_num_threads()
    torch.set_num_threads(1)     # one thread per chunk; no nested intra-op pools
    try:
        with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
            list(pool.map(draw, jobs))
    finally:
        torch.set_num_threads(intra)
    return [f.view(*s).to(device) for f, s in zip(flats, shapes)]


def _make_qkv(cfg: HarnessConfig, dtype: torch.dtype, requires_grad: bool = False):
    g = torch.Generator(device=cfg.device).manual_seed(0)
    sq = (cfg.batch, cfg.heads, cfg.seq_len_q, cfg.head_dim)
    skv = (cfg.batch, cfg.heads, cfg.seq_len_kv, cfg.head_dim)
    q = torch.randn(sq, generator=g, device=cfg.device, dtype=dtype)
    k = torch.randn(skv, generator=g, device=cfg.device, dtype=dtype)
    v = torch.randn(skv, generator=g, device=cfg.device, dtype=dtype)
    for t in (q, k, v):
        t.requires_grad_(requires_grad)
    return q, k, v


def _make_mask(cfg: HarnessConfig) -> torch.Tensor:
    return make_streaming_mask(cfg.seq_len_q, cfg.seq_len_kv,
                               StreamingMaskSpec(cfg.sink_size, cfg.window_size),
                               cfg.block_m, cfg.block_n, device=cfg.device)


def _warm(fn: Callable[[], None], warmup: int) -> None:
    t0, n = time.perf_counter(), 0
    while n < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        fn()
        n += 1
    torch.cuda.synchronize()


def _time(fn: Callable[[], None], warmup: int, iters: int) -> Tuple[List[float], float]:
    _warm(fn, warmup)
    torch.cuda.reset_peak_memory_stats()
    samples = []
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(iters):
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        samples.append(a.elapsed_time(b))
    return samples, torch.cuda.max_memory_allocated() / 2**20


MethodFn = Callable[[], torch.Tensor]


def _methods(q, k, v, mask, cfg: HarnessConfig) -> Dict[str, Optional[MethodFn]]:
    scale = 1.0 / math.sqrt(cfg.head_dim)
    S, W = cfg.sink_size, cfg.window_size
    n_q, n_kv = q.shape[-2], k.shape[-2]
    out: Dict[str, Optional[MethodFn]] = {}
    out[OURS] = lambda: block_sparse_attention(q, k, v, mask, softmax_scale=scale,
                                               block_m=cfg.block_m, block_n=cfg.block_n,
                                               is_causal=True, sink_size=S, window_size=W)
    out["flex-attention"] = None
    if _FLEX_AVAILABLE:
        off = n_kv - n_q

        def mask_mod(b, h, q_idx, kv_idx):  # noqa: ARG001
            qa = q_idx + off
            return (kv_idx <= qa) & ((kv_idx < S) | (kv_idx >= qa - W + 1))

        try:
            bm = _flex_create_block_mask(mask_mod, B=None, H=None, Q_LEN=n_q, KV_LEN=n_kv,
                                         device=str(q.device))
            flex = torch.compile(_flex_attention, dynamic=False)
            out["flex-attention"] = lambda: flex(q, k, v, block_mask=bm, scale=scale)
        except Exception as e:  # noqa: BLE001
            print(f"[skip] flex-attention: {type(e).__name__}: {e}", flush=True)
    if n_q * n_kv <= 1 << 31:
        tok = streaming_token_mask(n_q, n_kv, S, W, device=q.device)
        out["sdpa-explicit-mask"] = lambda: F.scaled_dot_product_attention(q, k, v, attn_mask=tok,
                                                                           scale=scale)
    else:
        out["sdpa-explicit-mask"] = None
    # dense causal SDPA (no sparsity) needs n_q == n_kv alignment for is_causal
    out["sdpa-causal-dense"] = (lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                                       scale=scale)) \
        if n_q == n_kv else None
    if q.shape[0] * q.shape[1] * n_q * n_kv <= EAGER_MAX_SCORES:
        out["eager-dense"] = lambda: reference_block_sparse_attention(
            q, k, v, mask, softmax_scale=scale, block_m=cfg.block_m, block_n=cfg.block_n,
            is_causal=True, sink_size=S, window_size=W)
    else:
        out["eager-dense"] = None
    return out


def _error_shape(cfg: HarnessConfig) -> HarnessConfig:
    """Scaled-down shape where a dense fp64 oracle fits (the reference's :633-648)."""
    return dataclasses.replace(
        cfg, batch=1, heads=2, seq_len_q=min(max(cfg.seq_len_q, 1), 256),
        seq_len_kv=min(cfg.seq_len_kv, 256), head_dim=min(cfg.head_dim, 64),
        block_m=min(cfg.block_m, max(1, min(cfg.seq_len_q, 64))), block_n=min(cfg.block_n, 64),
        window_size=min(cfg.window_size, 128), sink_size=min(cfg.sink_size, 32))


def measure_errors(cfg: HarnessConfig) -> Dict[str, Optional[float]]:
    small = _error_shape(cfg)
    q64, k64, v64 = _make_qkv(small, torch.float64)
    mask = _make_mask(small)
    oracle = reference_block_sparse_attention(q64, k64, v64, mask, block_m=small.block_m,
                                              block_n=small.block_n, is_causal=True,
                                              sink_size=small.sink_size,
                                              window_size=small.window_size)
    q, k, v = (t.to(small.dtype) for t in (q64, k64, v64))
    errors: Dict[str, Optional[float]] = {}
    for label, fn in _methods(q, k, v, mask, small).items():
        if fn is None:
            errors[label] = None
            continue
        try:
            with torch.no_grad():
                errors[label] = float((fn().to(torch.float64) - oracle).abs().max().item())
        except Exception as e:  # noqa: BLE001
            print(f"[err] {label}: {type(e).__name__}: {e}", flush=True)
            errors[label] = None
    return errors


def failure_text(e: BaseException) -> str:
    """One line naming a failed method's exception: its first line and, for a
    wrapped error (an Inductor subprocess failure, say), the last line that
    names an error, where the underlying cause is printed (generic hints such
    as "Set TORCHDYNAMO_VERBOSE=1 ..." are skipped)."""
    lines = [ln.strip() for ln in str(e).splitlines() if ln.strip()]
    if not lines:
        return type(e).__name__
    text = lines[0][:200]
    causes = [ln for ln in lines[1:] if ("Error" in ln or "error:" in ln) and not ln.startswith("Set ")]
    if causes and causes[-1] != lines[0]:
        text += " ... " + causes[-1][:200]
    return f"{type(e).__name__}: {text}"


def verdict(ours: BenchResult, flex: Optional[BenchResult], flex_error: Optional[str] = None) -> str:
    """Win / tie / loss against FlexAttention (docs/eval_plan.md §5); without a
    FlexAttention result, "no verdict" and why (``flex_error``)."""
    if flex is None:
        return "no FlexAttention result: no verdict" + (f" ({flex_error})" if flex_error else "")
    ratio = flex.fwd_p95_ms / ours.fwd_p95_ms
    noisy = any(r.fwd_p95_ms / r.fwd_p50_ms > 2 for r in (ours, flex))
    e_o, e_f = ours.max_abs_err_vs_fp64, flex.max_abs_err_vs_fp64
    err_worse = e_o is not None and e_f is not None and e_o > 2 * max(e_f, 1e-30)
    if err_worse or ratio < 1 / 1.1:
        kind = "LOSS"
    elif ratio > 1.2 and not noisy:
        kind = "WIN"
    else:
        kind = "TIE"
    return (f"{kind}: fwd p95 {ours.fwd_p95_ms:.3f} ms vs FlexAttention {flex.fwd_p95_ms:.3f} ms "
            f"({ratio:.2f}x), max|err| {e_o} vs {e_f}" + (" (noisy)" if noisy else ""))


def run_benchmark(cfg: HarnessConfig, csv_path: Optional[Path] = None,
                  backward: bool = True, skip: Sequence[str] = ()) -> List[BenchResult]:
    """Time every method at ``cfg`` (the methods in ``skip`` are left out: a
    dense baseline at a long sequence can take minutes per call); each
    method's times are printed as soon as they are measured."""
    if not torch.cuda.is_available():
        raise RuntimeError("benchmark.py needs a GPU")
    mask = _make_mask(cfg)
    density = float(mask.float().mean().item())
    print(f"[cfg] {cfg}", flush=True)
    print(f"[cfg] mask density {density:.4f}; flex_attention available: {_FLEX_AVAILABLE}", flush=True)
    errors = measure_errors(cfg)
    for label, err in errors.items():
        print(f"[err] {label}: max|d_fp64| = {'n/a' if err is None else f'{err:.2e}'}", flush=True)
    q_f, k_f, v_f = _make_qkv(cfg, cfg.dtype)
    q_g, k_g, v_g = _make_qkv(cfg, cfg.dtype, requires_grad=True)
    fwd_fns = _methods(q_f, k_f, v_f, mask, cfg)
    bwd_fns = _methods(q_g, k_g, v_g, mask, cfg)
    results: List[BenchResult] = []
    failures: Dict[str, str] = {}
    for label, f_fwd in fwd_fns.items():
        if label in skip:
            print(f"[skip] {label}: left out (--skip)", flush=True)
            failures[label] = "left out (--skip)"
            continue
        if f_fwd is None:
            print(f"[skip] {label}: not applicable at this shape / unavailable", flush=True)
            failures[label] = "not applicable at this shape / unavailable"
            continue
        print(f"[run ] {label}: fwd", flush=True)
        try:
            with torch.no_grad():
                lat, peak = _time(f_fwd, cfg.warmup_iters, cfg.measure_iters)
        except torch.cuda.OutOfMemoryError:
            print(f"[OOM ] {label}", flush=True)
            failures[label] = "out of memory"
            torch.cuda.empty_cache()
            continue
        except Exception as e:  # noqa: BLE001
            msg = failure_text(e)
            print(f"[fail] {label}: {msg}", flush=True)
            for ln in str(e).splitlines()[-12:]:
                print(f"[fail-detail] {ln}", flush=True)
            failures[label] = msg
            continue
        p50_b = p95_b = None
        f_bwd = bwd_fns.get(label)
        if backward and f_bwd is not None:
            print(f"[run ] {label}: fwd+bwd", flush=True)
            try:
                g_out = torch.randn_like(f_bwd())

                def one():
                    for t in (q_g, k_g, v_g):
                        t.grad = None
                    f_bwd().backward(g_out)

                lat_b, peak_b = _time(one, cfg.warmup_iters, cfg.measure_iters)
                p50_b, p95_b = statistics.median(lat_b), percentile(lat_b, 95)
                peak = max(peak, peak_b)
            except torch.cuda.OutOfMemoryError:
                print(f"[OOM ] {label} fwd+bwd", flush=True)
                torch.cuda.empty_cache()
            except Exception as e:  # noqa: BLE001
                print(f"[fail] {label} fwd+bwd: {type(e).__name__}: {e}", flush=True)
        results.append(BenchResult(label, str(cfg.dtype).replace("torch.", ""), cfg.seq_len_kv,
                                   density, statistics.median(lat), percentile(lat, 95), p50_b,
                                   p95_b, peak, errors.get(label)))
        r = results[-1]
        both = "" if p50_b is None else f", fwd+bwd p50 {p50_b:.3f} / p95 {p95_b:.3f} ms"
        print(f"[time] {label}: fwd p50 {r.fwd_p50_ms:.3f} / p95 {r.fwd_p95_ms:.3f} ms{both}", flush=True)
        torch.cuda.empty_cache()
    widths = [max(len(h), *(len(r.row()[i]) for r in results)) for i, h in enumerate(HEADERS)]
    print("  ".join(h.ljust(w) for h, w in zip(HEADERS, widths)))
    for r in results:
        print("  ".join(c.ljust(w) for c, w in zip(r.row(), widths)))
    by = {r.label: r for r in results}
    if OURS in by:
        print(f"[verdict] {verdict(by[OURS], by.get('flex-attention'), failures.get('flex-attention'))}",
              flush=True)
    if csv_path is not None:
        with open(csv_path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(HEADERS)
            for r in results:
                w.writerow(r.row())
    return results


def _parse(argv: Optional[Sequence[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0],
                                formatter_class=argparse.ArgumentDefaultsHelpFormatter)
    p.add_argument("mode", nargs="?", default="bench", choices=["bench"])
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--seq-q", type=int, default=1, help="query rows (1 = a decode step)")
    p.add_argument("--seq-len", type=int, default=131_072, help="key / value length")
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--block-m", type=int, default=64)
    p.add_argument("--block-n", type=int, default=64)
    p.add_argument("--sink", type=int, default=4)
    p.add_argument("--window", type=int, default=2_048)
    p.add_argument("--dtype", choices=["fp16", "bf16", "fp32"], default="fp16")
    p.add_argument("--warmup", type=int, default=25)
    p.add_argument("--iters", type=int, default=100)
    p.add_argument("--no-backward", action="store_true", help="time the forward only")
    p.add_argument("--csv", type=Path, default=None)
    p.add_argument("--skip", action="append", default=[], metavar="METHOD",
                   choices=["flex-attention", "sdpa-explicit-mask", "sdpa-causal-dense", "eager-dense"],
                   help="leave a comparison method out (repeatable)")
    return p.parse_args(argv)


def main(argv: Optional[Sequence[str]] = None) -> int:
    a = _parse(argv)
    dtype = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[a.dtype]
    cfg = HarnessConfig(batch=a.batch, heads=a.heads, seq_len_q=a.seq_q, seq_len_kv=a.seq_len,
                        head_dim=a.head_dim, block_m=min(a.block_m, a.seq_q), block_n=a.block_n,
                        sink_size=a.sink, window_size=a.window, dtype=dtype,
                        warmup_iters=a.warmup, measure_iters=a.iters)
    run_benchmark(cfg, a.csv, backward=not a.no_backward, skip=a.skip)
    return 0


if __name__ == "__main__":
    sys.exit(main())
