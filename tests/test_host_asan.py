"""The library's host code under AddressSanitizer (CPU only, no GPU needed).

Every HIP source is compiled with the sanitizer on its host pass only (the
flag follows ``-Xarch_host``; device code is built as usual), linked with the
driver ``tests/asan/capi_host_checks.cpp`` into one executable, and run: the
dK/dV work-list builder on random column lists with exactly sized outputs,
``gki_rolling_stream`` against a brute-force count, and every launching entry
point rejecting bad arguments before it reaches the device.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "graph-kernel-injection_amd" / "csrc"
HOST_ASAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    return None


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise AssertionError(f"{' '.join(map(str, cmd))}\n{err[-4000:]}")


def test_capi_host_code_under_address_sanitizer(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-fPIC", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             f"-I{ROOT / 'include'}", *HOST_ASAN]
    sources = sorted(CSRC.glob("*.hip"))

    def compile_one(src):
        obj = tmp_path / (src.stem + ".o")
        _run([hipcc, *flags, "-c", str(src), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_one, sources))
    drv = tmp_path / "capi_host_checks.o"
    _run([hipcc, "-std=c++17", "-O1", "-g", f"-I{ROOT / 'include'}", *HOST_ASAN, "-c",
          str(ROOT / "tests" / "asan" / "capi_host_checks.cpp"), "-o", str(drv)])
    exe = tmp_path / "capi_host_checks"
    _run([hipcc, "--offload-arch=gfx950", *HOST_ASAN, str(drv), *map(str, objs), "-o", str(exe)])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
    assert res.returncode == 0, (res.stdout + res.stderr)[-4000:]
    assert "host checks passed" in res.stdout
