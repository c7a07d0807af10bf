"""Build the gfx950 HIP library ``gki/libgki_bsa.so`` in-tree.

Usage: ``python graph-kernel-injection_amd/build.py`` (or via
``__graft_entry__.build()``). Each ``csrc/*.hip`` file is compiled separately
and in parallel with ``hipcc --offload-arch=gfx950``, then linked into one
shared library exposing the C ABI declared in ``include/gki_bsa.h``.

Packed FP32 VALU instructions are disabled (``-packed-fp32-ops``): the kernels
are written against scalar/float2 fp32 arithmetic only.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
REPO_ROOT = PKG_ROOT.parent
BUILD_DIR = REPO_ROOT / "_build" / "gki"
LIB_PATH = PKG_ROOT / "gki" / "libgki_bsa.so"
# a C++ caller of the C ABI alone (hipMalloc, no torch), run by a GPU test
EXAMPLE_SRC = REPO_ROOT / "tests" / "capi" / "capi_forward_example.cpp"
EXAMPLE_EXE = REPO_ROOT / "tests" / "capi" / "capi_forward_example"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_ROOT / 'include'}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _compile(hipcc: str, src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        # the host pass always warns that it does not know the packed-fp32 feature
        err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link ``libgki_bsa.so``. Always rebuilds."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[gki] built {LIB_PATH} from {len(sources)} HIP sources for {ARCH}")
    if EXAMPLE_SRC.exists():
        _build_example(hipcc)
        if verbose:
            print(f"[gki] built {EXAMPLE_EXE} against {LIB_PATH.name}")
    return LIB_PATH


def _build_example(hipcc: str) -> None:
    """Link the C-ABI example against the in-tree library (found via its rpath)."""
    rpath = os.path.relpath(LIB_PATH.parent, EXAMPLE_EXE.parent)
    cmd = [hipcc, *HIPCC_FLAGS, str(EXAMPLE_SRC), "-o", str(EXAMPLE_EXE),
           f"-L{LIB_PATH.parent}", "-lgki_bsa", f"-Wl,-rpath,$ORIGIN/{rpath}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed on {EXAMPLE_SRC.name}:\n{err}")


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
