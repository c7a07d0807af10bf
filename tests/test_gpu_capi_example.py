"""A C++ caller of the C ABI alone: ``tests/capi/capi_forward_example.cpp``
(hipMalloc'd buffers, no Python or torch in the process) builds the StreamingLLM
mask, the forward tile classes and the CSR schedule with the library, runs
``gki_bsa_fwd`` on a ragged bf16 shape (N = 300, not a multiple of any tile) and
checks O and the (natural) LSE against a double-precision attention over the token
rule computed in the same program (O within 2e-2 + 1e-2 |ref|, LSE within
2.5e-3); a schedule of the wrong size must be rejected. ``build()`` links the
program against the in-tree library."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "capi" / "capi_forward_example"


def test_c_abi_forward_from_a_cpp_caller():
    assert EXE.exists(), f"{EXE} is not built: run graph-kernel-injection_amd/build.py"
    print("[case] C++ caller: bf16 1x2x300x64 S4 W64 through gki_bsa_fwd", flush=True)
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=90)
    print(res.stdout, res.stderr, flush=True)
    assert res.returncode == 0, (res.stdout + res.stderr)[-2000:]
    assert "capi forward example passed" in res.stdout
