"""The C loader's whole call sequence on the GPU, in a process of its own.

``bridge_check run`` opens the reactor the way bridge.go:242-394 does
(dlopen, ABI 1, create with reduction ring depth 3, probe, sgemm and the
optional entries), then calls through each trampoline
(bridge_dlopen_linux.go:56-67, 305-327, 395-448) with answers fixed by exact
arithmetic or closed forms: integer SGEMMs compared bit for bit (2x3x2,
67x129x95, 1024x1024x2048), SGEMM argument errors, FFT64 of an impulse and
of a pure tone at 4096 points plus counts 1 and 3, an async
submit/query/consume/abandon cycle, Gemma input RMSNorm on constant rows
with a stale generation, and strict.go's matmul through its own runtime.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

from oct_amd import build as b
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

LIB = Path(p.__file__).resolve().parent / "libprometheus_reactor.so"


def test_c_loader_call_sequence_known_answers():
    exe = b.CBRIDGE_CHECK
    if not exe.exists():
        pytest.fail(f"{exe} is not built; run python -m oct_amd.build")
    print(f"running {exe} run {LIB}", flush=True)
    proc = subprocess.run([str(exe), "run", str(LIB)], capture_output=True, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    lines = proc.stdout.strip().splitlines()
    assert lines[-1] == "PASSED failures=0"
    assert not [ln for ln in lines if ln.startswith("FAIL")]
    assert sum(ln.startswith("ok ") for ln in lines) >= 20
