"""Run the host-logic tests against the AddressSanitizer + UBSan build of the reactor.

The library's host code (handle registry, request validation, async task
tables, batch arenas, the resident model-block state machine, the non-strict
runtime) is compiled with ``-fsanitize=address,undefined`` for the host pass
only (``oct_amd.build.build_reactor_sanitized``); device code is unchanged.
Python is not instrumented, so the clang ASan runtime is preloaded into the
test process and the library is selected with ``$OCT_PROMETHEUS_REACTOR``
(the reference's own override, bridge.go:552-582).  Leak checking is off
(the interpreter keeps its allocations to exit); every other report aborts
the run.

Usage::

    python -m oct_amd.sanitize            # build, then the device-less host tests
    python -m oct_amd.sanitize --no-build -m gpu tests/test_gpu_async.py   # any pytest arguments

The default test files are the device-less ones: on a machine without a GPU
every call stops at its validation or reports the device as unavailable.
With a device present this does not extend to the GPU tests: with the ASan
runtime preloaded, the ROCm runtime aborts while the first runtime handle
initialises the device (no sanitizer report precedes the abort), so the
device-backed paths of the host state machines are not covered.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

from oct_amd import build

DEFAULT_TESTS = ["tests/test_abi.py", "tests/test_model_block_abi.py", "tests/test_async_batch_abi.py",
                 "tests/test_runtime_nonstrict.py", "tests/test_sgemm_plan.py"]


def asan_runtime() -> str:
    clang = Path(build._hipcc()).resolve().parent.parent / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path("/opt/rocm/llvm/bin/clang")
    out = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    if out.returncode != 0 or not Path(path).exists():
        raise RuntimeError("clang's shared ASan runtime was not found")
    return path


def main(argv: list[str]) -> int:
    if argv and argv[0] == "--no-build":
        argv = argv[1:]
    else:
        build.build_reactor_sanitized(verbose=True)
    env = dict(os.environ)
    # the ASan runtime goes first; whatever the environment already preloads stays
    env["LD_PRELOAD"] = ":".join(x for x in (asan_runtime(), os.environ.get("LD_PRELOAD", "")) if x)
    env["ASAN_OPTIONS"] = ("detect_leaks=0:halt_on_error=1:abort_on_error=1:detect_odr_violation=0:"
                           "verify_asan_link_order=0")
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env[build.REACTOR_ENV] = str(build.SAN_LIB_PATH)
    args = argv or ["-m", "not gpu", *DEFAULT_TESTS]
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *args]
    print("running:", " ".join(cmd), flush=True)
    return subprocess.run(cmd, cwd=str(build.REPO_DIR), env=env).returncode


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
