"""Build the reactor library ``oct_amd/libprometheus_reactor.so`` for gfx950.

Every ``oct_amd/csrc/*.hip`` file is compiled with hipcc (in parallel) and
linked into one shared library whose only exported symbols are the C ABI
declared in ``include/prometheus_reactor.h``.  The build is in-tree so the
library travels with the repository snapshot to the GPU box.

Usage: ``python -m oct_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libprometheus_reactor.so"

ARCH = os.environ.get("OCT_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # Packed-fp32 instructions are excluded: some of their forms have given wrong results on these boxes.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the reactor needs the ROCm toolchain")


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build_reactor(verbose: bool = False) -> Path:
    """Compile and link the reactor library; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources found")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel stub clang failed to emit)
    # fails the build instead of the first call.
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build of the same
# sources (the GPU code is built as usual: each -fsanitize= applies to the host
# pass only).  Load it with $OCT_PROMETHEUS_REACTOR and the clang ASan runtime
# preloaded; oct_amd/sanitize.py does both and runs the host-logic tests.
SAN_DIR = PKG_DIR / "_build_san"
SAN_LIB_PATH = SAN_DIR / "libprometheus_reactor_san.so"
REACTOR_ENV = "OCT_PROMETHEUS_REACTOR"  # the library override the loader honours
SAN_FLAGS = ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
             "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer -Xarch_host -g1").split()


def build_reactor_sanitized(verbose: bool = False) -> Path:
    """Compile and link the host-sanitized reactor into oct_amd/_build_san/."""
    SAN_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC_DIR.glob("*.hip"))

    def compile_one(src: Path) -> Path:
        obj = SAN_DIR / (src.stem + ".o")
        cmd = [_hipcc(), *HIPCC_FLAGS, *SAN_FLAGS, "-c", str(src), "-o", str(obj)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc (sanitized) failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
        return obj

    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, sources))
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *SAN_FLAGS, "-o", str(SAN_LIB_PATH),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link (sanitized) failed:\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        print(f"built {SAN_LIB_PATH}")
    return SAN_LIB_PATH


def build_oracle(verbose: bool = False) -> Path:
    """Compile the CPU oracle (test infrastructure) with its Makefile."""
    proc = subprocess.run(["make", "-s", "-C", str(REPO_DIR / "oracle")], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")
    path = REPO_DIR / "oracle" / "liboct_oracle.so"
    if verbose:
        print(f"built {path}")
    return path


CBRIDGE_DIR = PKG_DIR / "cbridge"
CBRIDGE_CHECK = CBRIDGE_DIR / "bridge_check"
CBRIDGE_FLAGS = ["-std=c11", "-O2", "-Wall", "-Wextra", "-Wpedantic", "-Werror", f"-I{REPO_DIR / 'include'}"]


def build_cbridge(verbose: bool = False, out: Path = CBRIDGE_CHECK) -> Path:
    """Compile the C loader (``cbridge/prom_bridge.c``) with its check program.

    Plain gcc, no HIP: the loader only dlopens the reactor library."""
    cmd = ["gcc", *CBRIDGE_FLAGS, str(CBRIDGE_DIR / "prom_bridge.c"), str(CBRIDGE_DIR / "bridge_check.c"),
           "-o", str(out), "-ldl", "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"C bridge build failed:\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build_reactor(verbose=True)
    build_cbridge(verbose=True)
    build_oracle(verbose=True)
    sys.exit(0)
