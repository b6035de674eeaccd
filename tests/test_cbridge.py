"""The C loader (oct_amd/cbridge) on the CPU: build, discovery and every
ReactorIssue path of bridge.go:242-394.

Small stand-in reactor libraries are compiled from C in the test's temporary
directory so each failure can be forced: no abi symbol, a wrong ABI version,
a create that fails, a probe that succeeds but no sgemm; the reference's
own bridge tests (bridge_test.go:8-57: a missing symbol and an ABI mismatch
reported as structured issues, a stub library that loads and probes) are
among these cases.  The real library
with the SKIP_VULKAN_INIT test flag forces the probe-unavailable path on any
machine, as bridge.go's reactorTestFlagsFromEnv (bridge.go:584-594) passes
the flag through.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from oct_amd import build as b
from oct_amd import prometheus as p

REPO = Path(__file__).resolve().parent.parent
LIB = REPO / "oct_amd" / "libprometheus_reactor.so"

FAKE_REACTOR = r"""
#include <stdint.h>
#include <stdlib.h>
typedef struct { uint32_t available, backend_type, reason_code; } Caps;
#ifndef ABI
#define ABI 1u
#endif
#ifndef NO_ABI
uint32_t prometheus_reactor_abi_version(void) { return ABI; }
#endif
int prometheus_reactor_runtime_create(void* cfg, void** out) {
  (void)cfg;
#ifdef CREATE_FAILS
  (void)out;
  return 3;
#else
  *out = malloc(1);
  return 0;
#endif
}
int prometheus_reactor_runtime_destroy(void* h) { free(h); return 0; }
int prometheus_reactor_runtime_probe(void* h, Caps* c) {
  (void)h; c->available = 1; c->backend_type = 2; c->reason_code = 0; return 0;
}
"""


@pytest.fixture(scope="module")
def check(tmp_path_factory) -> Path:
    """A fresh -Werror build of the loader and its check program."""
    out = tmp_path_factory.mktemp("cbridge") / "bridge_check"
    return b.build_cbridge(out=out)


def _fake(tmp: Path, name: str, *defines: str) -> Path:
    src = tmp / f"{name}.c"
    src.write_text(FAKE_REACTOR)
    lib = tmp / f"{name}.so"
    cmd = ["gcc", "-shared", "-fPIC", "-O1", *[f"-D{d}" for d in defines], str(src), "-o", str(lib)]
    subprocess.run(cmd, check=True, capture_output=True)
    return lib


def _run(exe: Path, *args: str, env_extra=None, cwd=None):
    env = {k: v for k, v in os.environ.items() if k not in (p.REACTOR_ENV_VAR, p.REACTOR_TEST_FLAGS_ENV_VAR)}
    env.update(env_extra or {})
    proc = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=120, env=env, cwd=cwd)
    return proc.returncode, proc.stdout.strip()


def test_header_compiles_as_iso_c_and_cpp(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "prom_bridge.h"\nint main(void) { return prom_issue_name(PROM_ISSUE_NONE)[0] == 0; }\n')
    for compiler, std in (("gcc", "-std=c99"), ("g++", "-std=c++17")):
        cmd = [compiler, std, "-Wall", "-Wextra", "-Wpedantic", "-Werror", "-fsyntax-only",
               f"-I{REPO / 'include'}", f"-I{REPO / 'oct_amd' / 'cbridge'}"]
        cmd += ["-x", "c++", str(src)] if compiler == "g++" else [str(src)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr


def test_missing_library_is_not_found(check, tmp_path):
    rc, out = _run(check, "open", str(tmp_path / "absent.so"))
    assert rc == 3 and out.startswith("issue=reactor_not_found")
    assert "message=prometheus reactor not found" in out


def test_unloadable_file_is_load_failed(check, tmp_path):
    junk = tmp_path / "libprometheus_reactor.so"
    junk.write_text("not an ELF object\n")
    rc, out = _run(check, "open", str(junk))
    assert rc == 3 and out.startswith("issue=reactor_load_failed")
    assert "prometheus reactor load failed" in out


def test_missing_abi_symbol(check, tmp_path):
    rc, out = _run(check, "open", str(_fake(tmp_path, "noabi", "NO_ABI")))
    assert rc == 3
    assert out.startswith("issue=symbol_missing symbol=prometheus_reactor_abi_version")
    assert 'missing symbol "prometheus_reactor_abi_version"' in out


def test_abi_mismatch_reports_both_versions(check, tmp_path):
    rc, out = _run(check, "open", str(_fake(tmp_path, "abi2", "ABI=2u")))
    assert rc == 3 and out.startswith("issue=abi_mismatch") and " abi=2 " in out
    assert "expected=1 actual=2" in out


def test_create_failure(check, tmp_path):
    rc, out = _run(check, "open", str(_fake(tmp_path, "nocreate", "CREATE_FAILS")))
    assert rc == 3 and out.startswith("issue=runtime_create_failed")


def test_probe_ok_without_sgemm_is_symbol_missing(check, tmp_path):
    # create, destroy and probe resolve and the probe reports a device, but
    # the mandatory sgemm entry is absent (bridge.go:329-339).
    rc, out = _run(check, "open", str(_fake(tmp_path, "nosgemm")))
    assert rc == 3 and out.startswith("issue=symbol_missing symbol=prometheus_reactor_runtime_sgemm")


def test_forced_unavailable_runtime_is_probe_unavailable(check):
    flags = {p.REACTOR_TEST_FLAGS_ENV_VAR: hex(p.TESTCFG_SKIP_VULKAN_INIT)}
    rc, out = _run(check, "open", str(LIB), env_extra=flags)
    assert rc == 3 and out.startswith("issue=runtime_probe_unavailable")
    assert f"reason={p.PROM_REASON_VULKAN_UNAVAILABLE}" in out


def test_strict_matmul_never_substitutes_the_cpu(check):
    flags = {p.REACTOR_TEST_FLAGS_ENV_VAR: str(p.TESTCFG_SKIP_VULKAN_INIT)}
    rc, out = _run(check, "strict", str(LIB), env_extra=flags)
    assert rc == 3
    assert out.startswith("strict=error message=PROMETHEUS requires GPU matrix execution: ")


def test_discovery_env_var_then_executable_directory(check, tmp_path):
    # $OCT_PROMETHEUS_REACTOR wins (bridge.go:567-570) ...
    fake = _fake(tmp_path, "abi7", "ABI=7u")
    rc, out = _run(check, "open", env_extra={p.REACTOR_ENV_VAR: str(fake)}, cwd=tmp_path)
    assert rc == 3 and " abi=7 " in out
    # ... else a library beside the executable is found (bridge.go:573-575).
    exe_dir = tmp_path / "bin"
    exe_dir.mkdir()
    exe = exe_dir / "bridge_check"
    shutil.copy2(check, exe)
    shutil.copy2(_fake(tmp_path, "abi9", "ABI=9u"), exe_dir / "libprometheus_reactor.so")
    rc, out = _run(exe, "open", cwd=tmp_path)
    assert rc == 3 and " abi=9 " in out
    # ... and with nothing anywhere, not found.
    rc, out = _run(check, "open", cwd=tmp_path)
    assert rc == 3 and out.startswith("issue=reactor_not_found")


def test_loader_paths_under_address_and_undefined_sanitizers(tmp_path):
    """The loader and check program built with gcc's AddressSanitizer (leak
    checking on: a C program owns every allocation) and UBSan, through every
    issue path and the strict matmul's error path."""
    exe = tmp_path / "bridge_check_asan"
    cmd = ["gcc", *b.CBRIDGE_FLAGS, "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", str(b.CBRIDGE_DIR / "prom_bridge.c"), str(b.CBRIDGE_DIR / "bridge_check.c"),
           "-o", str(exe), "-ldl", "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0 and "asan" in proc.stderr.lower():
        pytest.skip(f"gcc's sanitizer runtime is not installed: {proc.stderr[-300:]}")
    assert proc.returncode == 0, proc.stderr
    san = {"ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}
    # With the real reactor, the HIP runtime it links (libamdhip64) is loaded
    # too; its start-up allocations stay live until dlclose unloads it and are
    # then reported as leaks from the unloaded module, so leak checking stays
    # on for the stand-in libraries only (every other report still aborts).
    flags = {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1", "UBSAN_OPTIONS": san["UBSAN_OPTIONS"],
             p.REACTOR_TEST_FLAGS_ENV_VAR: str(p.TESTCFG_SKIP_VULKAN_INIT)}
    cases = [
        (("open", str(tmp_path / "absent.so")), san, "issue=reactor_not_found"),
        (("open", str(_fake(tmp_path, "noabi", "NO_ABI"))), san, "issue=symbol_missing"),
        (("open", str(_fake(tmp_path, "abi2", "ABI=2u"))), san, "issue=abi_mismatch"),
        (("open", str(_fake(tmp_path, "nocreate", "CREATE_FAILS"))), san, "issue=runtime_create_failed"),
        (("open", str(_fake(tmp_path, "nosgemm"))), san, "issue=symbol_missing"),
        (("open", str(LIB)), flags, "issue=runtime_probe_unavailable"),
        (("strict", str(LIB)), flags, "strict=error message=PROMETHEUS requires GPU matrix execution: "),
    ]
    for args, env, want in cases:
        env_all = {k: v for k, v in os.environ.items() if k not in (p.REACTOR_ENV_VAR, p.REACTOR_TEST_FLAGS_ENV_VAR)}
        env_all.update(env)
        proc = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=120, env=env_all)
        assert proc.returncode == 3, (args, proc.returncode, proc.stdout, proc.stderr[-2000:])
        assert proc.stdout.startswith(want), (args, proc.stdout)
        assert "Sanitizer" not in proc.stderr and "runtime error" not in proc.stderr, proc.stderr[-2000:]
