"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

Builds the library (its host code: argument checks, the chunk-table builder, the
gradient patch's host loop, the no-alloc scratch lookup), the native host extension
(csrc/host.cpp: refcounting, the plan, prepare()'s checks and row patching), the oracle
and the plain-C ABI test program with -fsanitize=address,undefined into _build/asan
(``python -m mi_adamw.build --sanitize``, ``make asan`` in oracle/ and tests/c/), then
runs, with clang's shared ASan runtime preloaded and leak detection off:
- ``abi_check cpu`` (version, error text, chunk tables, every argument rejection);
- the CPU suites that drive the host extension, the host logic and the oracle:
  tests/test_native_host.py, test_zero_host.py, test_host.py and test_oracle.py.
Any sanitizer report fails the run (halt_on_error).  The test also checks that every
sanitized binary calls the sanitizers' hooks, and that a heap overflow built and run the
same way is reported.  Skipped, with the reason, only if the sanitizer runtime or ROCm's
clang is missing.
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "_build", "asan")
SUITES = ["tests/test_native_host.py", "tests/test_zero_host.py", "tests/test_host.py",
          "tests/test_oracle.py"]
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _env(runtime: str) -> dict:
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": runtime,
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0:"
                        "alloc_dealloc_mismatch=0:new_delete_type_mismatch=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "MI_ADAMW_LIB_DIR": OUT,
        "MI_ADAMW_ORACLE_LIB": os.path.join(OUT, "liboracle.so"),
        "PYTHONPATH": os.pathsep.join([ROOT, os.path.join(ROOT, "mini-megatron_amd")]
                                      + ([env["PYTHONPATH"]] if env.get("PYTHONPATH") else [])),
    })
    return env


def _check(res: subprocess.CompletedProcess) -> str:
    out = res.stdout + res.stderr
    found = [r for r in REPORTS if r in out]
    assert res.returncode == 0 and not found, f"rc {res.returncode}, reports {found}\n{out[-6000:]}"
    return out


def test_host_code_under_asan_and_ubsan():
    from mi_adamw import build
    runtime = build.asan_runtime()
    if runtime is None:
        pytest.skip("clang's shared AddressSanitizer runtime (libclang_rt.asan-x86_64.so) "
                    "is not installed")
    build.build_sanitized(OUT)
    for d in ("oracle", os.path.join("tests", "c")):
        subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, d), "asan", f"OUT={OUT}"],
                       check=True)
    env = _env(runtime)
    # instrumented: each sanitized binary calls the ASan and UBSan hooks
    ext = [f for f in os.listdir(OUT) if f.startswith("_host") and f.endswith(".so")]
    for name in ["libmi_adamw.so", "liboracle.so", "abi_check", *ext]:
        syms = subprocess.run(["nm", "-D", "--undefined-only", os.path.join(OUT, name)],
                              capture_output=True, text=True, check=True).stdout
        assert "__asan_report_" in syms and "__ubsan_handle_" in syms, name
    # the harness sees a report: a heap overflow built and run the same way must fail
    src = os.path.join(OUT, "overflow.c")
    with open(src, "w") as f:
        f.write("#include <stdlib.h>\nint main(void) { volatile char *b = malloc(8); "
                "b[8] = 1; free((void *)b); return 0; }\n")
    subprocess.run([build.clang(cxx=False), "-g", "-fsanitize=address,undefined",
                    "-shared-libasan", src, "-o", os.path.join(OUT, "overflow")], check=True)
    bad = subprocess.run([os.path.join(OUT, "overflow")], env=env, capture_output=True,
                         text=True, timeout=60)
    assert bad.returncode != 0 and "heap-buffer-overflow" in bad.stderr, bad.stderr[-2000:]
    out = _check(subprocess.run([os.path.join(OUT, "abi_check"), "cpu"], env=env,
                                capture_output=True, text=True, timeout=300))
    assert "abi_check cpu: ok" in out
    # the sanitized builds are the ones the suites load
    probe = ("import mi_adamw._lib as L, oracle.oracle as O; L.load(); "
             "print(L._lib._name); print(L._host.__file__); print(O._LIB_PATH)")
    out = _check(subprocess.run([sys.executable, "-c", probe], env=env, cwd=ROOT,
                                capture_output=True, text=True, timeout=300))
    loaded = out.split()
    assert loaded[-3:] == [os.path.join(OUT, "libmi_adamw.so"),
                           os.path.join(OUT, os.path.basename(loaded[-2])),
                           os.path.join(OUT, "liboracle.so")], loaded[-3:]
    out = _check(subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                                 "-m", "not gpu", *SUITES], env=env, cwd=ROOT,
                                capture_output=True, text=True, timeout=900))
    assert " passed" in out and " failed" not in out
    print(out.strip().splitlines()[-1], flush=True)
