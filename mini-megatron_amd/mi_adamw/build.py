"""Compile libmi_adamw.so for gfx950 from csrc/ with hipcc, and the host
extension _host from csrc/host.cpp with g++, in place.

Run as ``python -m mi_adamw.build`` (with ``mini-megatron_amd`` on sys.path)
or through ``__graft_entry__.build()``.  Both land next to this file, where
``mi_adamw._lib`` loads them from.  The host extension is built against the
installed torch (its headers and libtorch_python), whose C++ ABI it must match.

``python -m mi_adamw.build --sanitize DIR`` builds both into DIR instead, with
their host code under AddressSanitizer and UndefinedBehaviorSanitizer: the
library's host code through hipcc (the sanitizers for the host pass only; the
gfx950 code object is built as usual) and the host extension with ROCm's clang++,
so that one ASan runtime, clang's shared one, serves the whole process.  Loaded
with ``MI_ADAMW_LIB_DIR=DIR`` and that runtime preloaded (``asan_runtime()``);
the CPU test tests/test_sanitizers.py does this.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
SOURCES = [os.path.join(HERE, "csrc", "mi_adamw.hip")]
INCLUDE = os.path.join(REPO, "include")
OUTPUT = os.path.join(HERE, "libmi_adamw.so")
HOST_SOURCE = os.path.join(HERE, "csrc", "host.cpp")
HOST_OUTPUT = os.path.join(HERE, "_host" + sysconfig.get_config_var("EXT_SUFFIX"))

# -ffp-contract=off: the kernels spell out every fused multiply-add themselves,
#   in the places torch-ROCm's kernels fuse, so the compiler must not add more.
# -packed-fp32-ops off: packed fp32 VALU forms are kept out of the code object.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build mi_adamw")
    return path


def _run(cmd: list[str], verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")


# Host-code sanitizer flags of the --sanitize build (clang's driver; with hipcc each
# follows -Xarch_host so that only the host pass gets it).
SANITIZE_FLAGS = ["-fsanitize=address", "-fsanitize=undefined", "-fno-omit-frame-pointer"]


def clang(cxx: bool = True) -> str:
    """ROCm's clang (C++ or C driver)."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "llvm", "bin", "clang++" if cxx else "clang")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: the sanitizer build needs ROCm's clang")
    return path


def asan_runtime() -> str | None:
    """clang's shared AddressSanitizer runtime (to preload), or None if it is absent."""
    try:
        res = subprocess.run([clang(cxx=False), "-print-file-name=libclang_rt.asan-x86_64.so"],
                             capture_output=True, text=True)
    except (OSError, RuntimeError):
        return None
    path = res.stdout.strip()
    return path if res.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def host_command(output: str, compiler: str | None = None, extra=()) -> list[str]:
    """g++ line of the host extension: torch's headers and C++ ABI, Python's headers."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    tlib = os.path.join(tdir, "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    gxx = compiler or shutil.which("g++") or "g++"
    return [gxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
            *extra,
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-I", os.path.join(tdir, "include"),
            "-I", os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
            "-I", sysconfig.get_paths()["include"], "-I", INCLUDE,
            HOST_SOURCE, "-o", output,
            "-L", tlib, "-ltorch_python", "-ltorch", "-ltorch_cpu", "-lc10",
            f"-Wl,-rpath,{tlib}"]


def build(verbose: bool = False) -> str:
    """Compile the kernels into libmi_adamw.so and the host extension; returns the
    library path."""
    tmp = OUTPUT + ".tmp"
    _run([hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, *SOURCES, "-o", tmp], verbose, "hipcc")
    os.replace(tmp, OUTPUT)
    tmp = HOST_OUTPUT + ".tmp"
    _run(host_command(tmp), verbose, "g++ (host extension)")
    os.replace(tmp, HOST_OUTPUT)
    return OUTPUT


def build_sanitized(outdir: str, verbose: bool = False) -> str:
    """The --sanitize build into `outdir`: libmi_adamw.so and the host extension with
    their host code under ASan + UBSan, linked against clang's shared ASan runtime.
    Returns `outdir`."""
    os.makedirs(outdir, exist_ok=True)
    host_san = [f for flag in SANITIZE_FLAGS for f in ("-Xarch_host", flag)]
    flags = [f for f in HIPCC_FLAGS if f != "-O3"] + ["-O1", "-g"]
    _run([hipcc(), *flags, *host_san, "-shared-libasan", "-I", INCLUDE, *SOURCES, "-o",
          os.path.join(outdir, "libmi_adamw.so")], verbose, "hipcc (sanitized)")
    ext = "_host" + sysconfig.get_config_var("EXT_SUFFIX")
    _run(host_command(os.path.join(outdir, ext), compiler=clang(),
                      extra=["-O1", "-g", *SANITIZE_FLAGS, "-shared-libasan"]),
         verbose, "clang++ (sanitized host extension)")
    return outdir


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized(sys.argv[sys.argv.index("--sanitize") + 1], verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
