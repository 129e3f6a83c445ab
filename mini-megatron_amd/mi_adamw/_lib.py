"""ctypes binding of libmi_adamw.so (the C ABI declared in include/mi_adamw.h).

The library is loaded after torch has initialised HIP, so that its
libamdhip64 dependency resolves to the HIP runtime torch already mapped and
the device pointers and stream handles torch hands out are valid in it.
The host extension ``_host`` (csrc/host.cpp: FusedAdamW.step()'s steady-state
bookkeeping in C++) is imported with it and bound to the same library's entry
points.  There is no CPU fallback: if either is missing or was built for
another ABI, loading raises.

Both load from this package's directory, or from the directory named by the
environment variable MI_ADAMW_LIB_DIR (another build of the same sources, e.g.
the sanitizer build of ``python -m mi_adamw.build --sanitize DIR``).
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sysconfig

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.environ.get("MI_ADAMW_LIB_DIR") or HERE
LIB_PATH = os.path.join(LIB_DIR, "libmi_adamw.so")

ABI_VERSION = 9
MAX_HYPER = 16
MAX_NORM_BLOCKS = 4096
NOALLOC_SCRATCH_BYTES = 4096
CHUNK_QUANTUM = 4096
ROW_SCALAR_BYTES = 64   # per table row, mi_adamw_step_capturable_rows

OK = 0
E_INVALID = -1
E_ALIGN = -2
E_SCRATCH = -3

STATE_F32 = 0
STATE_BF16 = 1

F_CLIP = 1 << 0
F_BF16_COPY = 1 << 1
F_WRITE_GRAD = 1 << 2
F_AMSGRAD = 1 << 3

T_VEC = 1 << 0

LR_FLOAT = 0
LR_VALUE = 1
LR_DEVICE = 2

# Every symbol include/mi_adamw.h declares.
EXPORTS = (
    "mi_adamw_version",
    "mi_adamw_strerror",
    "mi_adamw_build_chunks",
    "mi_adamw_grad_norm",
    "mi_adamw_grad_norm_flat",
    "mi_adamw_grad_norm_flat_noalloc",
    "mi_adamw_grad_sumsq",
    "mi_adamw_grad_sumsq_flat",
    "mi_adamw_norm_from_sumsq",
    "mi_adamw_set_grads",
    "mi_adamw_scale_grads",
    "mi_adamw_step",
    "mi_adamw_step_flat",
    "mi_adamw_step_prescaled",
    "mi_adamw_step_flat_prescaled",
    "mi_adamw_step_capturable",
    "mi_adamw_step_capturable_rows",
    "mi_adamw_step_fused_chain",
    "mi_adamw_step_fused_chain_rows",
    "mi_adamw_step_flat_fused_chain",
    "mi_adamw_widen_bf16",
    "mi_adamw_probe",
    "mi_adamw_probe_flat",
)


class TensorRow(ctypes.Structure):
    """mi_adamw_tensor: one row of the device-resident tensor table."""

    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("param_copy", ctypes.c_void_p),
        ("max_exp_avg_sq", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("hyper", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


class ChunkRow(ctypes.Structure):
    """mi_adamw_chunk: (tensor row, chunk number within the tensor)."""

    _fields_ = [("tensor", ctypes.c_int32), ("index", ctypes.c_int32)]


class Hyper(ctypes.Structure):
    """mi_adamw_hyper: the fp32 scalars of one (param group, step count)."""

    _fields_ = [
        ("wd_factor", ctypes.c_float),
        ("lerp_w", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("inv_bc2_sqrt", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("neg_step_size", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
    ]


class CaptHyper(ctypes.Structure):
    """mi_adamw_capt_hyper: one param group of a capturable step (no per-step values)."""

    _fields_ = [
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("lerp_w", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
        ("lr", ctypes.c_float),
        ("wd_factor", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("lr_mode", ctypes.c_int32),
        ("lr_ptr", ctypes.c_void_p),
    ]


class FusedHyper(ctypes.Structure):
    """mi_adamw_fused_hyper: one param group of a step in torch's fused=True chain."""

    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("step", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
        ("lr_ptr", ctypes.c_void_p),
    ]


assert ctypes.sizeof(TensorRow) == 64
assert ctypes.sizeof(ChunkRow) == 8
assert ctypes.sizeof(Hyper) == 32
assert ctypes.sizeof(CaptHyper) == 48 and CaptHyper.lr_ptr.offset == 40
assert ctypes.sizeof(FusedHyper) == 56 and FusedHyper.lr_ptr.offset == 48

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

_SIGNATURES = {
    "mi_adamw_version": ([], ctypes.c_char_p),
    "mi_adamw_strerror": ([ctypes.c_int], ctypes.c_char_p),
    "mi_adamw_build_chunks": ([_vp, _i32, _i64, _vp, _i64], _i64),
    "mi_adamw_grad_norm": ([_vp, _vp, _i64, _i64, _f32, _vp, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_grad_norm_flat": ([_vp, _i64, _i64, _f32, _vp, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_grad_norm_flat_noalloc": ([_vp, _i64, _i64, _f32, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_grad_sumsq": ([_vp, _vp, _i64, _i64, _f32, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_grad_sumsq_flat": ([_vp, _i64, _i64, _f32, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_norm_from_sumsq": ([_vp, _i32, _f32, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_set_grads": ([_vp, _i32, _i32, _vp, _vp, _vp, _vp], ctypes.c_int),
    "mi_adamw_scale_grads": ([_vp, _vp, _i64, _i64, _vp, _vp], ctypes.c_int),
    "mi_adamw_step": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_step_flat": ([_vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_step_prescaled": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _f32, _i32, _i32, _i32,
                                 _vp], ctypes.c_int),
    "mi_adamw_step_flat_prescaled": ([_vp, _vp, _vp, _f32, _i64, _i32, _i32, _i32, _vp],
                                     ctypes.c_int),
    "mi_adamw_step_capturable": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp, _i32, _i32,
                                  _i32, _vp], ctypes.c_int),
    "mi_adamw_step_capturable_rows": ([_vp, _i32, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp, _vp,
                                       _i32, _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_step_fused_chain": ([_vp, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp, _f32, _i32,
                                   _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_step_flat_fused_chain": ([_vp, _vp, _vp, _f32, _i64, _i32, _i32, _i32, _vp],
                                       ctypes.c_int),
    "mi_adamw_step_fused_chain_rows": ([_vp, _i32, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp,
                                        _vp, _f32, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_widen_bf16": ([_vp, _vp, _i64, _i64, _vp], ctypes.c_int),
    "mi_adamw_probe": ([_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mi_adamw_probe_flat": ([_vp, _i64, _i32, _i32, _i32, _vp], ctypes.c_int),
}

_lib = None
_host = None

# The entry points the host extension calls, in the order _host.bind takes them.
HOST_BINDINGS = ("mi_adamw_set_grads", "mi_adamw_grad_norm", "mi_adamw_grad_norm_flat",
                 "mi_adamw_grad_sumsq", "mi_adamw_grad_sumsq_flat", "mi_adamw_norm_from_sumsq",
                 "mi_adamw_step_prescaled", "mi_adamw_step_flat_prescaled",
                 "mi_adamw_step_fused_chain", "mi_adamw_step_flat_fused_chain")


class MiAdamwError(RuntimeError):
    """A non-zero return code from libmi_adamw."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and bind libmi_adamw.so.  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise MiAdamwError(
            f"libmi_adamw.so not found at {path}; build it with "
            "`python -m mi_adamw.build` (hipcc, gfx950) before using mi_adamw")
    # Bring up torch's HIP runtime first when a GPU is present, so the
    # library's libamdhip64 dependency binds to the same runtime instance.
    if torch.cuda.is_available():
        torch.cuda.init()
    lib = ctypes.CDLL(path)
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    version = lib.mi_adamw_version().decode()
    if not version.startswith(f"mi_adamw {ABI_VERSION} "):
        raise MiAdamwError(f"libmi_adamw ABI mismatch: library reports {version!r}")
    global _host
    try:
        host = _import_host()
    except ImportError as e:
        raise MiAdamwError(
            f"mi_adamw's host extension (_host) is not built or does not load ({e}); build it "
            "with `python -m mi_adamw.build` against the installed torch") from e
    host.bind(*(ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
                for name in HOST_BINDINGS))
    _host = host
    _lib = lib
    return lib


def _import_host():
    """The host extension: this package's ``_host``, or the one in MI_ADAMW_LIB_DIR."""
    if LIB_DIR == HERE:
        from . import _host as host
        return host
    path = os.path.join(LIB_DIR, "_host" + sysconfig.get_config_var("EXT_SUFFIX"))
    spec = importlib.util.spec_from_file_location(__package__ + "._host", path)
    if spec is None or not os.path.exists(path):
        raise ImportError(f"no host extension at {path}")
    host = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(host)
    return host


def host():
    """The bound host extension (loads the library first)."""
    load()
    return _host


def strerror(code: int) -> str:
    return load().mi_adamw_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code != OK:
        raise MiAdamwError(f"{what} failed: {strerror(code)} (code {code})")


def version() -> str:
    return load().mi_adamw_version().decode()
