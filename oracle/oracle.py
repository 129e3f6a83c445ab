"""CPU oracle for the fused clip + AdamW step -- TEST INFRASTRUCTURE ONLY.

The product never imports this module.  Only the pytest suite and the smoke
check (``__graft_entry__.smoke``) load it, and there only as the checker.

It restates, in NumPy plus the C kernels of ``adamw_oracle.c``:

* ``hyper_from_group`` -- the host-side float64 scalar arithmetic of
  ``torch/optim/adam.py:414-536`` (step += 1, bias corrections, step size,
  ``bc2 ** 0.5``) and ATen's cast of each Python scalar to the fp32 opmath
  type of the kernel that consumes it.
* ``adamw_step`` / ``adamw_step_bf16state`` -- the per-element op chain of
  ``_single_tensor_adam`` (``adam.py:419,457,476,545,547``; with amsgrad
  ``:539-543``) and ``ATen/native/Lerp.h:21-35``, one fp32 rounding per ATen
  kernel.
* ``capt_scalars`` / ``adamw_step_capt`` / ``adamw_step_capt_bf16state`` -- the
  same loop with ``capturable=True`` (``adam.py:480-527``): the per-step values
  as fp32 0-d tensor ops, then ``p + m / (sqrt(v) / (sqrt(bc2) * -step_size) +
  eps / -step_size)``.
* ``fused_scalars`` / ``adamw_step_fused`` / ``adamw_step_fused_bf16state`` -- torch's
  ``fused=True`` chain (``adam.py:803-895`` -> ``torch._fused_adamw_``, per element
  ``adam_math`` of ``ATen/native/hip/fused_adam_utils.cuh``): float64 hyperparameters,
  m, v and the decayed p formed in float64 and rounded once, per-step values formed
  in float64 and handed over as fp32.
* ``total_norm`` / ``clip_coef`` -- ``torch/nn/utils/clip_grad.py:50-117``
  (global L2 norm over all gradients) and ``:165-169`` (the clamped
  coefficient), the clip mini-megatron defines at ``config.py:16``
  (``MAX_GRAD_NORM = 1.0``).

How each function is pinned (none of it is trusted on its own):

* The op chain: ``OPMODEL_TORCH_CPU`` is checked bit-for-bit against golden
  fixtures written by ``torch.optim.AdamW(foreach=False)`` on the CPU
  (``tests/golden/make_golden.py``), and ``OPMODEL_TORCH_ROCM`` bit-for-bit
  against each ATen op of the same chain run by torch on the MI355X (a GPU
  test).  Closed forms pin the rest: ``lr = 0`` leaves p bitwise unchanged,
  step 1 from zero state gives ``m = f32(0.1 g)``, ``g = 0`` decays m and v
  geometrically, ``wd = 0`` is the identity on the first op.
* The clip norm: fixtures from ``clip_grad_norm_`` (rel 1e-6), the closed form
  ``|c| sqrt(N)`` for constant gradients, and an exact float64 brute force on
  tiny inputs.
* The capturable chain: torch does not run it on the CPU, so it is pinned
  bit-for-bit against ``torch.optim.AdamW(capturable=True, foreach=False)`` on
  the MI355X (a GPU test, with torch's own per-step values), and on the CPU by
  closed forms (step 1: ``bc1 = 1 - beta1``; lr 0 leaves p unchanged) and the
  mutation tests.
* The fused=True chain: torch runs it only on the GPU (its CPU kernel is other
  arithmetic), so fixtures written by torch's own GPU kernel
  (``tests/golden/make_fused_golden.py``) pin it bit for bit on the CPU: whole chains
  over the options, inputs on which the candidate fused multiply-add forms round apart
  (found by ``tests/golden/fused_cases.c``; each other form is rejected), and per-step
  values at (lr, step) where their candidate forms round apart.  Closed forms (lr = 0,
  g = 0, the first step), a float64 bound, agreement with the default chain and the
  mutation tests pin it further; on the GPU it is compared with torch directly.
* The bf16 paths: a brute-force round-to-nearest-even check of
  ``oracle_f32_to_bf16`` over every rounding boundary class, and torch's own
  ``Tensor.to(torch.bfloat16)`` on the same values.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MI_ADAMW_ORACLE_LIB: another build of adamw_oracle.c (the sanitizer build, `make -C
# oracle asan OUT=DIR`)
_LIB_PATH = os.environ.get("MI_ADAMW_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")


class OpModel(ctypes.Structure):
    """Which ATen ops were compiled with fused multiply-adds (see adamw_oracle.c)."""

    _fields_ = [
        ("lerp_fma", ctypes.c_int),
        ("addcmul_mode", ctypes.c_int),
        ("addcdiv_mode", ctypes.c_int),
        ("div_recip", ctypes.c_int),
    ]

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return (f"OpModel(lerp_fma={self.lerp_fma}, addcmul_mode={self.addcmul_mode}, "
                f"addcdiv_mode={self.addcdiv_mode}, div_recip={self.div_recip})")


class Hyper(ctypes.Structure):
    _fields_ = [
        ("wd_factor", ctypes.c_float),
        ("lerp_w", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("bc2_sqrt", ctypes.c_double),
        ("eps", ctypes.c_float),
        ("neg_step_size", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
    ]


# torch 2.10 CPU build (AVX-512 vectorised ATen kernels): lerp is fused
# (fma(w, end-self, self)), addcmul is fma(s*g, g, v), addcdiv is
# p + (s*m)/d rounded per op, and the division by a Python scalar is a true
# fp32 division.  Its vectorised sqrt is not always correctly rounded (about
# 0.6% of inputs differ by 1 ulp from IEEE sqrt), so the oracle, which uses the
# IEEE sqrt, matches it exactly on m and v and within 1 ulp on p.
# Pinned by tests/test_oracle.py against the tests/golden fixtures.
OPMODEL_TORCH_CPU = OpModel(lerp_fma=1, addcmul_mode=2, addcdiv_mode=2, div_recip=0)

# torch 2.10.0+rocm7.0 on gfx950: lerp, addcmul (fma(s, g*g, v)) and addcdiv
# (fma(s, m/d, p)) are fused multiply-adds; sqrt and division are correctly
# rounded; a tensor divided by a Python scalar c runs as a multiply by
# f32(1.0 / c) with the reciprocal taken in float64.  Pinned bit-for-bit by the
# GPU test tests/test_gpu_parity.py::test_torch_rocm_matches_oracle_opmodel.
OPMODEL_TORCH_ROCM = OpModel(lerp_fma=1, addcmul_mode=1, addcdiv_mode=1, div_recip=1)


class Capt(ctypes.Structure):
    """oracle_capt: the capturable chain's scalars (adamw_oracle.h)."""

    _fields_ = [
        ("wd_factor", ctypes.c_float),
        ("lerp_w", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("den_scale", ctypes.c_float),
        ("den_add", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
    ]


class FusedModel(ctypes.Structure):
    """oracle_fused_model: which float64 ``a*b + c*d`` of the fused=True chain is one
    fused multiply-add (adamw_oracle.h)."""

    _fields_ = [("wd_fma", ctypes.c_int), ("m_mode", ctypes.c_int), ("v_mode", ctypes.c_int)]

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"FusedModel(wd_fma={self.wd_fma}, m_mode={self.m_mode}, v_mode={self.v_mode})"


# torch 2.10.0+rocm7.0 on gfx950, torch._fused_adamw_ (fused_adam_utils.cuh adam_math):
# the compiler contracted each float64 sum with its left product, m = fma(beta1, m,
# (1-beta1)*g) and v = fma(beta2, v, ((1-beta2)*g)*g), and p - (lr*wd)*p into one fma.
# The m and v forms are pinned bit for bit by torch's GPU results on inputs where the
# three candidates round apart (tests/golden/fused_golden.npz, written by
# tests/golden/make_fused_golden.py from the cases fused_cases.c finds); the two forms
# of the weight-decay op give the same fp32 result for every fp32 p at lr*wd = 3e-5
# (none of 4e9 random draws separates them), so that field is not pinned by data.
FUSED_TORCH_ROCM = FusedModel(wd_fma=1, m_mode=1, v_mode=1)


class Fused(ctypes.Structure):
    """oracle_fused: the fused=True chain's scalars (adamw_oracle.h)."""

    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("step_size", ctypes.c_float),
        ("bc2_sqrt", ctypes.c_float),
        ("grad_sign", ctypes.c_float),
    ]


def _load(path: str = _LIB_PATH):
    if not os.path.exists(path):
        raise RuntimeError(f"oracle library missing: build it with `make -C {_HERE}`")
    lib = ctypes.CDLL(path)
    f32p = ctypes.POINTER(ctypes.c_float)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    i64 = ctypes.c_int64
    lib.oracle_adamw_f32.argtypes = [f32p, f32p, f32p, f32p, f32p, i64, ctypes.POINTER(Hyper),
                                     ctypes.POINTER(OpModel), ctypes.c_float, ctypes.c_int]
    lib.oracle_adamw_f32.restype = None
    lib.oracle_adamw_bf16state.argtypes = [f32p, f32p, u16p, u16p, u16p, i64,
                                           ctypes.POINTER(Hyper), ctypes.POINTER(OpModel),
                                           ctypes.c_float, ctypes.c_int]
    lib.oracle_adamw_bf16state.restype = None
    lib.oracle_capt_scalars.argtypes = [ctypes.c_float] * 5 + [ctypes.c_int, f32p, f32p]
    lib.oracle_capt_scalars.restype = None
    lib.oracle_adamw_capt_f32.argtypes = [f32p, f32p, f32p, f32p, f32p, i64,
                                          ctypes.POINTER(Capt), ctypes.POINTER(OpModel),
                                          ctypes.c_float, ctypes.c_int]
    lib.oracle_adamw_capt_f32.restype = None
    lib.oracle_adamw_capt_bf16state.argtypes = [f32p, f32p, u16p, u16p, u16p, i64,
                                                ctypes.POINTER(Capt), ctypes.POINTER(OpModel),
                                                ctypes.c_float, ctypes.c_int]
    lib.oracle_adamw_capt_bf16state.restype = None
    lib.oracle_fused_scalars.argtypes = [ctypes.c_double] * 3 + [ctypes.c_float, f32p, f32p,
                                                                  f32p]
    lib.oracle_fused_scalars.restype = None
    lib.oracle_fused_scalars_many.argtypes = [ctypes.c_double, ctypes.c_double, f32p, i64,
                                              f32p, f32p]
    lib.oracle_fused_scalars_many.restype = None
    lib.oracle_adamw_fused_f32.argtypes = [f32p, f32p, f32p, f32p, f32p, i64,
                                           ctypes.POINTER(Fused), ctypes.POINTER(FusedModel),
                                           ctypes.c_float, ctypes.c_int]
    lib.oracle_adamw_fused_f32.restype = None
    lib.oracle_adamw_fused_bf16state.argtypes = [f32p, f32p, u16p, u16p, u16p, i64,
                                                 ctypes.POINTER(Fused),
                                                 ctypes.POINTER(FusedModel), ctypes.c_float,
                                                 ctypes.c_int]
    lib.oracle_adamw_fused_bf16state.restype = None
    lib.oracle_to_bf16.argtypes = [f32p, u16p, i64]
    lib.oracle_to_bf16.restype = None
    lib.oracle_sumsq_f64.argtypes = [f32p, i64]
    lib.oracle_sumsq_f64.restype = ctypes.c_double
    lib.oracle_clip_coef.argtypes = [ctypes.c_float, ctypes.c_double]
    lib.oracle_clip_coef.restype = ctypes.c_float
    lib.oracle_max_ulp.argtypes = [f32p, f32p, i64, ctypes.POINTER(i64)]
    lib.oracle_max_ulp.restype = i64
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def use_library(path: str | None):
    """Point the wrappers at another build of adamw_oracle.c (None: the default).

    The mutation tests use this to run the oracle's own pinning checks against
    copies of the oracle with a planted mistake."""
    global _lib
    _lib = None if path is None else _load(path)


def _f32(a: np.ndarray):
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError("oracle expects C-contiguous float32 arrays")
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u16(a: np.ndarray):
    if a.dtype != np.uint16 or not a.flags.c_contiguous:
        raise TypeError("oracle expects C-contiguous uint16 (bf16 bit) arrays")
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


@dataclass
class GroupScalars:
    """Float64 host values of one step, before the casts to fp32."""

    step: float
    bias_correction1: float
    bias_correction2: float
    step_size: float
    bias_correction2_sqrt: float


def group_scalars(lr: float, beta1: float, beta2: float, step: float) -> GroupScalars:
    """adam.py:529-536 (the non-capturable branch): Python float64 arithmetic."""
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    step_size = lr / bc1
    bc2_sqrt = bc2 ** 0.5
    return GroupScalars(step, bc1, bc2, step_size, bc2_sqrt)


def hyper_from_group(lr, beta1, beta2, eps, weight_decay, step, maximize=False) -> Hyper:
    """Host scalars for step number ``step`` (the value after ``step_t += 1``).

    ``step`` is what ``_get_value(step_t)`` returns: the fp32 step tensor read
    back as a Python float (adam.py:414,529; optimizer.py:91-96).
    """
    s = group_scalars(float(lr), float(beta1), float(beta2), float(np.float32(step)))
    wd_factor = np.float32(1 - lr * weight_decay) if weight_decay != 0 else np.float32(1.0)
    return Hyper(
        wd_factor=float(wd_factor),
        lerp_w=float(np.float32(1 - beta1)),
        beta2=float(np.float32(beta2)),
        one_minus_beta2=float(np.float32(1 - beta2)),
        bc2_sqrt=s.bias_correction2_sqrt,
        eps=float(np.float32(eps)),
        neg_step_size=float(np.float32(-s.step_size)),
        grad_sign=-1.0 if maximize else 1.0,
    )


def adamw_step(p, g, m, v, *, lr, betas, eps, weight_decay, step, maximize=False,
               grad_scale=None, vmax=None, opmodel=OPMODEL_TORCH_ROCM) -> None:
    """One AdamW step on fp32 numpy arrays, in place (p, m, v; vmax with amsgrad)."""
    h = hyper_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize)
    n = p.size
    if not (g.size == m.size == v.size == n) or (vmax is not None and vmax.size != n):
        raise ValueError("p, g, m, v sizes differ")
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_f32(_f32(p), _f32(g), _f32(m), _f32(v),
                           None if vmax is None else _f32(vmax), n, ctypes.byref(h),
                           ctypes.byref(opmodel), scale, 0 if grad_scale is None else 1)


def adamw_step_bf16state(p, g, m_bits, v_bits, *, lr, betas, eps, weight_decay, step,
                         maximize=False, grad_scale=None, vmax_bits=None,
                         opmodel=OPMODEL_TORCH_ROCM) -> None:
    """AdamW step with bf16-stored moments (uint16 bit arrays), fp32 math."""
    h = hyper_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize)
    n = p.size
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_bf16state(_f32(p), _f32(g), _u16(m_bits), _u16(v_bits),
                                 None if vmax_bits is None else _u16(vmax_bits), n,
                                 ctypes.byref(h), ctypes.byref(opmodel), scale,
                                 0 if grad_scale is None else 1)


def capt_scalars(lr, beta1, beta2, eps, step, lr_is_tensor=False) -> tuple[float, float]:
    """(den_scale, den_add) of the capturable chain at step ``step`` (adam.py:480-522),
    fp32 with this C library's powf."""
    a, e = ctypes.c_float(), ctypes.c_float()
    lib().oracle_capt_scalars(float(np.float32(beta1)), float(np.float32(beta2)),
                              float(np.float32(lr)), float(np.float32(eps)),
                              float(np.float32(step)), 1 if lr_is_tensor else 0,
                              ctypes.byref(a), ctypes.byref(e))
    return a.value, e.value


def capt_from_group(lr, beta1, beta2, eps, weight_decay, step, maximize=False,
                    lr_is_tensor=False, den=None) -> Capt:
    """The capturable chain's scalars.  ``den``: (den_scale, den_add) formed
    elsewhere (torch's device values); otherwise ``capt_scalars``.  The
    weight-decay factor is Python float64 for a float lr and two fp32 tensor ops
    (``1 - lr * wd``) for a tensor lr."""
    f32 = np.float32
    if weight_decay == 0:
        wd_factor = f32(1.0)
    elif lr_is_tensor:
        wd_factor = f32(1) - f32(lr) * f32(weight_decay)
    else:
        wd_factor = f32(1 - lr * weight_decay)
    a, e = den if den is not None else capt_scalars(lr, beta1, beta2, eps, step, lr_is_tensor)
    return Capt(wd_factor=float(wd_factor), lerp_w=float(f32(1 - beta1)),
                beta2=float(f32(beta2)), one_minus_beta2=float(f32(1 - beta2)),
                den_scale=float(a), den_add=float(e), grad_sign=-1.0 if maximize else 1.0)


def adamw_step_capt(p, g, m, v, *, lr, betas, eps, weight_decay, step, maximize=False,
                    grad_scale=None, vmax=None, lr_is_tensor=False, den=None,
                    opmodel=OPMODEL_TORCH_ROCM) -> None:
    """One capturable-chain AdamW step on fp32 numpy arrays, in place."""
    h = capt_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize,
                        lr_is_tensor, den)
    n = p.size
    if not (g.size == m.size == v.size == n) or (vmax is not None and vmax.size != n):
        raise ValueError("p, g, m, v sizes differ")
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_capt_f32(_f32(p), _f32(g), _f32(m), _f32(v),
                                None if vmax is None else _f32(vmax), n, ctypes.byref(h),
                                ctypes.byref(opmodel), scale, 0 if grad_scale is None else 1)


def adamw_step_capt_bf16state(p, g, m_bits, v_bits, *, lr, betas, eps, weight_decay, step,
                              maximize=False, grad_scale=None, vmax_bits=None,
                              lr_is_tensor=False, den=None, opmodel=OPMODEL_TORCH_ROCM) -> None:
    """Capturable-chain step with bf16-stored moments (uint16 bit arrays), fp32 math."""
    h = capt_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize,
                        lr_is_tensor, den)
    n = p.size
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_capt_bf16state(_f32(p), _f32(g), _u16(m_bits), _u16(v_bits),
                                      None if vmax_bits is None else _u16(vmax_bits), n,
                                      ctypes.byref(h), ctypes.byref(opmodel), scale,
                                      0 if grad_scale is None else 1)


def fused_scalars(lr, beta1, beta2, step) -> tuple[float, float, float]:
    """(bc1, bc2_sqrt, step_size) of the fused=True chain at step ``step`` (the fp32
    count after its increment): float64 on the device in torch
    (fused_adam_utils.cuh FusedAdamMathFunctor), each reaching adam_math as fp32.
    libm's pow here; the device pow differs from it in the last float64 bit at some
    steps, which the fp32 roundings absorb (a GPU test compares the two)."""
    bc1, bc2s, ss = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
    lib().oracle_fused_scalars(float(lr), float(beta1), float(beta2),
                               float(np.float32(step)), ctypes.byref(bc1), ctypes.byref(bc2s),
                               ctypes.byref(ss))
    return bc1.value, bc2s.value, ss.value


def fused_scalars_many(beta1, beta2, steps) -> tuple[np.ndarray, np.ndarray]:
    """(bc1, bc2_sqrt) of ``fused_scalars`` for an array of fp32 step counts."""
    steps = np.ascontiguousarray(steps, dtype=np.float32)
    bc1 = np.empty_like(steps)
    bc2s = np.empty_like(steps)
    lib().oracle_fused_scalars_many(float(beta1), float(beta2), _f32(steps), steps.size,
                                    _f32(bc1), _f32(bc2s))
    return bc1, bc2s


def fused_from_group(lr, beta1, beta2, eps, weight_decay, step, maximize=False) -> Fused:
    """The fused chain's scalars: lr (a float, or a tensor lr's value as float64), the
    betas, weight decay and eps as float64, the per-step values from ``fused_scalars``."""
    _, bc2s, ss = fused_scalars(lr, beta1, beta2, step)
    return Fused(lr=float(lr), beta1=float(beta1), beta2=float(beta2),
                 weight_decay=float(weight_decay), eps=float(eps), step_size=ss,
                 bc2_sqrt=bc2s, grad_sign=-1.0 if maximize else 1.0)


def adamw_step_fused(p, g, m, v, *, lr, betas, eps, weight_decay, step, maximize=False,
                     grad_scale=None, vmax=None, model=FUSED_TORCH_ROCM) -> None:
    """One step of torch's fused=True chain on fp32 numpy arrays, in place."""
    h = fused_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize)
    n = p.size
    if not (g.size == m.size == v.size == n) or (vmax is not None and vmax.size != n):
        raise ValueError("p, g, m, v sizes differ")
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_fused_f32(_f32(p), _f32(g), _f32(m), _f32(v),
                                 None if vmax is None else _f32(vmax), n, ctypes.byref(h),
                                 ctypes.byref(model), scale, 0 if grad_scale is None else 1)


def adamw_step_fused_bf16state(p, g, m_bits, v_bits, *, lr, betas, eps, weight_decay, step,
                               maximize=False, grad_scale=None, vmax_bits=None,
                               model=FUSED_TORCH_ROCM) -> None:
    """The fused=True chain with bf16-stored moments (uint16 bit arrays)."""
    h = fused_from_group(lr, betas[0], betas[1], eps, weight_decay, step, maximize)
    n = p.size
    scale = 1.0 if grad_scale is None else float(np.float32(grad_scale))
    lib().oracle_adamw_fused_bf16state(_f32(p), _f32(g), _u16(m_bits), _u16(v_bits),
                                       None if vmax_bits is None else _u16(vmax_bits), n,
                                       ctypes.byref(h), ctypes.byref(model), scale,
                                       0 if grad_scale is None else 1)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_to_bf16(_f32(x), _u16(out), x.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def sumsq(grads) -> float:
    """Sum of squares of every gradient, float64 (exact squares, blocked sums)."""
    total = 0.0
    for g in grads:
        g = np.ascontiguousarray(g, dtype=np.float32).reshape(-1)
        total += lib().oracle_sumsq_f64(_f32(g), g.size)
    return total


def total_norm(grads) -> np.float32:
    """clip_grad.py:50-117 for norm_type 2: the L2 norm of all gradients as one vector."""
    return np.float32(math.sqrt(sumsq(grads)))


def clip_coef(norm, max_norm: float) -> np.float32:
    """clip_grad.py:165-169: clamp(max_norm * reciprocal(norm + 1e-6), max=1)."""
    return np.float32(lib().oracle_clip_coef(float(np.float32(norm)), float(max_norm)))


def max_ulp(a: np.ndarray, b: np.ndarray) -> tuple[int, int]:
    """(largest ulp distance, index of it) between two fp32 arrays."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    if a.size != b.size:
        raise ValueError("size mismatch")
    where = ctypes.c_int64(-1)
    d = lib().oracle_max_ulp(_f32(a), _f32(b), a.size, ctypes.byref(where))
    return int(d), int(where.value)
