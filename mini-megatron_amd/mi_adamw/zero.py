"""ZeRO-1 range sharding of a flat-layout FusedAdamW: each rank's contiguous slice.

mini-megatron's ZeRO-1 optimizer (parallel/distributed_optimizer.py:7-48) assigns whole
tensors to data-parallel ranks round-robin (``i % dp_size == dp_rank``, :20-23), steps a
per-rank ``torch.optim.AdamW`` over them (:25-29, :36-37) and broadcasts every tensor
from its owner afterwards (:39-44).  Before that, ``allreduce_grads``
(parallel/data_parallel.py:5-15) all-reduces every gradient and divides it by the world
size in place.

Range sharding replaces the tensor round-robin with a cut of the flat buffers
(``FusedAdamW(flat_buffer=True)``): rank r owns one contiguous, 128-byte-aligned slice
``[lo_r, hi_r)`` of every buffer, which may cut through tensors and param groups.  The
elementwise step does not care where a tensor ends, so a rank runs the same kernels on
its slice, each piece with its param group's hyperparameters.  The global gradient clip
splits at the one exchange it needs: each rank sums the squares of its slice's
gradients into one float64 (``grad_sumsq``), the ranks' sums are combined (an 8-byte
all-reduce across GPUs), and every rank forms the same norm and coefficient from the
total (``finalize``).  The world-size division of ``allreduce_grads`` becomes a
gradient pre-scale inside both kernels (``grad_prescale``), so the gradients are read
once per pass and never rewritten.

On one GPU, ``ZeroRangeStep.step()`` runs every rank's part in sequence on the one
optimizer's buffers: all partial sums, the finalize, then every slice's update.  That
is the kernel work of each rank at its real shape; what it leaves out are the
collectives (reduce-scatter of the gradients before, the 8-byte all-reduce in the
middle, all-gather of the bf16 or fp32 parameters after).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .flat import ALIGN_ELEMS


def shard_bounds(total: int, world: int, align: int = ALIGN_ELEMS) -> list[tuple[int, int]]:
    """Contiguous [lo, hi) slices of `total` elements for `world` ranks: boundaries at
    multiples of `align` elements, sizes within `align` of each other (the last rank
    absorbs a ragged end)."""
    if world < 1:
        raise ValueError(f"world must be >= 1, got {world}")
    units = -(-total // align)
    cuts = [min(total, (r * units // world) * align) for r in range(world)] + [total]
    return [(cuts[r], cuts[r + 1]) for r in range(world)]


class _BeginPlan:
    """The native plan of ZeroRangeStep.begin() and what it was made from."""
    __slots__ = ("plan", "steps", "state", "groups_key", "hyper_steps", "row", "nonempty")

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)


def dp_prescale(world: int) -> float:
    """The fp32 factor that ``grad.div_(world)`` multiplies by on the GPU: torch divides a
    tensor by a host scalar as a multiply by the reciprocal, rounded to fp32."""
    return float(np.float32(1.0 / world))


class ZeroRangeStep:
    """Drive a flat-layout FusedAdamW as `world` ZeRO-1 ranks, one contiguous slice each.

    Methods follow one step of one rank:
      ``begin()``                    once per step: every step count +1, per-group scalars;
      ``grad_sumsq(rank, out)``      the rank's float64 sum of squares (clip only);
      ``finalize(sumsq)``            norm and coefficient from the ranks' sums;
      ``update(rank, hypers, coef)`` the AdamW update of the rank's slice.
    ``step()`` runs them for every rank in turn on one GPU.

    ``grad_prescale``: the factor every gradient is multiplied by in both kernels (the
    world-size division of ``allreduce_grads``).  None takes the optimizer's own
    ``grad_prescale``, so ``step()`` here and ``opt.step()`` see the same gradients.  An
    explicit value that differs from a pre-scale the optimizer was built with raises;
    over an optimizer without one (1) it applies to the ranks' kernels only.
    """

    def __init__(self, opt, world: int, grad_prescale: float | None = None):
        flat = getattr(opt, "_flat", None)
        if flat is None:
            raise ValueError("ZeroRangeStep needs FusedAdamW(flat_buffer=True)")
        if opt.capturable:
            raise NotImplementedError("ZeroRangeStep: capturable=True is not supported")
        own = float(opt.grad_prescale)
        if grad_prescale is None:
            grad_prescale = own
        elif own != 1.0 and float(np.float32(grad_prescale)) != own:
            raise ValueError(f"ZeroRangeStep: grad_prescale={grad_prescale} differs from the "
                             f"optimizer's grad_prescale={own}")
        self.opt = opt
        self.flat = flat
        self.world = int(world)
        self.grad_prescale = float(np.float32(grad_prescale))
        self.bounds = shard_bounds(flat.total, self.world)
        self._sumsq = torch.zeros(max(self.world, 1), dtype=torch.float64, device=flat.device)
        self._coef = torch.ones(1, dtype=torch.float32, device=flat.device)
        self._plan = None       # the native checks of begin(), made by a begin() in Python
        self.native_begins = 0

    def _make_plan(self, stream: int) -> None:
        """The native host path's plan for the checks and the step counting of begin():
        every parameter's storage, gradient view (which must stay where it is) and state
        entries, one step count per param group.  Its launch fields are unused (begin()
        launches nothing)."""
        opt = self.opt
        self._plan = None
        steps = opt._steps
        if not steps.is_contiguous() or steps.device.type != "cpu":
            return
        entries = [(gi, p) for gi, g in enumerate(opt.param_groups) for p in g["params"]]
        n = len(entries)
        hyper_steps = np.zeros(max(len(opt.param_groups), 1), dtype=np.float64)
        row = _lib.TensorRow()
        try:
            plan = _lib.host().plan(
                [p for _, p in entries], [opt.state[p] for _, p in entries],
                [opt._slots[id(p)] for _, p in entries], [gi for gi, _ in entries],
                [-2] * n, [True] * n, [p.grad.data_ptr() for _, p in entries], False,
                (steps.data_ptr(), steps.numel()), (hyper_steps.ctypes.data, len(hyper_steps)),
                (False, 0, 0, 0, 0, 0, ctypes.addressof(row), 0),
                (0, 0, 0, 0, False, 0.0, 1.0, 0, 0, 0, int(stream), False),
                (steps, hyper_steps, row))
        except (TypeError, ValueError):
            return
        self._plan = _BeginPlan(plan=plan, steps=steps, state=opt.state,
                                groups_key=opt._groups_key(), hyper_steps=hyper_steps, row=row,
                                nonempty=[bool(g["params"]) for g in opt.param_groups])

    def _native_begin(self):
        """begin() through the native checks, or None when the Python begin() must run."""
        opt = self.opt
        pl = self._plan
        # the plan points into the step buffer and holds the state dicts it was made from
        if (pl is None or pl.steps is not opt._steps or pl.state is not opt.state
                or pl.groups_key != opt._groups_key()):
            return None
        host = _lib._host
        if host.prepare(pl.plan, self._stream()) != host.READY:
            return None
        self.native_begins += 1
        return [self._group_hyper(g, float(pl.hyper_steps[gi])) if nonempty else None
                for gi, (g, nonempty) in enumerate(zip(opt.param_groups, pl.nonempty))]

    def _group_hyper(self, group: dict, step: float):
        """The group's set at step `step`: torch's fused=True chain for a fused group, the
        default chain otherwise (as FusedAdamW.step takes them)."""
        from .optimizer import _fused_hyper, _hyper
        if group["fused"]:
            return _fused_hyper(group, step, self.flat.device)
        return _hyper(group, step)

    def segments(self, rank: int) -> list[tuple[int, int, int]]:
        """(param group, lo, hi) pieces of rank's slice, one per group it overlaps."""
        lo, hi = self._bounds(rank)
        out = []
        for gi, (a, b) in enumerate(self.flat.group_ranges):
            s, e = max(lo, a), min(hi, b)
            if s < e:
                out.append((gi, s, e))
        return out

    @torch.no_grad()
    def begin(self) -> list:
        """Advance every parameter's step count by one (each rank keeps the same count) and
        return one hyperparameter set per param group (an mi_adamw_hyper, or for a group
        with fused=True an mi_adamw_fused_hyper).  Every parameter must have its
        gradient view and all parameters of a group one step count, as in the flat step.
        After the first call, the checks and the counting run natively while nothing they
        cover changed; any change (a replaced tensor, a moved gradient, a new group, a loaded
        checkpoint) takes this Python body, which handles it and makes a new plan."""
        hypers = self._native_begin()
        if hypers is not None:
            return hypers
        opt = self.opt
        steps = opt._steps_for(self.flat.device)
        group_slots = []
        for group in opt.param_groups:
            if group["amsgrad"]:
                raise NotImplementedError("ZeroRangeStep: amsgrad is not supported")
            for p in group["params"]:
                if p.grad is None or not self.flat.is_grad_view(p, p.grad):
                    raise RuntimeError("ZeroRangeStep: every parameter needs its gradient view "
                                       "of the flat buffer (zero_grad() keeps them)")
        for group in opt.param_groups:
            slots = []
            for p in group["params"]:
                if not self.flat.is_param_view(p):
                    self.flat.absorb_param(p)          # p.data was replaced
                slot = opt._slots[id(p)]
                st = opt.state[p]
                if len(st) == 0:
                    opt._init_state(p, st, False)
                else:
                    if st["step"] is not opt._step_views[slot]:
                        opt._adopt_step(p, st, slot)
                    self.flat.absorb_state(p, st)      # moments put into the dict directly
                slots.append(slot)
            group_slots.append(torch.as_tensor(slots, dtype=torch.long))
        for idx in group_slots:
            if idx.numel() and bool((steps[idx] != steps[idx[0]]).any()):
                raise RuntimeError("ZeroRangeStep: a param group's parameters have different "
                                   "step counts")
        hypers = []
        for group, idx in zip(opt.param_groups, group_slots):
            if idx.numel() == 0:
                hypers.append(None)
                continue
            steps[idx] += 1
            hypers.append(self._group_hyper(group, float(steps[idx[0]])))
        self._make_plan(self._stream())
        return hypers

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.flat.device).cuda_stream

    def _bounds(self, rank: int) -> tuple[int, int]:
        if not 0 <= rank < self.world:
            raise ValueError(f"rank must be in [0, {self.world}), got {rank}")
        return self.bounds[rank]

    def _device_buffer(self, t: torch.Tensor, dtype: torch.dtype, what: str) -> None:
        # the kernels read or write t's memory as `dtype` elements from its first one
        if (not isinstance(t, torch.Tensor) or t.dtype != dtype or t.device != self.flat.device
                or t.numel() < 1 or not t.is_contiguous()):
            raise ValueError(f"{what} must be a contiguous {dtype} tensor of at least one "
                             f"element on {self.flat.device}")

    def grad_sumsq(self, rank: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """The float64 sum of squares of rank's pre-scaled gradients, written to out[0]
        (default: entry `rank` of this object's buffer of one sum per rank)."""
        lib = _lib.load()
        lo, hi = self._bounds(rank)
        if out is None:
            out = self._sumsq[rank:rank + 1]
        self._device_buffer(out, torch.float64, "grad_sumsq: out")
        partials, _ = self.opt._ws(self.flat.device)
        with torch.cuda.device(self.flat.device):
            if hi <= lo:
                out[:1].zero_()
                return out
            _lib.check(lib.mi_adamw_grad_sumsq_flat(
                self.flat.grad.data_ptr() + 4 * lo, hi - lo, self.opt.chunk_elems,
                self.grad_prescale, partials.data_ptr(), out.data_ptr(), self._stream()),
                "mi_adamw_grad_sumsq_flat")
        return out

    def finalize(self, sumsq: torch.Tensor, max_norm: float | None = None):
        """(norm, coefficient) as 0-d / 1-element device tensors from the ranks' sums,
        added in rank order."""
        lib = _lib.load()
        self._device_buffer(sumsq, torch.float64, "finalize: sumsq")
        max_norm = self.opt.max_grad_norm if max_norm is None else max_norm
        if max_norm is None:
            raise ValueError("finalize: no max_norm (the optimizer has max_grad_norm=None)")
        norm = torch.empty((), dtype=torch.float32, device=self.flat.device)
        with torch.cuda.device(self.flat.device):
            _lib.check(lib.mi_adamw_norm_from_sumsq(
                sumsq.data_ptr(), sumsq.numel(), float(max_norm), norm.data_ptr(),
                self._coef.data_ptr(), self._stream()), "mi_adamw_norm_from_sumsq")
        return norm, self._coef

    def update(self, rank: int, hypers, coef: torch.Tensor | None = None) -> None:
        """The AdamW update of rank's slice: one launch per param group it overlaps."""
        lib = _lib.load()
        opt, flat = self.opt, self.flat
        flags = 0
        if opt.bf16_copy:
            flags |= _lib.F_BF16_COPY
        if coef is not None:
            self._device_buffer(coef, torch.float32, "update: coef")
            flags |= _lib.F_CLIP
            if opt.clip_write_grads:
                flags |= _lib.F_WRITE_GRAD
        state = _lib.STATE_BF16 if opt.state_dtype == torch.bfloat16 else _lib.STATE_F32
        s_item = flat.exp_avg.element_size()
        with torch.cuda.device(flat.device):
            stream = self._stream()
            for gi, lo, hi in self.segments(rank):
                row = _lib.TensorRow(
                    param=flat.param.data_ptr() + 4 * lo, grad=flat.grad.data_ptr() + 4 * lo,
                    exp_avg=flat.exp_avg.data_ptr() + s_item * lo,
                    exp_avg_sq=flat.exp_avg_sq.data_ptr() + s_item * lo,
                    param_copy=0 if flat.copy is None else flat.copy.data_ptr() + 2 * lo,
                    max_exp_avg_sq=0, numel=hi - lo, hyper=0, flags=_lib.T_VEC)
                h = hypers[gi]
                fused = isinstance(h, _lib.FusedHyper)
                fn = (lib.mi_adamw_step_flat_fused_chain if fused
                      else lib.mi_adamw_step_flat_prescaled)
                _lib.check(fn(ctypes.byref(row), ctypes.byref(h),
                              None if coef is None else coef.data_ptr(), self.grad_prescale,
                              opt.chunk_elems, state, flags, opt.max_blocks, stream),
                           "mi_adamw_step_flat_fused_chain" if fused
                           else "mi_adamw_step_flat_prescaled")

    @torch.no_grad()
    def step(self):
        """One optimizer step as `world` ranks would take it, every rank's kernels in turn
        on this GPU.  Returns the clip norm (0-d device tensor) or None without the clip."""
        hypers = self.begin()
        coef = None
        norm = None
        if self.opt.max_grad_norm is not None:
            for r in range(self.world):
                self.grad_sumsq(r)
            norm, coef = self.finalize(self._sumsq[:self.world])
            self.opt.last_grad_norm = norm
        for r in range(self.world):
            self.update(r, hypers, coef)
        if self.opt._copy_sync is not None:
            # the update wrote every master's bf16 copy
            for group in self.opt.param_groups:
                for p in group["params"]:
                    self.opt._copy_sync[id(p)] = (p._version, p.data_ptr())
        return norm
