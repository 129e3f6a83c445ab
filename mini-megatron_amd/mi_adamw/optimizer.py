"""FusedAdamW: a drop-in torch.optim.AdamW whose step is one HIP launch (two with clip).

Reference interface.  mini-megatron builds ``torch.optim.AdamW(params,
lr=LEARNING_RATE, weight_decay=WEIGHT_DECAY, fused=args.fused)`` (main.py:144,
main.py:177), drives ``group["lr"]`` through LambdaLR (main.py:178-180), calls
``zero_grad()`` and ``step()`` once per iteration (main.py:204,209;
parallel/pipeline_parallel.py:219-220,260), reads ``param_groups[0]["params"]``
(parallel/pipeline_parallel.py:219) and checkpoints ``state_dict()``
(checkpoint.py:9,19).  Without ``--fused`` that AdamW runs torch's
``_single_tensor_adam`` (torch/optim/adam.py:347-551): 8 ATen kernels per
parameter tensor.  FusedAdamW keeps the constructor, ``param_groups``,
``state`` layout, ``state_dict`` format and ``step()`` semantics of
``torch.optim.AdamW`` (torch/optim/adamw.py:21-49, adam.py:35-272) and
replaces the per-tensor loop with the kernels of libmi_adamw:

* ``mi_adamw_grad_norm`` -- optional global gradient-norm clip (config.py:16
  names MAX_GRAD_NORM; torch/nn/utils/clip_grad.py:186-233), computed and
  applied on the device with no host synchronisation;
* ``mi_adamw_step`` / ``mi_adamw_step_flat`` -- the AdamW update of every
  tensor, with fp32 or bf16 moments, an optional bf16 model copy and amsgrad's
  running maximum (adam.py:538-543) for the groups that set it;
* ``mi_adamw_step_capturable_rows`` -- the same update in torch's capturable
  chain (capturable=True): step counts on the device, the per-step scalars
  formed on the device (once per tensor, by a launch before the update), so
  that step() can be recorded into a HIP graph.

Per-element results match ``torch.optim.AdamW(foreach=False)`` on the same GPU
tensors: the kernels follow the fp32 op chain and the fused multiply-adds of
torch-ROCm's ATen kernels, and the per-step scalars below are computed on the
host in float64 exactly as adam.py:414-536 computes them (with
capturable=True: on the device in fp32, as adam.py:480-527 does).
"""
from __future__ import annotations

import ctypes
from typing import Any

import numpy as np
import torch
from torch.optim import Optimizer
from torch.optim.optimizer import _device_dtype_check_for_fused

from . import _lib
from .flat import FlatLayout

DEFAULT_CHUNK_ELEMS = 4096

_ROW_DTYPE = np.dtype([
    ("param", "<u8"), ("grad", "<u8"), ("exp_avg", "<u8"), ("exp_avg_sq", "<u8"),
    ("param_copy", "<u8"), ("max_exp_avg_sq", "<u8"), ("numel", "<i8"), ("hyper", "<i4"),
    ("flags", "<i4"),
])
assert _ROW_DTYPE.itemsize == 64


def _hyper(group: dict, step: float) -> _lib.Hyper:
    """The fp32 scalars one (group, step) hands the kernel.

    adam.py:414-536 in the non-capturable branch: lr, betas and the step count
    are Python floats; bias corrections, step size and ``bc2 ** 0.5`` are
    float64; each scalar reaches its ATen kernel cast to fp32, and the division
    of ``sqrt(v)`` by the host scalar ``bc2_sqrt`` runs on the GPU as a multiply
    by the reciprocal taken in float64.  A tensor lr stays a tensor in torch
    (optimizer.py ``_to_scalar`` only squeezes it), so ``1 - lr * wd`` and
    ``lr / bc1`` are then tensor ops in lr's dtype; they are evaluated here with
    the same torch ops on the CPU.
    """
    lr = group["lr"]
    beta1, beta2 = (float(b) for b in group["betas"])
    wd = group["weight_decay"]
    bias_correction1 = 1 - beta1 ** step
    bias_correction2 = 1 - beta2 ** step
    bias_correction2_sqrt = bias_correction2 ** 0.5
    f32 = np.float32
    if isinstance(lr, torch.Tensor):
        lr_t = lr.detach().reshape(()).cpu()
        wd_factor = float(f32((1 - lr_t * wd).item())) if wd != 0 else 1.0
        neg_step_size = float(f32((-(lr_t / bias_correction1)).item()))
    else:
        lr = float(lr)
        wd_factor = float(f32(1 - lr * wd)) if wd != 0 else 1.0
        neg_step_size = float(f32(-(lr / bias_correction1)))
    return _lib.Hyper(
        wd_factor=wd_factor,
        lerp_w=float(f32(1 - beta1)),
        beta2=float(f32(beta2)),
        one_minus_beta2=float(f32(1 - beta2)),
        inv_bc2_sqrt=float(f32(1.0 / bias_correction2_sqrt)),
        eps=float(f32(group["eps"])),
        neg_step_size=neg_step_size,
        grad_sign=-1.0 if group["maximize"] else 1.0,
    )


def _capt_hyper(group: dict, device: torch.device) -> _lib.CaptHyper:
    """The fp32 constants of one group for the capturable chain (adam.py:396-527 with
    capturable=True).  Nothing depends on the step count, which the kernel reads
    from the device.  A float lr enters ``lr / bias_correction1`` as
    ``bc1.reciprocal() * lr`` (Tensor.__rtruediv__); a tensor lr as a true
    division, read by the kernel when it lives on the device."""
    lr = group["lr"]
    beta1, beta2 = (float(b) for b in group["betas"])
    wd = float(group["weight_decay"])
    f32 = np.float32
    h = _lib.CaptHyper(
        beta1=float(f32(beta1)), beta2=float(f32(beta2)), lerp_w=float(f32(1 - beta1)),
        one_minus_beta2=float(f32(1 - beta2)), eps=float(f32(group["eps"])),
        grad_sign=-1.0 if group["maximize"] else 1.0, lr=0.0, wd_factor=1.0, weight_decay=0.0,
        lr_mode=_lib.LR_FLOAT, lr_ptr=None)
    if not isinstance(lr, torch.Tensor):
        h.lr = float(f32(lr))
        h.wd_factor = float(f32(1 - float(lr) * wd)) if wd != 0 else 1.0
    elif lr.device.type == "cpu":
        lr_t = lr.detach().reshape(())
        if lr_t.dtype != torch.float32:
            raise NotImplementedError("FusedAdamW(capturable=True): a tensor lr must be float32")
        h.lr_mode = _lib.LR_VALUE
        h.lr = float(lr_t.item())
        h.wd_factor = float(f32((1 - lr_t * wd).item())) if wd != 0 else 1.0
    else:
        if lr.dtype != torch.float32 or lr.device != device or lr.numel() != 1:
            raise NotImplementedError("FusedAdamW(capturable=True): a device lr must be a "
                                      "one-element float32 tensor on the parameters' device")
        h.lr_mode = _lib.LR_DEVICE
        h.lr_ptr = lr.data_ptr()
        h.weight_decay = float(f32(wd))
    return h


def _fused_hyper(group: dict, step: float, device: torch.device) -> _lib.FusedHyper:
    """One group's set for torch's fused=True chain (adam.py:803-895 -> _fused_adamw_).

    The hyperparameters go in as the float64 values that op receives; ``step`` is the
    count after this step's increment (unused when the launch reads device step counts).
    A tensor lr: on the CPU, its value as a float64 (the op's tensor-lr overload takes
    ``lr.item()``); on the parameters' device, a one-element fp32 tensor read by the
    kernel (the op reads it as fp32 there)."""
    lr = group["lr"]
    beta1, beta2 = (float(b) for b in group["betas"])
    h = _lib.FusedHyper(lr=0.0, beta1=beta1, beta2=beta2,
                        weight_decay=float(group["weight_decay"]), eps=float(group["eps"]),
                        step=float(np.float32(step)),
                        grad_sign=-1.0 if group["maximize"] else 1.0, lr_ptr=None)
    if not isinstance(lr, torch.Tensor):
        h.lr = float(lr)
    elif lr.device.type == "cpu":
        h.lr = float(lr.item())
    else:
        if lr.dtype != torch.float32 or lr.device != device or lr.numel() != 1:
            raise NotImplementedError("FusedAdamW(fused=True): a device lr must be a one-element "
                                      "float32 tensor on the parameters' device")
        h.lr_ptr = lr.data_ptr()
    return h


def _refuse_under_capture(what: str) -> None:
    """Host-to-device uploads cannot be recorded into a graph: a step under capture
    must find everything an earlier eager step built."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"FusedAdamW: step() under graph capture, but {what} since the "
                           "last eager step; run one eager step with the same parameters and "
                           "gradient tensors before capturing")


def _ptr(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def _record(ev, i: int) -> None:
    """Record event i of a timing_events tuple, unless the tuple or that entry is None."""
    if ev is not None and ev[i] is not None:
        ev[i].record()


def _layout(t: torch.Tensor | None) -> tuple:
    """What a table row takes from a state tensor: its address, and that it is dense with
    this many elements."""
    return (0, 0, True) if t is None else (t.data_ptr(), t.numel(), t.is_contiguous())


class _Rec:
    """One parameter's bookkeeping: group index, the parameter, its step slot, its state dict."""

    __slots__ = ("gi", "p", "slot", "st")

    def __init__(self, gi: int, p: torch.Tensor, slot: int):
        self.gi = gi
        self.p = p
        self.slot = slot
        self.st = None


def _upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """A host array as a new device tensor, copied from pinned memory without blocking
    the host: the copy is ordered on the current stream, before the launches that
    read it, and torch keeps the pinned block until the copy has run.  (A CPU device,
    where only the host-side table logic runs, gets a plain copy.)"""
    host = torch.from_numpy(arr.view(np.uint8))
    if device.type != "cuda":
        return host.clone()
    return host.pin_memory().to(device, non_blocking=True)


class _Launch:
    """Device-resident tensor and chunk tables for one kernel launch."""

    __slots__ = ("rows", "chunks", "n_chunks", "n_rows", "host_rows", "tables", "src", "rest",
                 "step_index", "row_scalars")

    def __init__(self, rows: np.ndarray, chunk_elems: int, device: torch.device,
                 tables: bool = False, src: np.ndarray | None = None,
                 rest: np.ndarray | None = None, step_slots: np.ndarray | None = None):
        lib = _lib.load()
        self.n_rows = len(rows)
        # capturable launches: row i's index into the device step buffer, and the device
        # memory in which a step forms each row's per-step values before the update
        # (mi_adamw_step_capturable_rows), allocated here, never under graph capture
        self.step_index = (None if step_slots is None else
                           _upload(np.ascontiguousarray(step_slots, dtype=np.int32), device))
        self.row_scalars = (None if step_slots is None else
                            torch.empty(self.n_rows * _lib.ROW_SCALAR_BYTES, dtype=torch.uint8,
                                        device=device))
        self.host_rows = rows.copy()
        self.tables = tables or len(rows) != 1
        # src[i]: the entry whose gradient row i points at (-1: a flat group row, whose
        # gradient buffer never moves); rest[i]: row i's other pointers are aligned
        self.src = src
        self.rest = rest
        if not self.tables:
            # One contiguous range: launched through the flat entry points,
            # which derive chunk bounds arithmetically and need no tables.
            self.n_chunks = -(-int(rows["numel"][0]) // chunk_elems)
            self.rows = self.chunks = None
            return
        numels = np.ascontiguousarray(rows["numel"], dtype=np.int64)
        n = lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), chunk_elems, None, 0)
        _lib.check(int(n) if n < 0 else 0, "mi_adamw_build_chunks")
        chunks = np.empty(max(int(n), 1) * 2, dtype=np.int32)
        n2 = lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), chunk_elems,
                                       chunks.ctypes.data, int(n))
        if n2 != n:
            raise _lib.MiAdamwError("mi_adamw_build_chunks: inconsistent chunk count")
        self.n_chunks = int(n)
        self.rows = _upload(self.host_rows, device)
        self.chunks = _upload(chunks, device)

    def set_rows(self, rows: np.ndarray, device: torch.device) -> bool:
        """New pointers for the same tensors (the gradients moved): replace the rows,
        keep the chunk table.  False if the tensor sizes differ (rebuild instead)."""
        if len(rows) != self.n_rows or not np.array_equal(rows["numel"], self.host_rows["numel"]):
            return False
        self.host_rows = rows.copy()
        if self.tables:
            # a new buffer: a launch still queued on another stream keeps reading the old one
            self.rows = _upload(self.host_rows, device)
        return True

    def patch_grads(self, grads: np.ndarray, device: torch.device) -> None:
        """The gradients moved: write their addresses (grads[src[i]] for row i) into
        the rows and recompute the alignment flag; everything else stays."""
        rows = self.host_rows.copy()
        m = self.src >= 0
        g = grads[self.src[m]]
        rows["grad"][m] = g
        rows["flags"][m] = np.where(self.rest[m] & (g % 16 == 0), _lib.T_VEC, 0)
        self.host_rows = rows
        if self.tables:
            self.rows = _upload(rows, device)


class _LaunchCache:
    """The general path's launches, reused while `sig` (parameter and state pointers, the
    hyperparameter grouping, the amsgrad settings) and the device are unchanged.  `grads`
    are the gradient pointers the launch tables hold, or None after the native path
    patched the tables itself.  A new object replaces it whenever the general path
    rewrites the tables, so that a native plan made from the old one no longer applies."""

    __slots__ = ("sig", "device", "launches", "norm_launch", "grads")

    def __init__(self, sig, device, launches, norm_launch, grads):
        self.sig, self.device, self.launches = sig, device, launches
        self.norm_launch, self.grads = norm_launch, grads


class _Fast:
    """What the native host path needs to take the next steps: the plan (_host.plan) and
    the Python objects whose identity says the plan still describes this optimizer."""

    __slots__ = ("plan", "cache", "steps", "state", "groups_key", "options", "hyper_group",
                 "hyper_steps", "harr", "harr_addr", "clip", "device", "dev_index", "fused")


class FusedAdamW(Optimizer):
    """AdamW with the whole step fused into one MI355X kernel launch (three with the
    global-norm clip: sum of squares, finalize, update).

    The constructor takes torch.optim.AdamW's arguments, with its defaults and
    its ValueError checks (amsgrad and maximize work as in torch).  With
    capturable=True the step counts live on the device and the step follows
    torch's capturable op chain, so that step() can be recorded into a HIP
    graph (torch.cuda.graph) once an eager step has built the launch tables;
    results match torch.optim.AdamW(capturable=True, foreach=False).  Plus
    keyword-only options:

    max_grad_norm:    if set, clip the global gradient L2 norm to this value
                      before the update, as ``torch.nn.utils.clip_grad_norm_``
                      would, fused into the step (the norm of the last step is
                      kept in ``last_grad_norm``, a 0-d device tensor).
    clip_write_grads: with max_grad_norm, also store the clipped gradients back
                      into ``p.grad`` (clip_grad_norm_ does; costs 4 B/param).
    state_dtype:      torch.float32 (default) or torch.bfloat16 for exp_avg and
                      exp_avg_sq; the math stays fp32 and stores round to
                      nearest even.
    bf16_copy:        keep a bf16 copy of every parameter, written by the step
                      (``bf16_params()`` lists them in param order).
    flat_buffer:      pack every parameter, gradient and moment into flat
                      buffers (each tensor at a 128-byte-aligned offset) and
                      step each param group as one contiguous range.  Gradients
                      stay allocated: zero_grad() zeroes them in place.
    chunk_elems:      elements per work chunk (multiple of 4096).
    grad_prescale:    multiply every gradient by this fp32 factor first, in the
                      kernels (one rounding, as ``grad.div_(world)`` stores it):
                      with ``dp_prescale(world)`` it takes the place of the
                      world-size division of parallel/data_parallel.py:15 after
                      a summing all-reduce.  ``p.grad`` is left as it was (with
                      clip_write_grads the stored gradient is the pre-scaled,
                      clipped one).
    place_trials:     if > 0, run ``place_buffers(place_trials)`` once, after
                      the first step: the streams the update writes move to the
                      fastest of up to this many more allocations (report in
                      ``placement``).  State created later (a parameter without
                      a gradient at that step) keeps its own allocation.

    Not supported (NotImplementedError at construction): differentiable, betas
    as tensors, param groups with different capturable settings, place_trials
    with amsgrad.
    """

    def __init__(
        self,
        params,
        lr: float | torch.Tensor = 1e-3,
        betas: tuple[float | torch.Tensor, float | torch.Tensor] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
        amsgrad: bool = False,
        *,
        maximize: bool = False,
        foreach: bool | None = None,
        capturable: bool = False,
        differentiable: bool = False,
        fused: bool | None = None,
        max_grad_norm: float | None = None,
        clip_write_grads: bool = False,
        state_dtype: torch.dtype = torch.float32,
        bf16_copy: bool = False,
        flat_buffer: bool = False,
        chunk_elems: int = DEFAULT_CHUNK_ELEMS,
        grad_prescale: float = 1.0,
        place_trials: int = 0,
    ) -> None:
        # adam.py:58-86, in the same order and with the same messages.
        if isinstance(lr, torch.Tensor):
            if foreach and not capturable:
                raise ValueError(
                    "lr as a Tensor is not supported for capturable=False and foreach=True")
            if lr.numel() != 1:
                raise ValueError("Tensor lr must be 1-element")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if not ((isinstance(betas[0], float) and isinstance(betas[1], float))
                or (isinstance(betas[0], torch.Tensor) and isinstance(betas[1], torch.Tensor))):
            raise ValueError("betas must be either both floats or both Tensors")
        for i, b in enumerate(betas):
            if isinstance(b, torch.Tensor):
                if not capturable and foreach:
                    raise ValueError(f"betas[{i}] as a Tensor is not supported for "
                                     "capturable=False and foreach=True")
                if b.numel() != 1:
                    raise ValueError(f"Tensor betas[{i}] must be 1-element")
        if any(isinstance(b, torch.Tensor) for b in betas):
            raise NotImplementedError("FusedAdamW: betas as Tensors are not supported "
                                      "(torch steps them through tensor-weight kernels)")
        if fused and differentiable:
            raise RuntimeError("`fused` does not support `differentiable`")
        if fused and foreach:
            raise RuntimeError("`fused` and `foreach` cannot be `True` together.")
        if differentiable:
            raise NotImplementedError("FusedAdamW: differentiable=True is not supported")
        if max_grad_norm is not None and not max_grad_norm > 0:
            raise ValueError(f"Invalid max_grad_norm: {max_grad_norm}")
        if state_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"state_dtype must be torch.float32 or torch.bfloat16, got {state_dtype}")
        if chunk_elems <= 0 or chunk_elems % _lib.CHUNK_QUANTUM:
            raise ValueError(f"chunk_elems must be a positive multiple of {_lib.CHUNK_QUANTUM}")
        grad_prescale = float(np.float32(grad_prescale))
        if not (np.isfinite(grad_prescale) and grad_prescale > 0):
            raise ValueError(f"Invalid grad_prescale: {grad_prescale}")
        if capturable and grad_prescale != 1.0:
            raise NotImplementedError("FusedAdamW: grad_prescale with capturable=True is not "
                                      "supported")
        if not isinstance(place_trials, int) or place_trials < 0:
            raise ValueError(f"Invalid place_trials: {place_trials}")
        if place_trials and amsgrad:
            raise NotImplementedError("FusedAdamW: place_trials with amsgrad=True is not "
                                      "supported")

        self.capturable = bool(capturable)
        self.max_grad_norm = None if max_grad_norm is None else float(max_grad_norm)
        self.clip_write_grads = bool(clip_write_grads)
        self.state_dtype = state_dtype
        self.bf16_copy = bool(bf16_copy)
        self.flat_buffer = bool(flat_buffer)
        self.chunk_elems = int(chunk_elems)
        self.grad_prescale = grad_prescale
        self.place_trials = place_trials
        self.max_blocks = 0
        self._reset_bookkeeping()

        defaults = dict(
            lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
            maximize=maximize, foreach=foreach, capturable=capturable,
            differentiable=differentiable, fused=fused, decoupled_weight_decay=True,
        )
        # add_param_group (called by the base constructor) checks and registers every
        # parameter, and makes the per-parameter bf16 copies unless the flat layout
        # holds them
        super().__init__(params, defaults)
        self.register_load_state_dict_post_hook(FusedAdamW._after_load_state_dict)
        if self.flat_buffer:
            self._flat = FlatLayout(self.param_groups, self.state_dtype, self.bf16_copy)

    _OPTIONS = ("capturable", "max_grad_norm", "clip_write_grads", "state_dtype", "bf16_copy",
                "flat_buffer", "chunk_elems", "grad_prescale", "max_blocks", "place_trials")

    def _reset_bookkeeping(self) -> None:
        """The state this class keeps beside torch's: step slots, the packed step buffer,
        bf16 copies, launch tables, workspaces."""
        self.last_grad_norm: torch.Tensor | None = None
        self._slots: dict[int, int] = {}
        self._steps = torch.zeros(0, dtype=torch.float32)
        self._step_views: list[torch.Tensor | None] = []
        self._copies: dict[int, torch.Tensor] = {}
        self._launch_cache: _LaunchCache | None = None
        self._recs: list | None = None
        self._recs_key: tuple | None = None
        self._workspace: dict[torch.device, tuple] = {}
        self._flat: FlatLayout | None = None
        self._copy_sync: dict[int, tuple[int, int]] | None = None
        self._step_idx: tuple[tuple, torch.Tensor] | None = None
        self._fast: _Fast | None = None
        self.native_steps = 0          # steps taken by the native host path
        # measurement hook: None, or three torch.cuda.Event recorded on the launch stream
        # before the norm pass, before the update and after it; an entry that is None is
        # not recorded (a caller timing back-to-back steps may reuse one step's last event
        # as the next step's first: each record is a marker packet that costs GPU time)
        self.timing_events = None
        # place_trials: place_buffers' report once it has run (None until then)
        self.placement: dict | None = None
        # a step was recorded into a graph: the graph keeps the addresses of the
        # tables and buffers it recorded, so they must not move any more
        self.captured = False

    # ------------------------------------------------------------------ torch API

    def __getstate__(self) -> dict[str, Any]:
        """torch's optimizer state (defaults, state, param_groups) plus this class's
        options, so that pickling and copy.deepcopy give a working optimizer."""
        if getattr(self, "_flat", None) is not None:
            raise NotImplementedError("FusedAdamW(flat_buffer=True) cannot be pickled or copied: "
                                      "its parameters are views of its own buffers; save "
                                      "state_dict() instead")
        state = super().__getstate__()
        state["mi_adamw_options"] = {k: getattr(self, k) for k in self._OPTIONS if hasattr(self, k)}
        return state

    def __setstate__(self, state: dict[str, Any]) -> None:
        options = state.pop("mi_adamw_options", None)
        super().__setstate__(state)
        for group in self.param_groups:
            group.setdefault("amsgrad", False)
            group.setdefault("maximize", False)
            group.setdefault("foreach", None)
            group.setdefault("capturable", False)
            group.setdefault("differentiable", False)
            group.setdefault("fused", None)
            group["decoupled_weight_decay"] = True
        if options is None:
            self._recs = None
            self._launch_cache = None
            return
        # Unpickled or copied: rebuild the bookkeeping from the groups and the state.
        for k, v in options.items():
            setattr(self, k, v)
        self._reset_bookkeeping()
        self.register_load_state_dict_post_hook(FusedAdamW._after_load_state_dict)
        for group in self.param_groups:
            self._register_params(group["params"])
        FusedAdamW._after_load_state_dict(self)

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        if getattr(self, "_flat", None) is not None:
            raise NotImplementedError("FusedAdamW(flat_buffer=True): add_param_group after "
                                      "construction is not supported")
        if getattr(self, "bf16_copy", False):
            ps = param_group["params"]
            if not isinstance(ps, (torch.Tensor, set)):
                # materialised in place, as torch's add_param_group does, so that a
                # generator is not consumed by this check
                ps = param_group["params"] = list(ps)
            for p in ([ps] if isinstance(ps, torch.Tensor) else ps):
                # torch also takes (name, parameter) pairs (named_parameters())
                self._check_copyable(p[1] if isinstance(p, tuple) else p)
        if hasattr(self, "capturable") and \
                bool(param_group.get("capturable", self.capturable)) != self.capturable:
            raise NotImplementedError("FusedAdamW: every param group must share the "
                                      "optimizer's capturable setting")
        super().add_param_group(param_group)
        if not hasattr(self, "_slots"):
            return
        self._register_params(self.param_groups[-1]["params"])

    def _register_params(self, params) -> None:
        """Step slots (and bf16 copies) for parameters this optimizer has not seen."""
        new = [p for p in params if id(p) not in self._slots]
        if not new:
            return
        old_n = len(self._step_views)
        steps = torch.zeros(old_n + len(new), dtype=torch.float32, device=self._steps.device)
        steps[:old_n] = self._steps
        for i, p in enumerate(new):
            self._slots[id(p)] = old_n + i
        self._step_views.extend([None] * len(new))
        self._set_step_buffer(steps)
        if getattr(self, "bf16_copy", False) and not getattr(self, "flat_buffer", False):
            for p in new:
                self._copies[id(p)] = self._new_copy(p)
        self._launch_cache = None
        self._recs = None

    def _set_step_buffer(self, steps: torch.Tensor) -> None:
        """Replace the packed step buffer; the per-param step views and the state's
        "step" entries are re-pointed at the new one."""
        self._steps = steps
        for slot, view in enumerate(self._step_views):
            if view is not None:
                self._step_views[slot] = steps[slot]
        for p, st in self.state.items():
            if isinstance(p, torch.Tensor) and id(p) in self._slots and "step" in st:
                view = self._step_views[self._slots[id(p)]]
                if view is not None:
                    st["step"] = view
        self._step_idx = None

    def _steps_for(self, device: torch.device) -> torch.Tensor:
        """The packed step buffer where the step counts live: host memory, or with
        capturable=True the parameters' device (adam.py:168-176 keeps a capturable
        step on the parameter's device), moved there on first use."""
        want = device if self.capturable else torch.device("cpu")
        if self._steps.device != want:
            self._set_step_buffer(self._steps.to(want))
        return self._steps

    def zero_grad(self, set_to_none: bool = True) -> None:
        if self._flat is not None:
            # Gradients are views of the flat gradient buffer: zero them in
            # place so backward accumulates into the buffer again.
            self._flat.zero_grads(self.param_groups)
            return
        super().zero_grad(set_to_none=set_to_none)

    def bf16_params(self) -> list[torch.Tensor]:
        """The bf16 model copies, in param_groups order (bf16_copy=True)."""
        if not self.bf16_copy:
            raise RuntimeError("FusedAdamW was built without bf16_copy=True")
        if self._flat is not None:
            return [self._flat.copy_view(p) for g in self.param_groups for p in g["params"]]
        return [self._copies[id(p)] for g in self.param_groups for p in g["params"]]

    def bf16_param(self, p: torch.Tensor) -> torch.Tensor:
        if not self.bf16_copy:
            raise RuntimeError("FusedAdamW was built without bf16_copy=True")
        if self._flat is not None:
            return self._flat.copy_view(p)
        return self._copies[id(p)]

    @torch.no_grad()
    def refresh_bf16_copies(self) -> None:
        """Rewrite every bf16 copy from its fp32 master (after the masters were
        changed outside the optimizer, e.g. through ``p.data``)."""
        if not self.bf16_copy:
            raise RuntimeError("FusedAdamW was built without bf16_copy=True")
        for g in self.param_groups:
            for p in g["params"]:
                self._refresh_copy(p)

    @staticmethod
    def _check_copyable(p: torch.Tensor) -> None:
        if torch.is_complex(p):
            raise NotImplementedError("FusedAdamW: bf16_copy=True needs real fp32 parameters "
                                      "(a complex parameter has no bf16 copy)")

    @staticmethod
    def _new_copy(p: torch.Tensor) -> torch.Tensor:
        return p.detach().to(torch.bfloat16, memory_format=torch.contiguous_format)

    def _refresh_copy(self, p: torch.Tensor) -> torch.Tensor:
        if self._flat is not None:
            c = self._flat.copy_view(p)
            c.copy_(p.detach())
        else:
            c = self._copies.get(id(p))
            if (c is None or c.shape != p.shape or c.device != p.device
                    or not c.is_contiguous()):
                c = self._copies[id(p)] = self._new_copy(p)
                self._launch_cache = None
            else:
                c.copy_(p.detach())
        if self._copy_sync is not None:
            self._copy_sync[id(p)] = (p._version, p.data_ptr())
        return c

    def _track_copies(self) -> None:
        """Start tracking which copies are current (first use of bf16_weights):
        every copy is rewritten once, then each step records the masters it wrote."""
        if self._copy_sync is None:
            self._copy_sync = {}
            self.refresh_bf16_copies()

    def _current_copies(self, masters: list) -> list:
        """The masters' bf16 copies, each rewritten first if its master changed since
        the copy was written (one pass of cheap checks; grad mode is touched only when
        a copy must be refreshed)."""
        sync = self._copy_sync
        stale = [p for p in masters if sync.get(id(p)) != (p._version, p.data_ptr())]
        if stale:
            with torch.no_grad():
                for p in stale:
                    self._refresh_copy(p)
        return [self._copy_for(p) for p in masters]

    @torch.no_grad()
    def set_state(self, p: torch.Tensor, step: float, exp_avg: torch.Tensor,
                  exp_avg_sq: torch.Tensor, max_exp_avg_sq: torch.Tensor | None = None) -> None:
        """Install one parameter's state in place (like load_state_dict for one
        entry, without materialising a whole state dict): the step count and
        the moments, copied into this optimizer's own storage and dtype."""
        slot = self._slots[id(p)]
        st = self.state[p]
        if "exp_avg" not in st:
            self._init_state(p, st, self._amsgrad_of(p))
        self._steps[slot] = float(step)
        st["step"] = self._step_views[slot]
        st["exp_avg"].copy_(exp_avg)
        st["exp_avg_sq"].copy_(exp_avg_sq)
        if max_exp_avg_sq is not None:
            if "max_exp_avg_sq" not in st:
                self._init_vmax(p, st)
            st["max_exp_avg_sq"].copy_(max_exp_avg_sq)

    def place_buffers(self, trials: int = 16, launches: int = 3, rounds: int = 2,
                      reserve_bytes: int | None = None, min_gain: float = 0.01,
                      per_stream: bool = True, sweeps: int = 3) -> dict:
        """Move the streams the update writes to the fastest of up to `trials` newly
        allocated places, chosen by timing the update's memory-only twin on each against
        the current parameters and gradients (so call it after a backward, or with the
        gradients set).  Tables: exp_avg, exp_avg_sq and the bf16 copy become views of one
        block per stream; flat: the parameter, moment and copy buffers move, if the
        fastest twin beats the current set's by at least `min_gain`; with `per_stream`,
        then each stream alone the same way, the others kept, in up to `sweeps` sweeps
        over the streams (another sweep only after one that moved a stream).  Values are
        moved bit for bit.  Transient memory: one stream set per candidate, as many as fit
        keeping `reserve_bytes` (default max(2 GiB, 2% of HBM)) free.  Returns a report
        of the candidates' twin times and the choice.  No counterpart in torch: the
        MI355X's bandwidth for the update's mix depends on the physical pages of its
        written streams (10-13% between placements).  A move replaces the state entries
        and copies (and, flat, the parameters' ``.data``) with views of the new places, as
        load_state_dict replaces state: tensors taken from ``state``, ``bf16_params()`` or
        ``bf16_param()`` before the call keep the old values and are no longer updated;
        take them again after it.  With capturable=True, call it before capturing: it
        raises once a step has been recorded into a graph."""
        from .placement import place_buffers
        return place_buffers(self, trials=trials, launches=launches, rounds=rounds,
                             reserve_bytes=reserve_bytes, min_gain=min_gain,
                             per_stream=per_stream, sweeps=sweeps)

    def _amsgrad_of(self, p: torch.Tensor) -> bool:
        for g in self.param_groups:
            if any(q is p for q in g["params"]):
                return bool(g["amsgrad"])
        raise KeyError("parameter is not in any param group")

    def state_dict(self) -> dict[str, Any]:
        sd = super().state_dict()
        # The packed step buffer is an implementation detail: hand out
        # independent step tensors, as torch.optim.AdamW does.
        for st in sd["state"].values():
            if isinstance(st, dict) and isinstance(st.get("step"), torch.Tensor):
                st["step"] = st["step"].clone()
        return sd

    @staticmethod
    def _after_load_state_dict(self: "FusedAdamW") -> None:
        """Re-home loaded state: steps into the packed step buffer (host memory, or the
        device with capturable=True), moments in state_dtype."""
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if not st:
                    continue
                slot = self._slots[id(p)]
                steps = self._steps_for(p.device)
                step = st.get("step")
                if isinstance(step, torch.Tensor):
                    if self.capturable:
                        steps[slot] = step.detach().reshape(()).to(steps)   # no host sync
                    else:
                        steps[slot] = float(step.item())
                elif step is not None:
                    steps[slot] = float(step)
                self._step_views[slot] = self._steps[slot]
                st["step"] = self._step_views[slot]
                for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
                    if key in st:
                        t = st[key]
                        if self._flat is not None:
                            st[key] = self._flat.adopt_state(p, key, t)
                        elif t.dtype != self._state_dtype_for(p):
                            st[key] = t.to(self._state_dtype_for(p)).contiguous()
        if self.bf16_copy:
            # checkpoint.py:18-19 loads the model, then the optimizer: the masters may
            # have just changed, so the copies are rewritten from them
            self.refresh_bf16_copies()
        self._launch_cache = None
        self._recs = None

    # ------------------------------------------------------------------ step

    def _state_dtype_for(self, p: torch.Tensor) -> torch.dtype:
        return p.dtype if self.state_dtype == torch.float32 else self.state_dtype

    def _zeros_state(self, p: torch.Tensor) -> torch.Tensor:
        if self.state_dtype == torch.float32:
            return torch.zeros_like(p, memory_format=torch.preserve_format)
        return torch.zeros_like(p, dtype=self.state_dtype, memory_format=torch.contiguous_format)

    def _init_state(self, p: torch.Tensor, st: dict, amsgrad: bool) -> None:
        """adam.py:160-190 lazy state, with the step kept in the packed CPU buffer."""
        slot = self._slots[id(p)]
        self._steps[slot] = 0.0
        self._step_views[slot] = self._steps[slot]
        st["step"] = self._step_views[slot]
        if self._flat is not None:
            st["exp_avg"], st["exp_avg_sq"] = self._flat.state_views(p)
            st["exp_avg"].zero_()
            st["exp_avg_sq"].zero_()
        else:
            st["exp_avg"] = self._zeros_state(p)
            st["exp_avg_sq"] = self._zeros_state(p)
        if amsgrad:
            self._init_vmax(p, st)

    def _init_vmax(self, p: torch.Tensor, st: dict) -> None:
        """amsgrad's max_exp_avg_sq (adam.py:185-190), zero, in the state dtype."""
        if self._flat is not None:
            st["max_exp_avg_sq"] = self._flat.vmax_view(p)
            st["max_exp_avg_sq"].zero_()
        else:
            st["max_exp_avg_sq"] = self._zeros_state(p)

    def _check_param(self, p: torch.Tensor, g: torch.Tensor) -> None:
        if g.is_sparse:
            raise RuntimeError(
                "Adam does not support sparse gradients, please consider SparseAdam instead")
        if p.device.type != "cuda":
            raise RuntimeError(
                f"FusedAdamW steps parameters on a ROCm GPU only; got a {p.device.type} parameter")
        if p.dtype not in (torch.float32, torch.complex64):
            raise NotImplementedError(f"FusedAdamW: parameter dtype {p.dtype} is not supported "
                                      "(fp32 master parameters only)")
        if torch.is_complex(p) and self.state_dtype != torch.float32:
            raise NotImplementedError("FusedAdamW: complex parameters need fp32 state")
        if self.bf16_copy:
            self._check_copyable(p)
        if g.dtype != p.dtype or g.shape != p.shape or g.device != p.device:
            raise RuntimeError("FusedAdamW: gradient dtype/shape/device differs from its parameter")
        if not (p.is_contiguous() and g.is_contiguous()):
            raise NotImplementedError("FusedAdamW: parameters and gradients must be contiguous")

    def _records(self) -> list:
        """Per-parameter bookkeeping in param_groups order, rebuilt when the groups' parameters
        change (compared by identity, so a parameter swapped into a list in place counts)."""
        key = tuple(tuple(map(id, g["params"])) for g in self.param_groups)
        if self._recs is None or self._recs_key != key:
            if self._flat is not None and any(id(p) not in self._flat.offsets
                                              for g in self.param_groups for p in g["params"]):
                # the flat buffers were laid out at construction and have no slice for it
                raise NotImplementedError("FusedAdamW(flat_buffer=True): a parameter put into "
                                          "a param group after construction is not supported")
            # a parameter put into a group's list directly gets its step slot (and bf16 copy)
            self._register_params([p for g in self.param_groups for p in g["params"]])
            self._recs = [_Rec(gi, p, self._slots[id(p)])
                          for gi, g in enumerate(self.param_groups) for p in g["params"]]
            self._recs_key = key
            self._launch_cache = None
        return self._recs

    def step(self, closure=None):
        """One optimizer step (adam.py:214-272), fused.  Returns closure's loss.

        After a step that built the launch tables, the steps that follow go through the
        native host path (``_host``) while nothing but the gradient addresses changes;
        anything else takes the general path below, which rebuilds what changed."""
        self._cuda_graph_capture_health_check()
        if (self.capturable and torch.cuda.is_available()
                and torch.cuda.is_current_stream_capturing()):
            self.captured = True
        fast = self._fast
        if closure is None and fast is not None and self._fast_step(fast):
            return None
        return self._step(closure)

    @torch.no_grad()
    def _step(self, closure):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        # Gather params with grads (adam.py:148-153) and initialise their state.
        entries = [(rec, g) for rec in self._records() if (g := rec.p.grad) is not None]
        if not entries:
            return loss
        flat = self._flat
        ams_g = [bool(g["amsgrad"]) for g in self.param_groups]
        device = entries[0][0].p.device
        if self.capturable:
            self._steps_for(device)
        views = self._step_views
        for i, (rec, g) in enumerate(entries):
            if flat is not None:
                if not flat.is_param_view(rec.p):
                    flat.absorb_param(rec.p)      # p.data was replaced
                if not flat.is_grad_view(rec.p, g):
                    self._check_param(rec.p, g)
                    g = flat.absorb_grad(rec.p)
                    entries[i] = (rec, g)
            if g.is_sparse:
                raise RuntimeError("Adam does not support sparse gradients, please consider "
                                   "SparseAdam instead")
            st = rec.st
            if st is None:
                self._check_param(rec.p, g)   # before self.state gains an entry for p
                st = rec.st = self.state[rec.p]
            if len(st) == 0:
                self._check_param(rec.p, g)
                if self.param_groups[rec.gi]["fused"]:
                    # adam.py:162-163: torch's fused kernel takes real floating-point params
                    # only, and says so at their first step
                    _device_dtype_check_for_fused(rec.p)
                self._init_state(rec.p, st, ams_g[rec.gi])
            else:
                if st["step"] is not views[rec.slot]:
                    self._adopt_step(rec.p, st, rec.slot)
                if flat is not None:
                    flat.absorb_state(rec.p, st)   # moments put into the dict directly
            if ams_g[rec.gi] and "max_exp_avg_sq" not in st:
                # amsgrad switched on for a group after its state was created
                self._init_vmax(rec.p, st)

        if self.capturable:
            # step_t += 1 on the device (adam.py:414), one op for every param with a
            # grad; one constant set per group, the kernel forms the per-step values
            if len(entries) == len(self._step_views):
                self._steps.add_(1)
            else:
                self._steps.index_add_(0, *self._step_increment(entries, device))
            gis = sorted({rec.gi for rec, _ in entries})
            remap = {gi: i for i, gi in enumerate(gis)}
            hyper_idx = [remap[rec.gi] for rec, _ in entries]
            groups = self.param_groups
            hyper_fused = [bool(groups[gi]["fused"]) for gi in gis]
            hypers = [_fused_hyper(groups[gi], 0.0, device) if f
                      else _capt_hyper(groups[gi], device) for gi, f in zip(gis, hyper_fused)]
            hyper_ams = [ams_g[gi] for gi in gis]
        else:
            # step_t += 1 for every param with a grad (adam.py:414), in one op.
            if len(entries) == len(self._step_views):
                self._steps += 1
            else:
                idx = torch.as_tensor([rec.slot for rec, _ in entries], dtype=torch.long)
                self._steps[idx] += 1
            steps_np = self._steps.numpy()

            # One hyperparameter set per distinct (group, step value).
            keys: dict[tuple[int, float], int] = {}
            sel = steps_np[[rec.slot for rec, _ in entries]]
            if len(self.param_groups) == 1 and sel.min() == sel.max():
                keys[(0, float(sel[0]))] = 0          # the usual case: one set for everything
                hyper_idx = [0] * len(entries)
            else:
                hyper_idx = []
                for (rec, _), step in zip(entries, sel.tolist()):
                    k = (rec.gi, step)
                    h = keys.get(k)
                    if h is None:
                        h = keys[k] = len(keys)
                    hyper_idx.append(h)
            groups = self.param_groups
            hyper_fused = [bool(groups[gi]["fused"]) for (gi, _) in keys]
            hypers = [_fused_hyper(groups[gi], step, device) if f else _hyper(groups[gi], step)
                      for (gi, step), f in zip(keys, hyper_fused)]
            hyper_ams = [ams_g[gi] for (gi, _) in keys]
            hyper_group = [gi for (gi, _) in keys]

        with torch.cuda.device(device):
            self._launch(entries, hyper_idx, hypers, hyper_ams, hyper_fused, device,
                         None if self.capturable else hyper_group)
        if self._copy_sync is not None:
            # the launch wrote these masters' copies
            for rec, _ in entries:
                self._copy_sync[id(rec.p)] = (rec.p._version, rec.p.data_ptr())
        if getattr(self, "place_trials", 0) and self.placement is None:
            # once, after the first step: place the written streams of every parameter
            # with state, timed against this step's gradients
            self.placement = self.place_buffers(trials=self.place_trials)
        return loss

    def _step_increment(self, entries, device):
        """(index, ones) on the device for index_add_ of the stepped params' counts,
        kept while the same params step (built outside graph capture)."""
        key = tuple(rec.slot for rec, _ in entries)
        cached = self._step_idx
        if cached is None or cached[0] != key or cached[1].device != device:
            _refuse_under_capture("the set of parameters with gradients changed")
            idx = torch.as_tensor(key, dtype=torch.long).to(device)
            cached = self._step_idx = (key, idx, torch.ones(len(key), device=device))
        return cached[1], cached[2]

    def _adopt_step(self, p, st, slot):
        """state["step"] was replaced from outside: copy its value into the buffer."""
        step = st["step"]
        if isinstance(step, torch.Tensor) and self.capturable:
            self._steps[slot] = step.detach().reshape(()).to(self._steps)
        else:
            self._steps[slot] = float(step.item()) if isinstance(step, torch.Tensor) else float(step)
        self._step_views[slot] = self._steps[slot]
        st["step"] = self._step_views[slot]

    # ------------------------------------------------------------------ native path

    def _options_key(self) -> tuple:
        return (self.max_grad_norm, self.clip_write_grads, self.grad_prescale, self.max_blocks,
                self.chunk_elems, self.bf16_copy, self.state_dtype)

    def _groups_key(self) -> tuple:
        """The groups' parameters (by identity, so a parameter swapped into a group's list
        in place is seen), amsgrad settings and chains (fused)."""
        return tuple((tuple(map(id, g["params"])), bool(g["amsgrad"]), bool(g["fused"]))
                     for g in self.param_groups)

    def _make_fast(self, entries, hyper_idx, hyper_group, ams, fused, launch, device, stream,
                   partials, coef, state_code, flags):
        """The native path's plan for the steps after this one, when this step's launch is
        one the native path can repeat: every parameter stepped, one launch that the norm
        pass shares, one hyperparameter set per param group."""
        if (len(set(hyper_group)) != len(hyper_group) or launch.n_chunks == 0
                or len(entries) != len(self._records())
                or not self._steps.is_contiguous() or self._steps.device.type != "cpu"):
            return None
        host = _lib.host()
        n = len(entries)
        if self._flat is not None:
            rows = [-2] * n          # gradients are views of the flat buffer: they must stay
            rest = [True] * n
        else:
            rows, rest = [-1] * n, [False] * n
            for r, i in enumerate(launch.src.tolist()):
                rows[i] = r
                rest[i] = bool(launch.rest[r])
        hyper_steps = np.zeros(len(hyper_group), dtype=np.float64)
        flat_row = None if launch.tables else self._row_struct(launch)
        if ams:
            flags |= _lib.F_AMSGRAD
        sumsq = self._sumsq_buf(device) if self.grad_prescale != 1.0 else None
        clip = self.max_grad_norm is not None
        if not clip:
            flags &= ~_lib.F_WRITE_GRAD
        try:
            plan = host.plan(
                [rec.p for rec, _ in entries], [rec.st for rec, _ in entries],
                [rec.slot for rec, _ in entries], [int(h) for h in hyper_idx], rows, rest,
                [g.data_ptr() for _, g in entries], bool(ams),
                (self._steps.data_ptr(), self._steps.numel()),
                (hyper_steps.ctypes.data, len(hyper_group)),
                (bool(launch.tables), 0 if launch.rows is None else launch.rows.data_ptr(),
                 0 if launch.chunks is None else launch.chunks.data_ptr(), int(launch.n_chunks),
                 int(launch.n_rows), launch.host_rows.ctypes.data,
                 0 if flat_row is None else ctypes.addressof(flat_row),
                 0 if launch.tables else int(launch.host_rows[0]["hyper"])),
                (int(self.chunk_elems), int(self.max_blocks), int(state_code), int(flags), clip,
                 float(self.max_grad_norm or 0.0), float(self.grad_prescale),
                 partials.data_ptr(), coef.data_ptr(), 0 if sumsq is None else sumsq.data_ptr(),
                 int(stream), bool(fused)),
                (launch.rows, launch.chunks, launch.host_rows, self._steps, hyper_steps,
                 partials, coef, sumsq))
        except (TypeError, ValueError):
            return None     # a state entry the plan cannot check (not a tensor): general path
        fast = _Fast()
        fast.plan = plan
        fast.cache = self._launch_cache
        fast.steps = self._steps
        fast.state = self.state
        fast.groups_key = self._groups_key()
        fast.options = self._options_key()
        fast.hyper_group = list(hyper_group)
        fast.hyper_steps = hyper_steps
        fast.fused = bool(fused)
        fast.harr = ((_lib.FusedHyper if fused else _lib.Hyper) * len(hyper_group))()
        fast.harr_addr = ctypes.addressof(fast.harr)
        fast.clip = clip
        fast.device = device
        fast.dev_index = device.index if device.index is not None else torch.cuda.current_device()
        return fast

    def _fast_step(self, fast: _Fast) -> bool:
        """One step through the native host path; False (nothing done) when it does not
        apply, and the general path takes the step."""
        if (self._launch_cache is not fast.cache or self._steps is not fast.steps
                or self.state is not fast.state or self._options_key() != fast.options
                or self._groups_key() != fast.groups_key):
            return False
        host = _lib._host
        dev = fast.dev_index
        if torch._C._cuda_getDevice() != dev:
            with torch.cuda.device(dev):
                return self._fast_launch(fast, host)
        return self._fast_launch(fast, host)

    def _fast_prepare(self, fast: _Fast, host, stream: int) -> bool:
        """The native checks, gradient patch and step counting of one step: True when the
        native path takes the step, False (nothing changed) when the general path must.
        A failed gradient patch raises, after dropping the plan and the tables: the step
        counts are unchanged, but the device table may hold part of the patch."""
        rc = host.prepare(fast.plan, stream)
        if rc == host.FALLBACK:
            return False
        if rc == host.ERROR:
            code = host.last_error(fast.plan)
            self._fast = None
            self._launch_cache = None
            raise _lib.MiAdamwError(f"mi_adamw_set_grads failed: {_lib.strerror(code)} "
                                    f"(code {code})")
        if rc == host.READY_MOVED:
            fast.cache.grads = None   # the general path's record of the gradients is stale
        elif rc != host.READY:
            raise RuntimeError(f"mi_adamw._host.prepare returned an unknown status {rc}")
        self.native_steps += 1
        return True

    def _fast_launch(self, fast: _Fast, host) -> bool:
        stream = torch._C._cuda_getCurrentRawStream(fast.dev_index)
        if not self._fast_prepare(fast, host, stream):
            return False
        groups = self.param_groups
        harr = fast.harr
        if fast.fused:
            for h, gi in enumerate(fast.hyper_group):
                harr[h] = _fused_hyper(groups[gi], float(fast.hyper_steps[h]), fast.device)
        else:
            for h, gi in enumerate(fast.hyper_group):
                harr[h] = _hyper(groups[gi], float(fast.hyper_steps[h]))
        ev = self.timing_events
        _record(ev, 0)
        if fast.clip:
            norm = torch.empty((), dtype=torch.float32, device=fast.device)
            _lib.check(host.norm(fast.plan, stream, norm.data_ptr()), "mi_adamw_grad_norm")
            self.last_grad_norm = norm
        _record(ev, 1)
        _lib.check(host.update(fast.plan, stream, fast.harr_addr, len(harr)), "mi_adamw_step")
        _record(ev, 2)
        if self._copy_sync is not None:
            host.sync_versions(fast.plan, self._copy_sync)
        return True

    # ------------------------------------------------------------------ launches

    def _ws(self, device: torch.device):
        ws = self._workspace.get(device)
        if ws is None:
            partials = torch.zeros(_lib.MAX_NORM_BLOCKS, dtype=torch.float64, device=device)
            coef = torch.zeros(1, dtype=torch.float32, device=device)
            ws = self._workspace[device] = (partials, coef)
        return ws

    def _sumsq_buf(self, device: torch.device) -> torch.Tensor:
        """One float64 on the device: the pre-scaled gradients' sum of squares."""
        buf = self._workspace.get(("sumsq", device))
        if buf is None:
            buf = self._workspace[("sumsq", device)] = torch.zeros(1, dtype=torch.float64,
                                                                    device=device)
        return buf

    def _rows(self, entries, hyper_idx, ams):
        """(rows, src, rest): the table rows of `entries`, the entry each row's gradient
        belongs to (-1 for a flat group row) and whether its other pointers are aligned."""
        if self._flat is not None:
            return self._flat_rows(entries, hyper_idx, ams)
        return self._tensor_rows(entries, hyper_idx, ams)

    def _new_launch(self, entries, hyper_idx, ams, device) -> _Launch:
        if self.capturable:
            # one row per tensor (each has its own device step count), always as tables
            rows, src, rest = self._tensor_rows(entries, hyper_idx, ams)
            slots = np.asarray([entries[i][0].slot for i in src], dtype=np.int32)
            return _Launch(rows, self.chunk_elems, device, tables=True, src=src, rest=rest,
                           step_slots=slots)
        rows, src, rest = self._rows(entries, hyper_idx, ams)
        return _Launch(rows, self.chunk_elems, device, src=src, rest=rest)

    def _flat_rows(self, entries, hyper_idx, ams):
        """One row per param group whose every param steps with one hyper set."""
        by_group: dict[int, list[int]] = {}
        for i, (rec, _) in enumerate(entries):
            by_group.setdefault(rec.gi, []).append(i)
        rows, srcs, rests = [], [], []
        for gi, idx in by_group.items():
            hs = {hyper_idx[i] for i in idx}
            if len(idx) == len(self.param_groups[gi]["params"]) and len(hs) == 1:
                pp, gp, mp, vp, cp, xp, n = self._flat.group_row(gi, ams)
                r = np.zeros(1, dtype=_ROW_DTYPE)
                r[0] = (pp, gp, mp, vp, cp, xp, n, hs.pop(), _lib.T_VEC)
                rows.append(r)
                srcs.append(np.full(1, -1, dtype=np.int64))
                rests.append(np.ones(1, dtype=bool))
            else:
                r, src, rest = self._tensor_rows([entries[i] for i in idx],
                                                 [hyper_idx[i] for i in idx], ams)
                rows.append(r)
                srcs.append(np.asarray(idx, dtype=np.int64)[src])
                rests.append(rest)
        if not rows:
            return np.zeros(0, dtype=_ROW_DTYPE), np.zeros(0, np.int64), np.zeros(0, bool)
        return np.concatenate(rows), np.concatenate(srcs), np.concatenate(rests)

    def _state_tensor(self, p: torch.Tensor, st: dict, key: str) -> torch.Tensor:
        """st[key] as the kernel reads it: p's element count, state dtype, p's
        device, contiguous (converted in place in the state if it is not)."""
        t = st[key]
        want = self._state_dtype_for(p)
        if t.numel() != p.numel():
            raise RuntimeError(f"FusedAdamW: state[{key!r}] has {t.numel()} elements but its "
                               f"parameter has {p.numel()}")
        if t.dtype != want or t.device != p.device or not t.is_contiguous():
            # .contiguous(), not to(memory_format=contiguous_format): to() returns the
            # tensor itself when dtype and device already match and its suggested
            # memory format is contiguous, which a 1-D or 2-D strided view reports
            with torch.no_grad():
                t = st[key] = t.to(device=p.device, dtype=want).contiguous()
        return t

    def _tensor_rows(self, entries, hyper_idx, ams):
        rows = np.zeros(len(entries), dtype=_ROW_DTYPE)
        rest = np.zeros(len(entries), dtype=bool)
        bf16_state = self.state_dtype == torch.bfloat16
        for i, ((rec, g), h) in enumerate(zip(entries, hyper_idx)):
            p, st = rec.p, rec.st
            m = self._state_tensor(p, st, "exp_avg")
            v = self._state_tensor(p, st, "exp_avg_sq")
            c = None
            if self.bf16_copy:
                c = self._copy_for(p)
                if c.numel() != p.numel() or c.device != p.device or not c.is_contiguous():
                    c = self._refresh_copy(p)   # p.data was replaced: a new copy of its size
            pp, gp, mp, vp, cp = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), _ptr(c)
            xp = self._state_tensor(p, st, "max_exp_avg_sq").data_ptr() if ams else 0
            n = p.numel() * (2 if torch.is_complex(p) else 1)
            sa = 8 if bf16_state else 16
            rest[i] = (pp % 16 == 0 and mp % sa == 0 and vp % sa == 0 and cp % 8 == 0
                       and xp % sa == 0)
            vec = rest[i] and gp % 16 == 0
            rows[i] = (pp, gp, mp, vp, cp, xp, n, h, _lib.T_VEC if vec else 0)
        keep = rows["numel"] > 0
        return rows[keep], np.flatnonzero(keep).astype(np.int64), rest[keep]

    def _copy_for(self, p):
        if self._flat is not None:
            return self._flat.copy_view(p)
        return self._copies[id(p)]

    @staticmethod
    def _signature(entries, hyper_idx, hyper_ams, hyper_fused) -> tuple[list, list]:
        """What a launch's tables encode, in two parts: the hyperparameter assignment,
        the amsgrad setting and chain of each hyperparameter set (which decide how the
        entries are split into launches), and the parameter and state pointers, which rarely
        change; and the gradient pointers, which change whenever zero_grad() frees the
        gradients and backward allocates them elsewhere."""
        # the element count and contiguity too: a parameter or a moment narrowed or
        # re-strided in place through .data keeps its address (a rebuild then checks or
        # converts it)
        sig = [(rec.p.data_ptr(), rec.p.numel(), rec.p.is_contiguous(),
                _layout(rec.st["exp_avg"]), _layout(rec.st["exp_avg_sq"]),
                _layout(rec.st.get("max_exp_avg_sq")))
               for rec, _ in entries]
        sig.append(tuple(hyper_idx))
        sig.append(tuple(bool(a) for a in hyper_ams))
        sig.append(tuple(bool(f) for f in hyper_fused))
        return sig, [g.data_ptr() for _, g in entries]

    @staticmethod
    def _row_struct(launch: _Launch) -> _lib.TensorRow:
        r = launch.host_rows[0]
        return _lib.TensorRow(param=int(r["param"]), grad=int(r["grad"]),
                              exp_avg=int(r["exp_avg"]), exp_avg_sq=int(r["exp_avg_sq"]),
                              param_copy=int(r["param_copy"]),
                              max_exp_avg_sq=int(r["max_exp_avg_sq"]), numel=int(r["numel"]),
                              hyper=0, flags=int(r["flags"]))

    def _launch(self, entries, hyper_idx, hypers, hyper_ams, hyper_fused, device,
                hyper_group: list | None = None) -> None:
        lib = _lib.load()
        self._fast = None
        stream = torch.cuda.current_stream(device).cuda_stream
        partials, coef = self._ws(device)
        flags = 0
        if self.bf16_copy:
            flags |= _lib.F_BF16_COPY
        state_code = _lib.STATE_BF16 if self.state_dtype == torch.bfloat16 else _lib.STATE_F32

        # Partition into launches of one amsgrad setting and one chain (default or
        # fused=True) and at most MAX_HYPER hyperparameter sets each.
        kinds = list(zip(hyper_ams, hyper_fused))
        if len(hypers) <= _lib.MAX_HYPER and len(set(kinds)) == 1:
            parts = [(entries, hyper_idx, hypers, kinds[0], None)]
        else:
            parts = []
            for kind in sorted(set(kinds)):
                hsel = [h for h in range(len(hypers)) if kinds[h] == kind]
                for start in range(0, len(hsel), _lib.MAX_HYPER):
                    block = hsel[start:start + _lib.MAX_HYPER]
                    remap = {h: j for j, h in enumerate(block)}
                    sel = [i for i, h in enumerate(hyper_idx) if h in remap]
                    parts.append(([entries[i] for i in sel],
                                  [remap[hyper_idx[i]] for i in sel],
                                  [hypers[h] for h in block], kind,
                                  np.asarray(sel, dtype=np.int64)))

        # Tables: reused while the pointers and the hyperparameter assignment are
        # unchanged; when only the gradients moved, the rows are rewritten and the
        # chunk tables kept.
        sig, grads = self._signature(entries, hyper_idx, hyper_ams, hyper_fused)
        # the chunk tables are cut at chunk_elems: a new value needs new tables
        sig.append(("chunk_elems", self.chunk_elems))
        cache = self._launch_cache
        if cache is not None and cache.sig == sig and cache.device == device:
            launches, norm_launch = cache.launches, cache.norm_launch
            if cache.grads != grads:
                _refuse_under_capture("gradient tensors moved")
                # torch checks shape, dtype and device when .grad is assigned; the
                # kernels also need dense storage of the row's size
                for rec, g in entries:
                    if not g.is_contiguous() or g.numel() != rec.p.numel():
                        self._check_param(rec.p, g)
                garr = np.asarray(grads, dtype=np.uint64)
                for launch, part in zip(launches, parts):
                    launch.patch_grads(garr if part[4] is None else garr[part[4]], device)
                if norm_launch is not launches[0]:
                    norm_launch.patch_grads(garr, device)
                self._launch_cache = _LaunchCache(sig, device, launches, norm_launch, grads)
        else:
            _refuse_under_capture("the parameters, state or hyperparameter grouping changed")
            for rec, g in entries:
                self._check_param(rec.p, g)
                if rec.p.device != device:
                    raise NotImplementedError("FusedAdamW: all parameters must be on one device")
            launches = [self._new_launch(e, hi, k[0], device) for e, hi, _, k, _ in parts]
            if len(parts) == 1:
                norm_launch = launches[0]
            else:
                norm_launch = self._new_launch(entries, [0] * len(entries), False, device)
            self._launch_cache = _LaunchCache(sig, device, launches, norm_launch, grads)

        ev = self.timing_events
        _record(ev, 0)
        if self.max_grad_norm is not None:
            norm = torch.empty((), dtype=torch.float32, device=device)
            if norm_launch.n_chunks == 0:
                # nothing but empty tensors: torch's norm of no elements is 0
                norm.zero_()
                coef.fill_(1.0)
            elif self.grad_prescale != 1.0:
                # the sum of squares of the pre-scaled gradients, then the finalize over it
                sumsq = self._sumsq_buf(device)
                if norm_launch.n_rows == 1:
                    row = self._row_struct(norm_launch)
                    _lib.check(lib.mi_adamw_grad_sumsq_flat(
                        row.grad, row.numel, self.chunk_elems, self.grad_prescale,
                        partials.data_ptr(), sumsq.data_ptr(), stream), "mi_adamw_grad_sumsq_flat")
                else:
                    _lib.check(lib.mi_adamw_grad_sumsq(
                        norm_launch.rows.data_ptr(), norm_launch.chunks.data_ptr(),
                        norm_launch.n_chunks, self.chunk_elems, self.grad_prescale,
                        partials.data_ptr(), sumsq.data_ptr(), stream), "mi_adamw_grad_sumsq")
                _lib.check(lib.mi_adamw_norm_from_sumsq(
                    sumsq.data_ptr(), 1, float(self.max_grad_norm), norm.data_ptr(),
                    coef.data_ptr(), stream), "mi_adamw_norm_from_sumsq")
            elif norm_launch.n_rows == 1:
                row = self._row_struct(norm_launch)
                _lib.check(lib.mi_adamw_grad_norm_flat(
                    row.grad, row.numel, self.chunk_elems, float(self.max_grad_norm),
                    partials.data_ptr(), norm.data_ptr(), coef.data_ptr(),
                    stream), "mi_adamw_grad_norm_flat")
            else:
                _lib.check(lib.mi_adamw_grad_norm(
                    norm_launch.rows.data_ptr(), norm_launch.chunks.data_ptr(),
                    norm_launch.n_chunks, self.chunk_elems, float(self.max_grad_norm),
                    partials.data_ptr(), norm.data_ptr(), coef.data_ptr(),
                    stream), "mi_adamw_grad_norm")
            self.last_grad_norm = norm
            flags |= _lib.F_CLIP
            if self.clip_write_grads:
                flags |= _lib.F_WRITE_GRAD
        _record(ev, 1)
        for launch, (_, _, hs, (ams, fused), _) in zip(launches, parts):
            if launch.n_chunks == 0:
                continue
            lflags = flags | (_lib.F_AMSGRAD if ams else 0)
            if fused:
                self._launch_fused_chain(launch, hs, coef, state_code, lflags, stream)
                continue
            if self.capturable:
                carr = (_lib.CaptHyper * len(hs))(*hs)
                _lib.check(lib.mi_adamw_step_capturable_rows(
                    launch.rows.data_ptr(), launch.n_rows, launch.chunks.data_ptr(),
                    launch.n_chunks, self.chunk_elems, carr, len(hs), self._steps.data_ptr(),
                    launch.step_index.data_ptr(), launch.row_scalars.data_ptr(),
                    coef.data_ptr(), state_code, lflags, self.max_blocks, stream),
                    "mi_adamw_step_capturable_rows")
                continue
            harr = (_lib.Hyper * len(hs))(*hs)
            pre = self.grad_prescale
            if launch.n_rows == 1:
                row = self._row_struct(launch)
                row_h = hs[int(launch.host_rows[0]["hyper"])]
                if pre != 1.0:
                    _lib.check(lib.mi_adamw_step_flat_prescaled(
                        ctypes.byref(row), ctypes.byref(row_h), coef.data_ptr(), pre,
                        self.chunk_elems, state_code, lflags, self.max_blocks, stream),
                        "mi_adamw_step_flat_prescaled")
                    continue
                _lib.check(lib.mi_adamw_step_flat(
                    ctypes.byref(row), ctypes.byref(row_h), coef.data_ptr(), self.chunk_elems,
                    state_code, lflags, self.max_blocks, stream), "mi_adamw_step_flat")
                continue
            if pre != 1.0:
                _lib.check(lib.mi_adamw_step_prescaled(
                    launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks,
                    self.chunk_elems, harr, len(hs), coef.data_ptr(), pre, state_code, lflags,
                    self.max_blocks, stream), "mi_adamw_step_prescaled")
                continue
            _lib.check(lib.mi_adamw_step(
                launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks,
                self.chunk_elems, harr, len(hs), coef.data_ptr(), state_code, lflags,
                self.max_blocks, stream), "mi_adamw_step")
        _record(ev, 2)
        if len(parts) == 1 and hyper_group is not None:
            self._fast = self._make_fast(entries, hyper_idx, hyper_group, hyper_ams[0],
                                         hyper_fused[0], launches[0], device, stream, partials,
                                         coef, state_code, flags & ~_lib.F_CLIP)

    def _launch_fused_chain(self, launch: _Launch, hs: list, coef: torch.Tensor,
                            state_code: int, flags: int, stream: int) -> None:
        """One launch of torch's fused=True chain: the tables (with the device step counts
        when capturable) or the one flat range."""
        lib = _lib.load()
        pre = self.grad_prescale
        if launch.n_rows == 1 and not launch.tables:
            row = self._row_struct(launch)
            row_h = hs[int(launch.host_rows[0]["hyper"])]
            _lib.check(lib.mi_adamw_step_flat_fused_chain(
                ctypes.byref(row), ctypes.byref(row_h), coef.data_ptr(), pre, self.chunk_elems,
                state_code, flags, self.max_blocks, stream), "mi_adamw_step_flat_fused_chain")
            return
        farr = (_lib.FusedHyper * len(hs))(*hs)
        if self.capturable:
            # device step counts: the per-step values formed once per row before the update
            _lib.check(lib.mi_adamw_step_fused_chain_rows(
                launch.rows.data_ptr(), launch.n_rows, launch.chunks.data_ptr(), launch.n_chunks,
                self.chunk_elems, farr, len(hs), self._steps.data_ptr(),
                launch.step_index.data_ptr(), launch.row_scalars.data_ptr(), coef.data_ptr(),
                pre, state_code, flags, self.max_blocks, stream),
                "mi_adamw_step_fused_chain_rows")
            return
        # host step counts (hs[i].step): no step buffer
        _lib.check(lib.mi_adamw_step_fused_chain(
            launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks, self.chunk_elems,
            farr, len(hs), None, None, coef.data_ptr(), pre, state_code, flags, self.max_blocks,
            stream), "mi_adamw_step_fused_chain")
