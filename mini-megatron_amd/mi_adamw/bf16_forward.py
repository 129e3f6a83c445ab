"""The step's bf16 model copy as the forward pass's GEMM weights.

Reference path.  With ``--amp`` mini-megatron runs its forward under
``torch.autocast("cuda", dtype=torch.bfloat16)`` (main.py:93,190,205) over fp32
parameters.  Every GEMM weight reaches ``F.linear`` in the tensor-parallel
linear layers (parallel/tensor_parallel.py:55,79), and autocast casts it to
bf16 there: one cast kernel per weight per forward (4 B read + 2 B written per
parameter), whose backward widens the bf16 weight gradient to fp32 into
``p.grad``.  ``FusedAdamW(bf16_copy=True)`` already writes that same bf16 value
-- round-to-nearest-even of the updated fp32 master -- inside its step.

``bf16_weights(optimizer, *modules)`` hands those copies to the linear layers
for the duration of a forward, in place of the casts:

* forward: ``module.weight`` (and ``bias``) is the bf16 copy; autocast leaves a
  tensor that already has its target dtype alone, so the GEMM sees the same
  operands as under the cast;
* backward: the weight gradient, bf16, is widened to fp32 and accumulated into
  the master's ``.grad`` -- the backward of autocast's own cast.  (Autocast
  also caches one cast per weight per region, so a layer called twice inside
  the context sums its two bf16 gradients before the widening, as here.)

Loss, activations and master gradients are therefore bit-identical to plain
autocast, without the per-forward weight casts.  Only layers whose weights
autocast casts to bf16 may be swapped (``F.linear``-based layers); layer norms
and embeddings keep their fp32 weights, as under autocast.  A copy is refreshed
from its master when the master changed outside the optimizer (its version
counter or storage moved, e.g. ``model.load_state_dict``); a change made
through ``p.data`` is not visible that way: call
``optimizer.refresh_bf16_copies()`` after one.

Meant for eager-mode models, the reference's default; it is not tested with a
``torch.compile``'d model (``--compile``, main.py), whose graphs guard on the
parameters this context replaces.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib

_WIDEN_CHUNK = 4096
_widen_tables: dict[tuple, object] = {}


def _widen_on_gpu(srcs: list[torch.Tensor], device: torch.device) -> list[torch.Tensor]:
    """fp32 copies of contiguous bf16 tensors on one GPU, one launch for all of them
    (mi_adamw_widen_bf16).  The chunk table depends on the sizes only and is kept; the
    rows, whose pointers change with every backward, are rewritten."""
    from .optimizer import _ROW_DTYPE, _Launch
    dsts = [torch.empty(t.shape, dtype=torch.float32, device=device) for t in srcs]
    rows = np.zeros(len(srcs), dtype=_ROW_DTYPE)
    rows["param"] = [d.data_ptr() for d in dsts]
    rows["param_copy"] = [t.data_ptr() for t in srcs]
    rows["numel"] = [t.numel() for t in srcs]
    rows["flags"] = np.where((rows["param"] % 16 == 0) & (rows["param_copy"] % 8 == 0),
                             _lib.T_VEC, 0)
    rows = rows[rows["numel"] > 0]
    if len(rows) == 0:
        return dsts
    # Per stream: the tables are then allocated on the stream whose launches read them,
    # so a replaced or dropped table returns to that stream's pool, ordered after them.
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device, stream, tuple(int(n) for n in rows["numel"]))
    launch = _widen_tables.get(key)
    if launch is None:
        if len(_widen_tables) > 8:
            _widen_tables.clear()
        launch = _widen_tables[key] = _Launch(rows, _WIDEN_CHUNK, device, tables=True)
    else:
        launch.set_rows(rows, device)
    lib = _lib.load()
    with torch.cuda.device(device):
        _lib.check(lib.mi_adamw_widen_bf16(
            launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks, _WIDEN_CHUNK,
            stream), "mi_adamw_widen_bf16")
    return dsts


def _widen(grads) -> tuple:
    """Each bf16 gradient widened to fp32 (exact: a bf16 value is the upper half of
    its fp32 bits).  The GPU ones, all of a backward's weight gradients, in one launch
    per device; CPU tensors (the CPU autocast of the tests) by torch's cast."""
    out: list = [None] * len(grads)
    by_device: dict[torch.device, list[int]] = {}
    for i, g in enumerate(grads):
        if g is None:
            continue
        if g.is_cuda and g.dtype == torch.bfloat16:
            by_device.setdefault(g.device, []).append(i)
        else:
            out[i] = g.to(torch.float32)
    for device, idx in by_device.items():
        for i, d in zip(idx, _widen_on_gpu([grads[i].contiguous() for i in idx], device)):
            out[i] = d
    return tuple(out)


class _MastersAsBf16(torch.autograd.Function):
    """Forward: the bf16 copies of n masters.  Backward: each copy's gradient
    widened to fp32 for its master (what ``Tensor.to``'s backward does for
    autocast's cast), all of them in one launch.  One node for every swapped
    weight, so the host pays one Python call per forward and one per backward,
    not one per weight."""

    @staticmethod
    def forward(ctx, copies, *masters):
        # the copies come in as one list: only the masters are autograd inputs
        ctx.set_materialize_grads(False)
        return tuple(c.view_as(c) for c in copies)

    @staticmethod
    def backward(ctx, *grads):
        return (None,) + _widen(grads)


def linear_layers(module: torch.nn.Module) -> bool:
    """Default selection: ``nn.Linear`` and any layer class named ``*Linear`` (the
    reference's ColumnParallelLinear / RowParallelLinear), which call F.linear."""
    return isinstance(module, torch.nn.Linear) or type(module).__name__.endswith("Linear")


class bf16_weights:
    """Context manager: selected layers of ``modules`` run on the optimizer's bf16 copies.

    Enter it inside the bf16 autocast region, around the forward::

        with torch.autocast("cuda", dtype=torch.bfloat16), mi_adamw.bf16_weights(opt, model):
            loss = model(tokens, labels, mask)[1]
        loss.backward()

    ``select(module) -> bool`` chooses the layers (default ``linear_layers``);
    only their directly owned fp32 parameters that the optimizer steps are
    swapped.  While the context is open, ``layer.weight`` is the bf16 copy;
    on exit the parameters are back in place.  Entering outside a bf16 autocast
    region raises.
    """

    def __init__(self, optimizer, *modules: torch.nn.Module, select=linear_layers):
        if not getattr(optimizer, "bf16_copy", False):
            raise RuntimeError("bf16_weights needs an optimizer built with bf16_copy=True")
        owned = {id(p) for g in optimizer.param_groups for p in g["params"]}
        self.optimizer = optimizer
        self.swaps: list[tuple[torch.nn.Module, str, torch.nn.Parameter]] = []
        seen: set[int] = set()
        for root in modules:
            for mod in root.modules():
                if id(mod) in seen or not select(mod):
                    continue
                seen.add(id(mod))
                for n, p in mod.named_parameters(recurse=False):
                    if id(p) in owned and p.dtype == torch.float32:
                        self.swaps.append((mod, n, p))
        self._active = False

    def __enter__(self) -> "bf16_weights":
        if not self.swaps:
            return self
        dev = self.swaps[0][2].device.type
        if not (torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16):
            raise RuntimeError("bf16_weights: enter it inside a bf16 autocast region; outside "
                               "one the swapped weights would not match autocast's casts")
        opt = self.optimizer
        opt._track_copies()
        masters = [p for _, _, p in self.swaps]
        copies = opt._current_copies(masters)
        aliases = _MastersAsBf16.apply(copies, *masters)
        for (mod, n, _), a in zip(self.swaps, aliases):
            # Assigned into _parameters directly: a non-leaf bf16 tensor for the
            # duration of the context, restored on exit.
            mod._parameters[n] = a
        self._active = True
        return self

    def __exit__(self, *exc) -> None:
        if self._active:
            for mod, n, p in self.swaps:
                mod._parameters[n] = p
            self._active = False
