"""clip_grad_norm_: drop-in for torch.nn.utils.clip_grad_norm_ on the MI355X kernels.

mini-megatron names the clip value (config.py:16, MAX_GRAD_NORM = 1.0); the
standard way to apply it in its loop is ``torch.nn.utils.clip_grad_norm_``
between ``loss.backward()`` and ``optimizer.step()`` (main.py:207-209).  This
function keeps that signature and result: the global L2 norm of every gradient
as one vector (torch/nn/utils/clip_grad.py:50-117), then
``g *= min(max_norm / (norm + 1e-6), 1)`` in place (clip_grad.py:121-183).
Two launches: the float64 sum-of-squares pass (which also computes the
coefficient on the device) and an in-place scale pass.  Use
``FusedAdamW(max_grad_norm=...)`` instead to fold the scale into the step.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib

_CHUNK = 4096
_workspace: dict[tuple, tuple] = {}
_cache: dict[tuple, tuple] = {}


def _ws(device, stream: int):
    """Partial sums and coefficient, one set per (device, stream): calls on different
    streams may overlap and must not share scratch (calls on one stream are ordered)."""
    key = (device, stream)
    ws = _workspace.get(key)
    if ws is None:
        if len(_workspace) > 16:
            # a freed block returns to the pool of the stream it was allocated on, and
            # any reuse there is ordered after the work already queued on that stream
            _workspace.clear()
        ws = _workspace[key] = (
            torch.zeros(_lib.MAX_NORM_BLOCKS, dtype=torch.float64, device=device),
            torch.zeros(1, dtype=torch.float32, device=device),
        )
    return ws


def _tables(grads, device, stream: int):
    """The tables of one gradient list.  The chunk table depends on the sizes only and is
    cached by them, per stream (so the tables are allocated on the stream whose launches
    read them, and a replaced or dropped table returns to that stream's pool, ordered
    after those launches); when the gradients moved (zero_grad freed them and backward
    allocated them elsewhere) only the rows are rewritten."""
    from .optimizer import _ROW_DTYPE, _Launch
    rows = np.zeros(len(grads), dtype=_ROW_DTYPE)
    ptrs = np.array([g.data_ptr() for g in grads], dtype=np.uint64)
    # Only the gradient pointer is read by the norm and scale kernels.
    rows["param"] = ptrs
    rows["grad"] = ptrs
    rows["numel"] = [g.numel() * (2 if torch.is_complex(g) else 1) for g in grads]
    rows["flags"] = np.where(ptrs % 16 == 0, _lib.T_VEC, 0)
    rows = rows[rows["numel"] > 0]
    key = (device, stream, tuple(int(n) for n in rows["numel"]))
    launch = _cache.get(key)
    if launch is not None:
        if not np.array_equal(launch.host_rows["grad"], rows["grad"]):
            launch.set_rows(rows, device)
        return launch
    launch = _Launch(rows, _CHUNK, device, tables=True)
    if len(_cache) > 8:
        _cache.clear()
    _cache[key] = launch
    return launch


@torch.no_grad()
def clip_grad_norm_(parameters, max_norm: float, norm_type: float = 2.0,
                    error_if_nonfinite: bool = False, foreach: bool | None = None) -> torch.Tensor:
    """Clip the global gradient norm in place; returns the total norm (0-d tensor)."""
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    grads = [p.grad for p in parameters if p.grad is not None]
    if float(norm_type) != 2.0:
        raise NotImplementedError("mi_adamw.clip_grad_norm_ supports norm_type=2 only")
    if len(grads) == 0:
        return torch.tensor(0.0)
    device = grads[0].device
    for g in grads:
        if g.device != device or g.device.type != "cuda":
            raise RuntimeError("mi_adamw.clip_grad_norm_ needs every gradient on one ROCm GPU")
        if g.dtype not in (torch.float32, torch.complex64) or not g.is_contiguous() or g.is_sparse:
            raise NotImplementedError("mi_adamw.clip_grad_norm_ supports dense contiguous fp32 "
                                      "gradients only")
    lib = _lib.load()
    norm = torch.empty((), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        launch = _tables(grads, device, stream)
        partials, coef = _ws(device, stream)
        if launch.n_chunks == 0:
            norm.zero_()
            return norm
        _lib.check(lib.mi_adamw_grad_norm(
            launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks, _CHUNK,
            float(max_norm), partials.data_ptr(), norm.data_ptr(),
            coef.data_ptr(), stream), "mi_adamw_grad_norm")
        if error_if_nonfinite and bool(torch.logical_or(norm.isnan(), norm.isinf())):
            raise RuntimeError(
                f"The total norm of order {float(norm_type)} for gradients from "
                "`parameters` is non-finite, so it cannot be clipped. To disable "
                "this error and scale the gradients by the non-finite norm anyway, "
                "set `error_if_nonfinite=False`")
        _lib.check(lib.mi_adamw_scale_grads(
            launch.rows.data_ptr(), launch.chunks.data_ptr(), launch.n_chunks, _CHUNK,
            coef.data_ptr(), stream), "mi_adamw_scale_grads")
    return norm
