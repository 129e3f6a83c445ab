"""The memory ceiling of an optimizer's update, measured on its own tensors.

``time_probe(opt)`` runs ``mi_adamw_probe`` (or ``mi_adamw_probe_flat``) over the
launch tables of the optimizer's last step: the same tensors, launch shape, access
widths and cache hints as the update kernel, with the arithmetic left out and every
value stored back unchanged.  Where the step clips, each probe launch follows the
step's own norm pass, as the update does (the norm pass leaves the last gradients it
read in the Infinity Cache, and the update reads them from there).  The update's time
over the probe's is then what the AdamW arithmetic costs on top of the memory traffic
of its read/write mix on those pages.

A measurement helper: nothing on the optimizer's step path calls it.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def time_probe(opt, launches: int = 20) -> float | None:
    """Average ms of one probe launch, timed with HIP events on the current stream.
    None when the optimizer's last step needed more than one update launch (amsgrad and
    plain groups mixed, or more hyperparameter sets than one launch holds)."""
    cache = opt._launch_cache
    if cache is None:
        raise RuntimeError("time_probe: run one optimizer step first")
    device, launches_, norm_launch = cache.device, cache.launches, cache.norm_launch
    if len(launches_) != 1 or launches_[0].n_chunks == 0:
        return None
    launch = launches_[0]
    lib = _lib.load()
    flags = 0
    if opt.bf16_copy:
        flags |= _lib.F_BF16_COPY
    if opt.max_grad_norm is not None and opt.clip_write_grads:
        flags |= _lib.F_WRITE_GRAD
    if int(launch.host_rows["max_exp_avg_sq"].max()) != 0:
        flags |= _lib.F_AMSGRAD
    state = _lib.STATE_BF16 if opt.state_dtype == torch.bfloat16 else _lib.STATE_F32
    chunk = opt.chunk_elems
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        partials, coef = opt._ws(device)
        norm = torch.empty((), dtype=torch.float32, device=device)

        def norm_pass():
            if norm_launch.n_rows == 1 and not norm_launch.tables:
                row = opt._row_struct(norm_launch)
                _lib.check(lib.mi_adamw_grad_norm_flat(
                    row.grad, row.numel, chunk, float(opt.max_grad_norm), partials.data_ptr(),
                    norm.data_ptr(), coef.data_ptr(), stream), "mi_adamw_grad_norm_flat")
            else:
                _lib.check(lib.mi_adamw_grad_norm(
                    norm_launch.rows.data_ptr(), norm_launch.chunks.data_ptr(),
                    norm_launch.n_chunks, chunk, float(opt.max_grad_norm), partials.data_ptr(),
                    norm.data_ptr(), coef.data_ptr(), stream), "mi_adamw_grad_norm")

        def probe():
            if launch.n_rows == 1 and not launch.tables:
                row = opt._row_struct(launch)
                _lib.check(lib.mi_adamw_probe_flat(ctypes.byref(row), chunk, state, flags,
                                                   opt.max_blocks, stream), "mi_adamw_probe_flat")
            else:
                _lib.check(lib.mi_adamw_probe(launch.rows.data_ptr(), launch.chunks.data_ptr(),
                                              launch.n_chunks, chunk, state, flags,
                                              opt.max_blocks, stream), "mi_adamw_probe")

        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(launches)]
        probe()   # warm-up
        for e0, e1 in events:
            if opt.max_grad_norm is not None:
                norm_pass()
            e0.record()
            probe()
            e1.record()
        torch.cuda.synchronize(device)
    return sum(e0.elapsed_time(e1) for e0, e1 in events) / launches
