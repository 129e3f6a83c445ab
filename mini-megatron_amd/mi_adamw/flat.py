"""Flat-buffer layout: every parameter, gradient and moment packed contiguously.

mini-megatron's ZeRO-1 optimizer (parallel/distributed_optimizer.py:7-48)
assigns whole tensors to data-parallel ranks round-robin and steps a per-rank
torch AdamW over them.  The flat layout here is the single-GPU building block
of a range-sharded ZeRO-1: each param group occupies one contiguous range of
four flat buffers (params, grads, exp_avg, exp_avg_sq), plus an optional bf16
model copy and, once a group uses amsgrad, max_exp_avg_sq.  Every tensor starts
at a 128-byte-aligned offset (32 fp32 elements), and the step of a group is
one contiguous range for the kernel.

Parameters become views of the flat parameter buffer (``p.data`` is replaced)
and gradients stay allocated as views of the flat gradient buffer, so
backward accumulates straight into it.  Consequence: every parameter whose
``p.grad`` is a view is stepped every step, exactly as torch.optim.AdamW does
after ``zero_grad(set_to_none=False)``.  A parameter whose grad was set to
None is skipped (torch semantics); a gradient tensor that autograd allocated
elsewhere is copied into the buffer at the next step.  So are new values given
through ``p.data = t`` and moments put into the state dict directly: the step
copies them into the tensor's slice and points ``p.data`` (or the state entry)
back at the slice, so the results equal torch's for p while t itself is no
longer p's storage.  A tensor whose element count changed cannot be taken back
into its slice and is refused.
"""
from __future__ import annotations

import torch

ALIGN_ELEMS = 32  # 128 bytes of fp32


def _align(n: int) -> int:
    return (n + ALIGN_ELEMS - 1) // ALIGN_ELEMS * ALIGN_ELEMS


class FlatLayout:
    def __init__(self, param_groups, state_dtype: torch.dtype, bf16_copy: bool):
        params = [p for g in param_groups for p in g["params"]]
        if not params:
            raise ValueError("flat_buffer=True needs at least one parameter")
        device = params[0].device
        for p in params:
            if p.dtype != torch.float32:
                raise NotImplementedError("flat_buffer=True supports fp32 parameters only")
            if p.device != device:
                raise NotImplementedError("flat_buffer=True needs every parameter on one device")
        if device.type != "cuda":
            raise RuntimeError("flat_buffer=True needs parameters on a ROCm GPU")
        self.device = device
        self.offsets: dict[int, int] = {}
        self.numels: dict[int, int] = {}
        self.group_ranges: list[tuple[int, int]] = []
        off = 0
        for g in param_groups:
            start = off
            for p in g["params"]:
                self.offsets[id(p)] = off
                self.numels[id(p)] = p.numel()
                off = _align(off + p.numel())
            self.group_ranges.append((start, off))
        self.total = off
        self.param = torch.zeros(off, dtype=torch.float32, device=device)
        self.grad = torch.zeros(off, dtype=torch.float32, device=device)
        self.exp_avg = torch.zeros(off, dtype=state_dtype, device=device)
        self.exp_avg_sq = torch.zeros(off, dtype=state_dtype, device=device)
        self.copy = torch.zeros(off, dtype=torch.bfloat16, device=device) if bf16_copy else None
        self.max_exp_avg_sq: torch.Tensor | None = None   # allocated on first amsgrad use
        self._copy_views: dict[int, torch.Tensor] = {}
        with torch.no_grad():
            for p in params:
                view = self._view(self.param, p)
                view.copy_(p.detach())
                p.data = view
                gview = self._view(self.grad, p)
                if p.grad is not None:
                    gview.copy_(p.grad)
                p.grad = gview
            if self.copy is not None:
                self.copy.copy_(self.param)

    def _view(self, buf: torch.Tensor, p: torch.Tensor) -> torch.Tensor:
        # the slice has the element count p had when the buffer was laid out; a p since
        # resized through .data no longer fits and view() raises
        off = self.offsets[id(p)]
        return buf[off:off + self.numels[id(p)]].view(p.shape)

    def grad_view(self, p: torch.Tensor) -> torch.Tensor:
        return self._view(self.grad, p)

    def is_grad_view(self, p: torch.Tensor, g: torch.Tensor) -> bool:
        off = self.offsets[id(p)]
        return g.data_ptr() == self.grad.data_ptr() + 4 * off and g.is_contiguous()

    def absorb_grad(self, p: torch.Tensor) -> torch.Tensor:
        """Copy a gradient allocated outside the buffer into it; p.grad becomes the view."""
        view = self.grad_view(p)
        view.copy_(p.grad)
        p.grad = view
        return view

    def _check_size(self, p: torch.Tensor, t: torch.Tensor, what: str) -> None:
        n = self.numels[id(p)]
        if t.numel() != n:
            raise RuntimeError(f"flat_buffer=True: {what} has {t.numel()} elements but the "
                               f"buffer holds {n} for this parameter")

    def is_param_view(self, p: torch.Tensor) -> bool:
        return (p.data_ptr() == self.param.data_ptr() + 4 * self.offsets[id(p)]
                and p.numel() == self.numels[id(p)] and p.is_contiguous())

    def absorb_param(self, p: torch.Tensor) -> None:
        """Values given to p through ``p.data = t`` are copied into its slice of the
        parameter buffer and p.data becomes the slice again (the step updates the slice,
        as it does every other parameter; t itself is no longer p's storage)."""
        self._check_size(p, p, "the parameter's new data")
        if p.dtype != torch.float32 or p.device != self.device:
            raise NotImplementedError("flat_buffer=True: a parameter's new data must be fp32 "
                                      "on the buffer's device")
        view = self._view(self.param, p)
        view.copy_(p.detach())
        p.data = view

    def absorb_state(self, p: torch.Tensor, st: dict) -> None:
        """State tensors put into p's state dict directly (not through load_state_dict)
        are copied into p's slices of the moment buffers, which the step updates."""
        off = self.offsets[id(p)]
        for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
            t = st.get(key)
            if t is None:
                continue
            buf = (self.exp_avg if key == "exp_avg" else self.exp_avg_sq
                   if key == "exp_avg_sq" else self.max_exp_avg_sq)
            if (buf is not None and t.data_ptr() == buf.data_ptr() + buf.element_size() * off
                    and t.numel() == self.numels[id(p)] and t.is_contiguous()):
                continue
            st[key] = self.adopt_state(p, key, t)

    def state_views(self, p: torch.Tensor):
        return self._view(self.exp_avg, p), self._view(self.exp_avg_sq, p)

    def vmax_view(self, p: torch.Tensor) -> torch.Tensor:
        """p's slice of the max_exp_avg_sq buffer (amsgrad), allocating the buffer once."""
        if self.max_exp_avg_sq is None:
            self.max_exp_avg_sq = torch.zeros_like(self.exp_avg_sq)
        return self._view(self.max_exp_avg_sq, p)

    def adopt_state(self, p: torch.Tensor, key: str, t: torch.Tensor) -> torch.Tensor:
        if key == "max_exp_avg_sq":
            view = self.vmax_view(p)
        else:
            view = self._view(self.exp_avg if key == "exp_avg" else self.exp_avg_sq, p)
        self._check_size(p, t, f"state[{key!r}]")
        src = t.reshape(view.shape)
        if src.untyped_storage().data_ptr() == view.untyped_storage().data_ptr():
            # the slice's own memory read in another order (re-strided in place): copy
            # the values out first, so that no element is overwritten before it is read
            src = src.clone()
        view.copy_(src)
        return view

    def copy_view(self, p: torch.Tensor) -> torch.Tensor:
        """p's slice of the bf16 copy buffer (made once per buffer: adopt_buffers, which
        replaces the buffer, drops the slices made of the old one)."""
        v = self._copy_views.get(id(p))
        if v is None:
            v = self._copy_views[id(p)] = self._view(self.copy, p)
        return v

    def _holds(self, buf: torch.Tensor, p: torch.Tensor, t: torch.Tensor | None) -> bool:
        """t is p's slice of buf (a dense view at p's offset with p's element count)."""
        off = self.offsets[id(p)]
        return (t is not None and t.data_ptr() == buf.data_ptr() + buf.element_size() * off
                and t.numel() == self.numels[id(p)] and t.is_contiguous())

    @torch.no_grad()
    def adopt_buffers(self, bufs: dict, params, state) -> None:
        """Move the values of the buffers named in `bufs` ("param", "exp_avg", "exp_avg_sq",
        "copy") into the given tensors of the same size and dtype, and point everything
        that was a view of an old buffer (parameters' .data, state entries) at the new
        one.  A parameter or state entry that was not a view stays as it is; the next step
        takes its values into the new slice, as it would have into the old one."""
        old = {name: getattr(self, name) for name in bufs}
        for name, new in bufs.items():
            if new.shape != old[name].shape or new.dtype != old[name].dtype:
                raise ValueError(f"adopt_buffers: {name} differs in size or dtype")
        was = {}
        for p in params:
            st = state.get(p) or {}
            was[id(p)] = {"param": "param" in bufs and self._holds(old["param"], p, p)}
            for key in ("exp_avg", "exp_avg_sq"):
                was[id(p)][key] = key in bufs and self._holds(old[key], p, st.get(key))
        for name, new in bufs.items():
            if new is not old[name]:
                new.copy_(old[name])
            setattr(self, name, new)
        self._copy_views = {}
        for p in params:
            if was[id(p)]["param"]:
                p.data = self._view(self.param, p)
            st = state.get(p)
            for key in ("exp_avg", "exp_avg_sq"):
                if was[id(p)][key]:
                    st[key] = self._view(getattr(self, key), p)

    def zero_grads(self, param_groups) -> None:
        self.grad.zero_()
        for g in param_groups:
            for p in g["params"]:
                if p.grad is None or not self.is_grad_view(p, p.grad):
                    p.grad = self.grad_view(p)

    def group_row(self, gi: int, amsgrad: bool = False):
        """(param, grad, exp_avg, exp_avg_sq, copy, max_exp_avg_sq) pointers and length
        of group gi's range; max_exp_avg_sq is 0 unless amsgrad."""
        start, end = self.group_ranges[gi]
        s_item = self.exp_avg.element_size()
        vmax = 0
        if amsgrad:
            if self.max_exp_avg_sq is None:
                raise RuntimeError("flat layout: amsgrad state was never initialised")
            vmax = self.max_exp_avg_sq.data_ptr() + s_item * start
        return (self.param.data_ptr() + 4 * start, self.grad.data_ptr() + 4 * start,
                self.exp_avg.data_ptr() + s_item * start,
                self.exp_avg_sq.data_ptr() + s_item * start,
                0 if self.copy is None else self.copy.data_ptr() + 2 * start,
                vmax, end - start)
