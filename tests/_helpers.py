"""Shared helpers for the parity tests: seeded parameter sets and ulp metrics.

Seeds follow one scheme everywhere: tensor i of a set draws from a generator
seeded with base + i (params 1000, exp_avg 2000, exp_avg_sq 3000, grads
4000 + 10000 * step), on the device the tensors live on.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from mi_adamw.workloads import GPTShape, init_kind


def seeds(default: int) -> range:
    """The seeds of a seeded random test: range(default), or, for a wider sweep, the range
    that the environment variable MI_ADAMW_SEEDS names as "lo:hi" (hi excluded)."""
    spec = os.environ.get("MI_ADAMW_SEEDS")
    if not spec:
        return range(default)
    lo, hi = (int(x) for x in spec.split(":"))
    if not 0 <= lo < hi:
        raise ValueError(f"MI_ADAMW_SEEDS={spec!r}: expected lo:hi with 0 <= lo < hi")
    return range(lo, hi)


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether two tensors of one 16-bit dtype (a bf16 copy and the bf16 of its master)
    hold the same bits.  Unlike torch.equal, a NaN equals a NaN of the same bits: torch's
    capturable chain with lr = 0 forms NaN where a second moment is 0, and so do the
    kernels, so the copy holds the bf16 NaN of that master."""
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.int16),
                                              b.contiguous().view(torch.int16))


def gen(device, seed: int) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def make_params(shapes, device, names=None, seed: int = 1000) -> list[torch.nn.Parameter]:
    """fp32 params: LayerNorm weights 1, biases 0, everything else N(0, 0.02)."""
    out = []
    for i, shape in enumerate(shapes):
        kind = init_kind(names[i]) if names else "normal"
        if kind == "ones":
            t = torch.ones(shape, device=device)
        elif kind == "zeros":
            t = torch.zeros(shape, device=device)
        else:
            t = torch.randn(shape, device=device, generator=gen(device, seed + i)) * 0.02
        out.append(torch.nn.Parameter(t))
    return out


def gpt_params(shape: GPTShape, device) -> list[torch.nn.Parameter]:
    named = shape.tensors()
    return make_params([s for _, s in named], device, names=[n for n, _ in named])


def set_grads(params, step: int, std: float, base: int = 4000) -> None:
    for i, p in enumerate(params):
        g = torch.randn(p.shape, device=p.device, generator=gen(p.device, base + 10000 * step + i))
        g.mul_(std)
        if p.grad is None:
            p.grad = g
        else:
            p.grad.copy_(g)


def midtrain_state(params, step: float = 1000.0, dtype=torch.float32):
    """m ~ N(0, 1e-3), v ~ |N(0, 1e-6)| (std), stored step."""
    states = []
    for i, p in enumerate(params):
        m = torch.randn(p.shape, device=p.device, generator=gen(p.device, 2000 + i)) * 1e-3
        v = (torch.randn(p.shape, device=p.device, generator=gen(p.device, 3000 + i)) * 1e-6).abs()
        states.append({"step": torch.tensor(float(step)), "exp_avg": m.to(dtype),
                       "exp_avg_sq": v.to(dtype)})
    return states


def load_states(opt, params, states) -> None:
    """Install explicit (step, exp_avg, exp_avg_sq) states through load_state_dict."""
    sd = opt.state_dict()
    sd["state"] = {i: {k: (v.clone() if isinstance(v, torch.Tensor) else v)
                       for k, v in st.items()} for i, st in enumerate(states)}
    opt.load_state_dict(sd)


def clone_params(params) -> list[torch.nn.Parameter]:
    out = []
    for p in params:
        q = torch.nn.Parameter(p.detach().clone())
        if p.grad is not None:
            q.grad = p.grad.detach().clone()
        out.append(q)
    return out


def _mono(x: torch.Tensor) -> torch.Tensor:
    i = x.detach().contiguous().view(torch.int32).to(torch.int64)
    return torch.where(i < 0, -(2 ** 31) - i, i)


def max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    """Largest ulp distance between two fp32 tensors (NaN == NaN)."""
    a = a.detach().float().reshape(-1)
    b = b.detach().float().reshape(-1)
    both_nan = torch.isnan(a) & torch.isnan(b)
    d = (_mono(a) - _mono(b)).abs()
    d = torch.where(both_nan, torch.zeros_like(d), d)
    return int(d.max().item()) if d.numel() else 0


def max_ulp_all(xs, ys) -> int:
    return max((max_ulp(x, y) for x, y in zip(xs, ys)), default=0)


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Elementwise relative error max |a-b| / max(|b|, tiny), in float64."""
    a = a.detach().double().reshape(-1)
    b = b.detach().double().reshape(-1)
    return float(((a - b).abs() / b.abs().clamp_min(1e-30)).max().item()) if a.numel() else 0.0


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def close_rel(a: torch.Tensor, b: torch.Tensor, rtol: float, floor: float) -> float:
    """Largest |a-b| / (rtol*|b| + floor); <= 1 means within tolerance.

    The floor covers elements where the update nearly cancels the decayed
    parameter: a relative perturbation of the update (for example from a clip
    coefficient 1 ulp apart) then shows as a large relative error on a tiny
    result, while its absolute size stays below rtol times the step size.
    """
    a = a.detach().double().reshape(-1)
    b = b.detach().double().reshape(-1)
    if a.numel() == 0:
        return 0.0
    both_nan = torch.isnan(a) & torch.isnan(b)
    r = (a - b).abs() / (rtol * b.abs() + floor)
    r = torch.where(both_nan, torch.zeros_like(r), r)
    return float(r.max().item())


def rms(t: torch.Tensor) -> float:
    t = t.detach().double()
    return float(t.pow(2).mean().sqrt().item()) if t.numel() else 0.0
