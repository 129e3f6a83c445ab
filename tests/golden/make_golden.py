"""Write the golden fixtures that pin the CPU oracle (tests/golden/adamw_golden.npz).

The expected values come from torch 2.10's own optimizer and clip on the CPU:
``torch.optim.AdamW(..., foreach=False)`` -- the per-tensor path mini-megatron
runs (main.py:177, fused=False) -- and ``torch.nn.utils.clip_grad_norm_``.
torch is the third-party library that holds the arithmetic of this path; the
reference repository itself has no optimizer arithmetic and no golden vectors
for it.  Inputs are seeded; every case stores its inputs and its outputs.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "adamw_golden.npz")
SHAPES = [(1000,), (37,), (48, 64), (3,)]


def _randn(shape, seed, std):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * std


def run_case(name, *, lr, betas, eps, wd, steps, gstd, maximize=False, clip=None,
             start_step=0, amsgrad=False, gdecay=1.0, store):
    params = [torch.nn.Parameter(_randn(s, 100 + i, 0.02)) for i, s in enumerate(SHAPES)]
    opt = torch.optim.AdamW(params, lr=lr, betas=betas, eps=eps, weight_decay=wd,
                            maximize=maximize, amsgrad=amsgrad, foreach=False)
    if start_step:
        for i, p in enumerate(params):
            opt.state[p]["step"] = torch.tensor(float(start_step))
            opt.state[p]["exp_avg"] = _randn(p.shape, 200 + i, 1e-3)
            opt.state[p]["exp_avg_sq"] = _randn(p.shape, 300 + i, 1e-6).abs()
            if amsgrad:
                # a running maximum that sits above v for about half the elements
                opt.state[p]["max_exp_avg_sq"] = torch.maximum(
                    opt.state[p]["exp_avg_sq"], _randn(p.shape, 400 + i, 1e-6).abs())
    for i, p in enumerate(params):
        store[f"{name}/p0/{i}"] = p.detach().numpy().copy()
        if start_step:
            store[f"{name}/m0/{i}"] = opt.state[p]["exp_avg"].numpy().copy()
            store[f"{name}/v0/{i}"] = opt.state[p]["exp_avg_sq"].numpy().copy()
            if amsgrad:
                store[f"{name}/vmax0/{i}"] = opt.state[p]["max_exp_avg_sq"].numpy().copy()
    norms = []
    for t in range(steps):
        for i, p in enumerate(params):
            # gdecay < 1 shrinks the gradients step by step, so v falls below its maximum
            p.grad = _randn(p.shape, 1000 * (t + 1) + i, gstd * gdecay ** t)
            store[f"{name}/g/{t}/{i}"] = p.grad.numpy().copy()
        if clip is not None:
            norms.append(float(torch.nn.utils.clip_grad_norm_(params, clip)))
        opt.step()
    for i, p in enumerate(params):
        store[f"{name}/p/{i}"] = p.detach().numpy().copy()
        store[f"{name}/m/{i}"] = opt.state[p]["exp_avg"].numpy().copy()
        store[f"{name}/v/{i}"] = opt.state[p]["exp_avg_sq"].numpy().copy()
        store[f"{name}/step/{i}"] = np.float32(opt.state[p]["step"].item())
        if amsgrad:
            store[f"{name}/vmax/{i}"] = opt.state[p]["max_exp_avg_sq"].numpy().copy()
    store[f"{name}/meta"] = np.array([lr, betas[0], betas[1], eps, wd, steps, float(maximize),
                                      -1.0 if clip is None else clip, start_step,
                                      float(amsgrad)], dtype=np.float64)
    if clip is not None:
        store[f"{name}/norms"] = np.array(norms, dtype=np.float32)


def clip_cases(store):
    """clip_grad_norm_ on several gradient sets: returned norm and clipped grads."""
    # (std, max_norm): norms ~6.4 (clipped), ~0.064 (not clipped), ~64 (clipped), ~0.64
    # against 0.25 (clipped, with the 1e-6 visible in fp32)
    for c, (std, max_norm) in enumerate([(1e-1, 1.0), (1e-3, 1.0), (1.0, 0.5), (1e-2, 0.25)]):
        params = [torch.nn.Parameter(torch.zeros(s)) for s in SHAPES]
        for i, p in enumerate(params):
            p.grad = _randn(p.shape, 5000 + 10 * c + i, std)
            store[f"clip{c}/g/{i}"] = p.grad.numpy().copy()
        norm = torch.nn.utils.clip_grad_norm_(params, max_norm)
        store[f"clip{c}/norm"] = np.float32(norm.item())
        store[f"clip{c}/max_norm"] = np.float64(max_norm)
        for i, p in enumerate(params):
            store[f"clip{c}/gc/{i}"] = p.grad.numpy().copy()


def main():
    torch.set_num_threads(1)
    store: dict[str, np.ndarray] = {}
    base = dict(eps=1e-8, steps=1, gstd=1e-3, store=store)
    run_case("step1_zero", lr=3e-4, betas=(0.9, 0.95), wd=0.1, **base)
    run_case("chain10_refcfg", lr=6e-4, betas=(0.9, 0.999), wd=0.1, eps=1e-8, steps=10, gstd=1e-3,
             store=store)
    # grads N(0, 0.1) over 4112 elements: norm ~6.4, so the clip scales every step
    run_case("midtrain_clip", lr=3e-4, betas=(0.9, 0.95), wd=0.1, eps=1e-8, steps=3, gstd=1e-1,
             clip=1.0, start_step=1000, store=store)
    # norm ~0.64 against max_norm 0.25: the 1e-6 in norm + 1e-6 is 16 ulp of the norm here
    run_case("small_norm_clip", lr=6e-4, betas=(0.9, 0.999), wd=0.1, eps=1e-8, steps=2, gstd=1e-2,
             clip=0.25, start_step=0, store=store)
    run_case("lerp_big", lr=1e-3, betas=(0.3, 0.95), wd=0.01, eps=1e-8, steps=3, gstd=1e-3,
             store=store)
    run_case("maximize", lr=3e-4, betas=(0.9, 0.95), wd=0.1, eps=1e-8, steps=2, gstd=1e-3,
             maximize=True, store=store)
    run_case("wd0", lr=6e-4, betas=(0.9, 0.999), wd=0.0, eps=1e-8, steps=2, gstd=1e-3, store=store)
    run_case("lr0", lr=0.0, betas=(0.9, 0.999), wd=0.1, eps=1e-8, steps=1, gstd=1e-3, store=store)
    # amsgrad from zero state with gradients shrinking 4x per step: after the first
    # steps v decays below its running maximum and the maximum drives the update
    run_case("amsgrad_decay", lr=6e-4, betas=(0.9, 0.95), wd=0.1, eps=1e-8, steps=5, gstd=1e-2,
             gdecay=0.25, amsgrad=True, store=store)
    # amsgrad mid-training with a stored maximum above v on about half the elements, clipped
    run_case("amsgrad_mid_clip", lr=3e-4, betas=(0.9, 0.999), wd=0.1, eps=1e-8, steps=3,
             gstd=1e-1, clip=1.0, start_step=1000, amsgrad=True, store=store)
    clip_cases(store)
    np.savez_compressed(OUT, **store)
    print(f"wrote {OUT}: {len(store)} arrays, torch {torch.__version__}")


if __name__ == "__main__":
    main()
