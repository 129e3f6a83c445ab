"""GPU: seeded random configurations of FusedAdamW against torch.optim.AdamW, bit for bit.

Each seed draws a parameter set and an optimizer configuration the fixed-case tests
cover one at a time, then runs a few chained steps of both optimizers on the same
values:

* 1-10 tensors, 1-D and 2-D, sizes around the 4-element vector width and the
  4096-element chunk (1, 3, 31-33, 4095-4097, 65537 ...);
* parameters and gradients that are views at 1-3 element offsets into a larger
  buffer (not 16-byte aligned: the scalar path);
* 1-3 param groups with their own lr (0 included), betas (the other lerp branch
  included), eps, weight decay, maximize and amsgrad (adam.py:396-547);
* the fused clip (clip_grad.py:50-183) or none, chunk sizes 4096-65536, the default
  or the capturable chain (adam.py:480-527);
* params that have no gradient at some steps (skipped, their step counts stay).

torch's clip computes its norm in fp32; the reference applies our float64 norm with
clip_grads_with_norm_ (torch's own scaling), so the update is compared bit for bit.
With bf16 moments and the bf16 copy, which torch has no counterpart for, the same kind
of draws are checked against the oracle's bf16-state model instead.
"""
from __future__ import annotations

import random
import warnings

import numpy as np
import pytest
import torch

from _helpers import max_ulp, same_bits, seeds

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 31, 32, 33, 1000, 4095, 4096, 4097, 8191, 12289, 65537]
BETAS = [(0.9, 0.999), (0.9, 0.95), (0.5, 0.9), (0.2, 0.99)]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    return torch.device("cuda", 0)


def _shape(rng: random.Random) -> tuple:
    if rng.random() < 0.6:
        return (rng.choice(SIZES),)
    return (rng.choice([1, 3, 17, 64]), rng.choice([1, 5, 64, 129]))


def _placed(values: torch.Tensor, offset: int) -> torch.Tensor:
    """values copied into a fresh buffer at `offset` elements (a contiguous view)."""
    if offset == 0:
        return values.clone()
    store = torch.zeros(values.numel() + offset + 7, device=values.device)
    v = store[offset:offset + values.numel()].view(values.shape)
    v.copy_(values)
    return v


@pytest.mark.parametrize("seed", seeds(24))
def test_random_configuration_matches_torch(dev, seed):
    import mi_adamw
    rng = random.Random(seed)
    g = torch.Generator(device=dev).manual_seed(seed)
    shapes = [_shape(rng) for _ in range(rng.randint(1, 10))]
    offsets = [rng.choice([0, 0, 0, 1, 2, 3]) for _ in shapes]
    n_groups = rng.randint(1, min(3, len(shapes)))
    group_of = [rng.randrange(n_groups) for _ in shapes]
    hp = [dict(lr=rng.choice([0.0, 1e-4, 3e-4, 6e-4, 1e-2]), betas=rng.choice(BETAS),
               eps=rng.choice([1e-8, 1e-6]), weight_decay=rng.choice([0.0, 0.01, 0.1]),
               maximize=rng.random() < 0.3, amsgrad=rng.random() < 0.3)
          for _ in range(n_groups)]
    clip = rng.choice([None, None, 0.05, 1.0, 1e3])
    chunk = rng.choice([4096, 8192, 65536])
    capturable = rng.random() < 0.3
    gstd = rng.choice([1e-4, 1e-2, 1.0])
    print(f"seed {seed}: shapes {shapes} offsets {offsets} groups {group_of} {hp} clip {clip} "
          f"chunk {chunk} capturable {capturable}", flush=True)

    values = [torch.randn(s, device=dev, generator=g) * 0.02 for s in shapes]
    ref = [torch.nn.Parameter(v.clone()) for v in values]
    ours = [torch.nn.Parameter(_placed(v, o)) for v, o in zip(values, offsets)]

    def groups(ps):
        return [dict(params=[p for p, gi in zip(ps, group_of) if gi == k], **hp[k])
                for k in range(n_groups) if k in group_of]

    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
        topt = torch.optim.AdamW(groups(ref), foreach=False, capturable=capturable)
        oopt = mi_adamw.FusedAdamW(groups(ours), capturable=capturable, max_grad_norm=clip,
                                   chunk_elems=chunk)
        for step in range(1, rng.randint(2, 5)):
            for i, (p, q) in enumerate(zip(ref, ours)):
                if step > 1 and rng.random() < 0.15:
                    p.grad = None
                    q.grad = None
                    continue
                grad = torch.randn(shapes[i], device=dev, generator=g) * gstd
                p.grad = grad.clone()
                q.grad = _placed(grad, offsets[i] if rng.random() < 0.5 else 0)
            if all(p.grad is None for p in ref):
                continue
            oopt.step()
            if clip is not None:
                torch.nn.utils.clip_grads_with_norm_(ref, clip, oopt.last_grad_norm.clone())
            topt.step()
            torch.cuda.synchronize()
            for i, (p, q) in enumerate(zip(ref, ours)):
                assert max_ulp(p, q) == 0, (seed, step, i, "param")
                ts, os_ = topt.state.get(p, {}), oopt.state.get(q, {})
                assert ts.keys() == os_.keys(), (seed, step, i)
                for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
                    if key in ts:
                        assert max_ulp(ts[key], os_[key]) == 0, (seed, step, i, key)
                if "step" in ts:
                    assert float(ts["step"]) == float(os_["step"]), (seed, step, i, "step")


def _torch_den(b1, b2, lr, eps, step, dev):
    """torch's per-step values of the capturable chain (adam.py:480-522) as the same
    0-d tensor ops on the GPU: (sqrt(bc2) * -step_size, eps / -step_size)."""
    step_t = torch.tensor(float(step), device=dev)
    bc1 = 1 - b1 ** step_t
    bc2 = 1 - b2 ** step_t
    neg = (lr / bc1).neg()
    return float(bc2.sqrt() * neg), float(eps / neg)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view("uint16").reshape(-1).copy()


@pytest.mark.parametrize("seed", seeds(12))
def test_random_bf16_state_configuration_matches_oracle(dev, seed):
    """bf16 moments (and amsgrad maximum) with the bf16 copy, which torch has no
    counterpart for: every tensor after every step equals the oracle's bf16-state
    model (default or capturable chain) applied to the tensor's values before the
    step, with the clip coefficient from the step's own norm."""
    import mi_adamw
    from oracle import oracle as O
    rng = random.Random(1000 + seed)
    g = torch.Generator(device=dev).manual_seed(1000 + seed)
    shapes = [_shape(rng) for _ in range(rng.randint(1, 8))]
    offsets = [rng.choice([0, 0, 1, 2, 3]) for _ in shapes]
    n_groups = rng.randint(1, min(3, len(shapes)))
    group_of = [rng.randrange(n_groups) for _ in shapes]
    hp = [dict(lr=rng.choice([0.0, 1e-4, 6e-4, 1e-2]), betas=rng.choice(BETAS),
               eps=rng.choice([1e-8, 1e-6]), weight_decay=rng.choice([0.0, 0.1]),
               maximize=rng.random() < 0.3, amsgrad=rng.random() < 0.3)
          for _ in range(n_groups)]
    clip = rng.choice([None, 0.05, 1e3])
    chunk = rng.choice([4096, 8192, 65536])
    capturable = rng.random() < 0.4
    gstd = rng.choice([1e-4, 1e-2, 1.0])
    print(f"seed {seed}: shapes {shapes} offsets {offsets} groups {group_of} {hp} clip {clip} "
          f"chunk {chunk} capturable {capturable}", flush=True)
    ours = [torch.nn.Parameter(_placed(torch.randn(s, device=dev, generator=g) * 0.02, o))
            for s, o in zip(shapes, offsets)]
    groups = [dict(params=[p for p, gi in zip(ours, group_of) if gi == k], **hp[k])
              for k in range(n_groups) if k in group_of]
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
        opt = mi_adamw.FusedAdamW(groups, state_dtype=torch.bfloat16, bf16_copy=True,
                                  capturable=capturable, max_grad_norm=clip, chunk_elems=chunk)
        for step in range(1, rng.randint(2, 5)):
            for i, q in enumerate(ours):
                if step > 1 and rng.random() < 0.15:
                    q.grad = None
                    continue
                grad = torch.randn(shapes[i], device=dev, generator=g) * gstd
                q.grad = _placed(grad, offsets[i] if rng.random() < 0.5 else 0)
            if all(q.grad is None for q in ours):
                continue
            before = []
            for q in ours:
                st = opt.state.get(q, {})
                n = q.numel()
                zero = np.zeros(n, dtype=np.uint16)
                before.append((q.detach().cpu().numpy().reshape(-1).copy(),
                               _bits(st["exp_avg"]) if "exp_avg" in st else zero.copy(),
                               _bits(st["exp_avg_sq"]) if "exp_avg_sq" in st else zero.copy(),
                               _bits(st["max_exp_avg_sq"]) if "max_exp_avg_sq" in st
                               else zero.copy(),
                               float(st["step"]) if "step" in st else 0.0))
            opt.step()
            torch.cuda.synchronize()
            coef = None
            if clip is not None:
                coef = O.clip_coef(np.float32(opt.last_grad_norm.item()), clip)
            for i, q in enumerate(ours):
                if q.grad is None:
                    continue
                h = hp[group_of[i]]
                p, mb, vb, xb, s0 = before[i]
                gr = q.grad.detach().cpu().numpy().reshape(-1).copy()
                kw = dict(lr=h["lr"], betas=h["betas"], eps=h["eps"],
                          weight_decay=h["weight_decay"], step=s0 + 1, maximize=h["maximize"],
                          grad_scale=coef, vmax_bits=xb if h["amsgrad"] else None)
                if capturable:
                    O.adamw_step_capt_bf16state(
                        p, gr, mb, vb, den=_torch_den(*h["betas"], h["lr"], h["eps"], s0 + 1, dev),
                        **kw)
                else:
                    O.adamw_step_bf16state(p, gr, mb, vb, **kw)
                st = opt.state[q]
                assert O.max_ulp(p, q.detach().cpu().numpy().reshape(-1))[0] == 0, (seed, step, i)
                assert np.array_equal(mb, _bits(st["exp_avg"])), (seed, step, i, "m")
                assert np.array_equal(vb, _bits(st["exp_avg_sq"])), (seed, step, i, "v")
                if h["amsgrad"]:
                    assert np.array_equal(xb, _bits(st["max_exp_avg_sq"])), (seed, step, i)
                assert float(st["step"]) == s0 + 1
                assert same_bits(opt.bf16_param(q), q.detach().to(torch.bfloat16))


@pytest.mark.parametrize("seed", seeds(8))
def test_random_clip_grad_norm_matches_torch(dev, seed):
    """mi_adamw.clip_grad_norm_ over random ragged and misaligned gradients: the norm
    equals the float64 norm of the fp32 gradients (rounded to fp32) and is within 1e-6
    of torch's fp32 norm; the scaled gradients equal clip_grads_with_norm_'s with that
    norm, bit for bit."""
    import mi_adamw
    from oracle import oracle as O
    rng = random.Random(2000 + seed)
    g = torch.Generator(device=dev).manual_seed(2000 + seed)
    shapes = [_shape(rng) for _ in range(rng.randint(1, 12))]
    scale = rng.choice([1e-6, 1e-3, 1.0, 1e3])
    max_norm = rng.choice([0.01, 1.0, 1e6])
    grads = [torch.randn(s, device=dev, generator=g) * scale for s in shapes]
    ours = [torch.nn.Parameter(torch.zeros(s, device=dev)) for s in shapes]
    ref = [torch.nn.Parameter(torch.zeros(s, device=dev)) for s in shapes]
    for q, p, gr in zip(ours, ref, grads):
        q.grad = _placed(gr, rng.choice([0, 0, 1, 2, 3]))
        p.grad = gr.clone()
    exact = O.total_norm([gr.cpu().numpy() for gr in grads])
    norm = mi_adamw.clip_grad_norm_(ours, max_norm)
    tnorm = torch.nn.utils.get_total_norm([p.grad for p in ref])
    torch.nn.utils.clip_grads_with_norm_(ref, max_norm, norm.clone())
    torch.cuda.synchronize()
    print(f"seed {seed}: {len(shapes)} tensors, scale {scale}, max_norm {max_norm}: norm "
          f"{norm.item():.9g} float64 {float(exact):.9g} torch {tnorm.item():.9g}", flush=True)
    assert np.float32(norm.item()) == exact
    assert abs(norm.item() - tnorm.item()) <= 1e-6 * tnorm.item()
    for q, p in zip(ours, ref):
        assert max_ulp(q.grad, p.grad) == 0
