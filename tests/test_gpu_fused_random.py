"""GPU: seeded random configurations of FusedAdamW(fused=True) against
torch.optim.AdamW(fused=True), bit for bit.

The draws are those of the default chain's random test, with the fused=True chain on
both sides (torch/optim/adam.py:803-895, ``torch._fused_adamw_``):

* 1-10 tensors, 1-D and 2-D, sizes around the 4-element vector width and the
  4096-element chunk, views at 1-3 element offsets into a larger buffer;
* 1-3 param groups with their own lr (0 included), betas, eps, weight decay, maximize
  and amsgrad;
* step counts loaded mid-training, anywhere in 1 .. 2e6, per parameter (the per-step
  values are formed in float64 from each tensor's own count);
* the fused clip or none, chunk sizes 4096-65536, the default or the capturable chain
  (device step counts, per-step values formed on the device);
* params that have no gradient at some steps.

With bf16 moments and the bf16 copy, which torch's fused kernel does not offer, the same
kind of draws are checked against the oracle's fused chain on bf16-stored moments.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from _helpers import max_ulp, same_bits, seeds

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 31, 32, 33, 1000, 4095, 4096, 4097, 8191, 12289, 65537]
BETAS = [(0.9, 0.999), (0.9, 0.95), (0.5, 0.9), (0.2, 0.99), (0.0, 0.5)]


@pytest.fixture(scope="module")
def dev():
    import mi_adamw  # noqa: F401  (loads the library; raises without it)
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


def _draw(rng, n_max):
    shapes = [_shape(rng) for _ in range(rng.randint(1, n_max))]
    offsets = [rng.choice([0, 0, 0, 1, 2, 3]) for _ in shapes]
    n_groups = rng.randint(1, min(3, len(shapes)))
    group_of = [rng.randrange(n_groups) for _ in shapes]
    hp = [dict(lr=rng.choice([0.0, 1e-5, 3e-4, 6e-4, 1e-2]), betas=rng.choice(BETAS),
               eps=rng.choice([1e-8, 1e-6, 1e-12]), weight_decay=rng.choice([0.0, 0.01, 0.1]),
               maximize=rng.random() < 0.3, amsgrad=rng.random() < 0.3, fused=True)
          for _ in range(n_groups)]
    steps = [float(rng.choice([0, 0, 3, 999, 65535, rng.randint(1, 2_000_000)]))
             for _ in shapes]
    return shapes, offsets, n_groups, group_of, hp, steps


def _groups(ps, group_of, hp, n_groups):
    return [dict(params=[p for p, gi in zip(ps, group_of) if gi == k], **hp[k])
            for k in range(n_groups) if k in group_of]


def _states(order, shapes, steps, hp, group_of, g, state_dtype=torch.float32):
    """Mid-training state for every parameter, in the optimizer's parameter order; a
    parameter whose drawn step is 0 starts without state (lazy init at its first step)."""
    out = {}
    for pos, i in enumerate(order):
        if steps[i] == 0:
            continue
        m = torch.randn(shapes[i], device=g.device, generator=g) * 1e-3
        v = (torch.randn(shapes[i], device=g.device, generator=g) * 1e-6).abs()
        st = {"step": torch.tensor(steps[i]), "exp_avg": m.to(state_dtype),
              "exp_avg_sq": v.to(state_dtype)}
        if hp[group_of[i]]["amsgrad"]:
            x = v * 1.5
            x.view(-1)[::2] = 0
            st["max_exp_avg_sq"] = x.to(state_dtype)
        out[pos] = st
    return out


def _load(opt, states):
    sd = opt.state_dict()
    sd["state"] = {k: {n: t.clone() for n, t in st.items()} for k, st in states.items()}
    opt.load_state_dict(sd)


@pytest.mark.filterwarnings("ignore:This instance was constructed with capturable=True")
@pytest.mark.parametrize("seed", seeds(24))
def test_random_fused_configuration_matches_torch_fused(dev, seed):
    import mi_adamw
    rng = random.Random(5000 + seed)
    g = torch.Generator(device=dev).manual_seed(5000 + seed)
    shapes, offsets, n_groups, group_of, hp, steps = _draw(rng, 10)
    clip = rng.choice([None, None, 0.05, 1.0, 1e3])
    chunk = rng.choice([4096, 8192, 65536])
    capturable = rng.random() < 0.3
    gstd = rng.choice([1e-4, 1e-2, 1.0])
    print(f"seed {seed}: shapes {shapes} offsets {offsets} groups {group_of} {hp} steps {steps} "
          f"clip {clip} chunk {chunk} capturable {capturable}", flush=True)
    values = [torch.randn(s, device=dev, generator=g) * 0.02 for s in shapes]
    ref = [torch.nn.Parameter(v.clone()) for v in values]
    ours = [torch.nn.Parameter(_placed(v, o)) for v, o in zip(values, offsets)]
    topt = torch.optim.AdamW(_groups(ref, group_of, hp, n_groups), capturable=capturable)
    oopt = mi_adamw.FusedAdamW(_groups(ours, group_of, hp, n_groups), capturable=capturable,
                               max_grad_norm=clip, chunk_elems=chunk)
    order = [i for k in range(n_groups) for i, gi in enumerate(group_of) if gi == k]
    states = _states(order, shapes, steps, hp, group_of, g)
    _load(topt, states)
    _load(oopt, states)
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


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view("uint16").reshape(-1).copy()


@pytest.mark.filterwarnings("ignore:This instance was constructed with capturable=True")
@pytest.mark.parametrize("seed", seeds(12))
def test_random_fused_bf16_state_configuration_matches_oracle(dev, seed):
    """bf16 moments (and amsgrad maximum) with the bf16 copy in the fused=True chain:
    every tensor after every step equals the oracle's fused chain on bf16-stored moments
    applied to the tensor's values before the step, with the clip coefficient from the
    step's own norm."""
    import mi_adamw
    from oracle import oracle as O
    rng = random.Random(6000 + seed)
    g = torch.Generator(device=dev).manual_seed(6000 + seed)
    shapes, offsets, n_groups, group_of, hp, steps = _draw(rng, 8)
    clip = rng.choice([None, 0.05, 1e3])
    chunk = rng.choice([4096, 8192, 65536])
    capturable = rng.random() < 0.4
    gstd = rng.choice([1e-4, 1e-2, 1.0])
    print(f"seed {seed}: shapes {shapes} offsets {offsets} groups {group_of} {hp} steps {steps} "
          f"clip {clip} chunk {chunk} capturable {capturable}", flush=True)
    ours = [torch.nn.Parameter(_placed(torch.randn(s, device=dev, generator=g) * 0.02, o))
            for s, o in zip(shapes, offsets)]
    opt = mi_adamw.FusedAdamW(_groups(ours, group_of, hp, n_groups), state_dtype=torch.bfloat16,
                              bf16_copy=True, capturable=capturable, max_grad_norm=clip,
                              chunk_elems=chunk)
    order = [i for k in range(n_groups) for i, gi in enumerate(group_of) if gi == k]
    _load(opt, _states(order, shapes, steps, hp, group_of, g, torch.bfloat16))
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
            zero = np.zeros(q.numel(), dtype=np.uint16)
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
            O.adamw_step_fused_bf16state(p, gr, mb, vb, lr=h["lr"], betas=h["betas"],
                                         eps=h["eps"], weight_decay=h["weight_decay"],
                                         step=s0 + 1, maximize=h["maximize"], grad_scale=coef,
                                         vmax_bits=xb if h["amsgrad"] else None)
            st = opt.state[q]
            assert O.max_ulp(p, q.detach().cpu().numpy().reshape(-1))[0] == 0, (seed, step, i)
            assert np.array_equal(mb, _bits(st["exp_avg"])), (seed, step, i, "m")
            assert np.array_equal(vb, _bits(st["exp_avg_sq"])), (seed, step, i, "v")
            if h["amsgrad"]:
                assert np.array_equal(xb, _bits(st["max_exp_avg_sq"])), (seed, step, i)
            assert float(st["step"]) == s0 + 1
            assert same_bits(opt.bf16_param(q), q.detach().to(torch.bfloat16))
