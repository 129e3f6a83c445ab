"""Seeded random step sequences through the native and general step paths, against torch.

Each step draws a change from what mini-megatron's loop and its users do between steps:
new gradient tensors (zero_grad + backward), the same gradient tensors refilled, a
gradient set to None, a state tensor replaced, ``p.data`` replaced, the learning rate
changed, a group's betas, eps, weight decay and maximize changed, amsgrad switched for a
group, the step on another stream, a checkpoint round trip, and (tables layout; the flat
one refuses it) a param group of new parameters added mid-training.  After every step
parameters and moments must equal torch.optim.AdamW (foreach=False, or fused=True on
both sides) bit for bit; the test also counts how many steps each path took.
"""
from __future__ import annotations

import copy
import gc
import random

import pytest
import torch

from _helpers import clone_params, gen, make_params, max_ulp_all, seeds

pytestmark = pytest.mark.gpu

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (1024,), (33,)]
ACTIONS = ["move", "move", "move", "refill", "none_grad", "state_replace", "data_replace",
           "lr", "hyper", "amsgrad", "stream", "checkpoint", "add_group"]


@pytest.fixture
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    yield torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()


def _state_diff(ref, ours, topt, oopt):
    keys = ("exp_avg", "exp_avg_sq", "max_exp_avg_sq")
    d = max_ulp_all(list(ref), list(ours))
    for p, q in zip(ref, ours):
        st, so = topt.state.get(p, {}), oopt.state.get(q, {})
        for k in keys:
            if k in st:
                d = max(d, max_ulp_all([st[k]], [so[k]]))
        if "step" in st:
            assert float(st["step"]) == float(so["step"])
    return d


@pytest.mark.parametrize("chain", ["default", "fused"])
@pytest.mark.parametrize("layout", ["tables", "flat"])
@pytest.mark.parametrize("seed", seeds(6))
def test_random_step_sequences(dev, seed, layout, chain):
    """In the flat layout the parameters, gradients and moments are views of its buffers:
    a replaced p.data, gradient or state tensor is copied into its slice at the next step,
    and the results must still equal torch's.  With chain "fused" both optimizers are
    built with fused=True (torch's _fused_adamw_ chain on both sides)."""
    import mi_adamw
    rng = random.Random(seed)
    clip = seed % 2 == 0
    ref = make_params(SHAPES, dev, seed=1000 + 100 * seed)
    ours = clone_params(ref)
    groups = lambda ps: [{"params": ps[:4], "amsgrad": True},      # noqa: E731
                         {"params": ps[4:], "lr": 1e-3, "weight_decay": 0.0, "amsgrad": True}]
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    fused = chain == "fused"
    topt = torch.optim.AdamW(groups(ref), foreach=False, fused=fused, **hp)
    oopt = mi_adamw.FusedAdamW(groups(ours), **hp, max_grad_norm=1.0 if clip else None,
                               flat_buffer=layout == "flat", fused=fused)
    side = torch.cuda.Stream()
    spacer = []
    log = []
    added = 0
    for k in range(40):
        # step 1 is one the native path takes: moved gradients in tables, gradients
        # refilled in place in the flat layout (whose moved gradients are copied into
        # its buffer by the general path).  A gradient set to None leaves that step count
        # behind its group's for good, which ends native steps (one hyperparameter set per
        # group is what the native path repeats), so it is drawn in the last 12 steps only.
        if k > 1:
            action = rng.choice(ACTIONS)
            if action == "none_grad" and k < 28:
                action = "move"
        else:
            action = "refill" if k == 1 and layout == "flat" else "move"
        if action == "add_group" and (layout == "flat" or added == 2):
            action = "move"
        stream = torch.cuda.current_stream()
        if action == "add_group":
            # new parameters in a group of their own; their state is made at their first
            # step, and every step from here on includes them
            added += 1
            shapes = [rng.choice(SHAPES) for _ in range(rng.randint(1, 3))]
            new_ref = make_params(shapes, dev, seed=50_000 + 100 * seed + 10 * added)
            new_ours = clone_params(new_ref)
            ghp = dict(lr=rng.choice([2e-4, 1e-3]), betas=(0.8, 0.99),
                       weight_decay=rng.choice([0.0, 0.05]), amsgrad=rng.random() < 0.5)
            topt.add_param_group({"params": new_ref, **ghp})
            oopt.add_param_group({"params": new_ours, **ghp})
            ref.extend(new_ref)
            ours.extend(new_ours)
        if (action in ("move", "none_grad", "add_group")
                or not all(q.grad is not None for q in ours)):
            for i, (p, q) in enumerate(zip(ref, ours)):
                g = torch.randn(p.shape, device=dev, generator=gen(dev, 7000 + 1000 * k + i))
                g.mul_(1e-2 * 0.8 ** (k % 7))
                p.grad = g.clone()
                spacer.append(torch.empty(4096 + rng.randrange(4096), device=dev))
                q.grad = g.clone()
            if action == "none_grad":
                j = rng.randrange(len(ref))
                ref[j].grad = None
                ours[j].grad = None
        elif action == "refill":
            for i, (p, q) in enumerate(zip(ref, ours)):
                g = torch.randn(p.shape, device=dev, generator=gen(dev, 9000 + 1000 * k + i))
                g.mul_(1e-2)
                p.grad.copy_(g)
                q.grad.copy_(g)
        elif action == "state_replace":
            j = rng.randrange(len(ref))
            if "exp_avg" in topt.state.get(ref[j], {}):
                key = rng.choice(["exp_avg", "exp_avg_sq"])
                topt.state[ref[j]][key] = topt.state[ref[j]][key].clone() * 0.5
                oopt.state[ours[j]][key] = oopt.state[ours[j]][key].clone() * 0.5
        elif action == "data_replace":
            j = rng.randrange(len(ref))
            with torch.no_grad():
                ref[j].data = ref[j].data.clone()
                ours[j].data = ours[j].data.clone()
        elif action == "lr":
            gi = rng.randrange(2)
            lr = rng.choice([1e-4, 3e-4, 6e-4, 0.0])
            topt.param_groups[gi]["lr"] = lr
            oopt.param_groups[gi]["lr"] = lr
        elif action == "hyper":
            gi = rng.randrange(len(topt.param_groups))
            change = dict(betas=rng.choice([(0.9, 0.95), (0.8, 0.99), (0.5, 0.999)]),
                          eps=rng.choice([1e-8, 1e-6]), weight_decay=rng.choice([0.0, 0.01, 0.1]),
                          maximize=rng.random() < 0.3)
            topt.param_groups[gi].update(change)
            oopt.param_groups[gi].update(change)
        elif action == "amsgrad":
            flag = rng.random() < 0.5
            topt.param_groups[1]["amsgrad"] = flag
            oopt.param_groups[1]["amsgrad"] = flag
        elif action == "stream":
            side.wait_stream(torch.cuda.current_stream())
            stream = side
        elif action == "checkpoint":
            oopt.load_state_dict(copy.deepcopy(topt.state_dict()))
        # torch's clip_grads_with_norm_ scaled ref's gradients in place at the last step;
        # ours keep theirs, so ref's values are refreshed from ours (ours keep their tensors)
        for p, q in zip(ref, ours):
            if q.grad is None:
                p.grad = None
            elif p.grad is None:
                p.grad = q.grad.clone()
            else:
                p.grad.copy_(q.grad)
        before = oopt.native_steps
        with torch.cuda.stream(stream):
            oopt.step()
            if clip:
                torch.nn.utils.clip_grads_with_norm_(
                    [p for p in ref if p.grad is not None], 1.0, oopt.last_grad_norm.clone())
            topt.step()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        d = _state_diff(ref, ours, topt, oopt)
        log.append((k, action, oopt.native_steps - before, d))
        assert d == 0, log[-5:]
    native = sum(n for _, _, n, _ in log)
    assert log[1][2] == 1, log[:2]
    if layout == "flat":
        # every parameter, gradient and moment is a view of the buffers again
        fl = oopt._flat
        for q in ours:
            assert fl.is_param_view(q) and (q.grad is None or fl.is_grad_view(q, q.grad))
            st = oopt.state.get(q, {})
            if "exp_avg" in st:
                assert st["exp_avg"].data_ptr() == (fl.exp_avg.data_ptr()
                                                    + 4 * fl.offsets[id(q)])
    print(f"seed {seed} {layout} {chain} clip {clip}: {native} of 40 steps on the native path; actions "
          f"{sorted(set(a for _, a, _, _ in log))}", flush=True)
    assert native >= 1
