"""Seeded random step sequences through the native and general step paths, against torch.

Each step draws a change from what mini-megatron's loop and its users do between steps:
new gradient tensors (zero_grad + backward), the same gradient tensors refilled, a
gradient set to None, a state tensor replaced, ``p.data`` replaced, the learning rate
changed, amsgrad switched for a group, the step on another stream, a checkpoint round
trip.  After every step parameters and moments must equal torch.optim.AdamW
(foreach=False) bit for bit; the test also counts how many steps each path took.
"""
from __future__ import annotations

import copy
import gc
import random

import pytest
import torch

from _helpers import clone_params, gen, make_params, max_ulp_all

pytestmark = pytest.mark.gpu

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (1024,), (33,)]
ACTIONS = ["move", "move", "move", "refill", "none_grad", "state_replace", "data_replace",
           "lr", "amsgrad", "stream", "checkpoint"]


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


@pytest.mark.parametrize("layout", ["tables", "flat"])
@pytest.mark.parametrize("seed", range(6))
def test_random_step_sequences(dev, seed, layout):
    """In the flat layout the parameters, gradients and moments are views of its buffers:
    a replaced p.data, gradient or state tensor is copied into its slice at the next step,
    and the results must still equal torch's."""
    import mi_adamw
    rng = random.Random(seed)
    clip = seed % 2 == 0
    ref = make_params(SHAPES, dev, seed=1000 + 100 * seed)
    ours = clone_params(ref)
    groups = lambda ps: [{"params": ps[:4], "amsgrad": True},      # noqa: E731
                         {"params": ps[4:], "lr": 1e-3, "weight_decay": 0.0, "amsgrad": True}]
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    topt = torch.optim.AdamW(groups(ref), foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(groups(ours), **hp, max_grad_norm=1.0 if clip else None,
                               flat_buffer=layout == "flat")
    side = torch.cuda.Stream()
    spacer = []
    log = []
    for k in range(40):
        action = rng.choice(ACTIONS) if k > 1 else "move"
        stream = torch.cuda.current_stream()
        if action == "move" or action == "none_grad" or not all(q.grad is not None for q in ours):
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
    if layout == "flat":
        # every parameter, gradient and moment is a view of the buffers again
        fl = oopt._flat
        for q in ours:
            assert fl.is_param_view(q) and (q.grad is None or fl.is_grad_view(q, q.grad))
            st = oopt.state.get(q, {})
            if "exp_avg" in st:
                assert st["exp_avg"].data_ptr() == (fl.exp_avg.data_ptr()
                                                    + 4 * fl.offsets[id(q)])
    print(f"seed {seed} {layout} clip {clip}: {native} of 40 steps on the native path; actions "
          f"{sorted(set(a for _, a, _, _ in log))}", flush=True)
    assert native >= 1
