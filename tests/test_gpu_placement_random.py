"""Seeded random step sequences with buffer placement interleaved, against torch.

Between steps the sequence draws what a training loop does (new gradient tensors, the
same ones refilled, a gradient set to None, a state tensor or ``p.data`` replaced, the
learning rate changed, the step on another stream, a checkpoint round trip) and, among
those, a placement: ``place_buffers`` with min_gain 0 (so it moves whenever a candidate
is any faster), or a forced move of the whole set or of a random subset of the streams
through the layout's stream classes.  A placement lands between a replacement and the
step that takes it in, on state that a checkpoint load just replaced, after a step on a
side stream.  After every step parameters and moments must equal torch.optim.AdamW
(foreach=False) bit for bit and the bf16 copy must equal the bf16 of the parameter.
"""
from __future__ import annotations

import copy
import gc
import random

import pytest
import torch

from _helpers import clone_params, gen, make_params, max_ulp_all, same_bits, seeds

pytestmark = pytest.mark.gpu

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (1024,), (33,)]
ACTIONS = ["move", "move", "refill", "none_grad", "state_replace", "data_replace", "lr",
           "stream", "checkpoint", "place", "place_forced", "place_forced"]
# a fixed start: the native path must take the steps after a placement (it repeats one
# hyperparameter set per group, which a gradient left out once, later, can rule out)
START = ["move", "move", "place", "refill", "refill"]


@pytest.fixture
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    yield torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()


def _diff(ref, ours, topt, oopt):
    d = max_ulp_all(list(ref), list(ours))
    for p, q in zip(ref, ours):
        st, so = topt.state.get(p, {}), oopt.state.get(q, {})
        for k in ("exp_avg", "exp_avg_sq"):
            if k in st:
                d = max(d, max_ulp_all([st[k]], [so[k]]))
        if "step" in st:
            assert float(st["step"]) == float(so["step"])
        if q in oopt.state:
            assert same_bits(oopt.bf16_param(q), q.detach().to(torch.bfloat16))
    return d


def _forced(oopt, dev, rng):
    """Move the whole set, or a random subset of its streams, into new allocations."""
    from mi_adamw import placement
    flat = oopt._flat is not None
    streams = placement._FlatStreams(oopt, dev) if flat else placement._TableStreams(oopt, dev)
    names = list(streams.names)
    if rng.random() < 0.5:
        names = rng.sample(names, rng.randrange(1, len(names) + 1))
    torch.cuda.synchronize()
    new = streams.allocate(names)
    streams.adopt(new if flat else {**streams.current(), **new})
    oopt._launch_cache = None
    oopt._fast = None
    return names


@pytest.mark.parametrize("layout", ["tables", "flat"])
@pytest.mark.parametrize("seed", seeds(4))
def test_random_sequences_with_placement(dev, seed, layout):
    import mi_adamw
    rng = random.Random(seed)
    clip = seed % 2 == 0
    ref = make_params(SHAPES, dev, seed=5000 + 100 * seed)
    ours = clone_params(ref)
    groups = lambda ps: [{"params": ps[:4]},                           # noqa: E731
                         {"params": ps[4:], "lr": 1e-3, "weight_decay": 0.0}]
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    topt = torch.optim.AdamW(groups(ref), foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(groups(ours), **hp, max_grad_norm=1.0 if clip else None,
                               bf16_copy=True, flat_buffer=layout == "flat",
                               place_trials=2 if seed == 3 else 0)
    side = torch.cuda.Stream()
    log = []
    placed = 0
    for k in range(30):
        action = START[k] if k < len(START) else rng.choice(ACTIONS)
        stream = torch.cuda.current_stream()
        what = action
        if action == "move" or action == "none_grad" or not all(q.grad is not None for q in ours):
            for i, (p, q) in enumerate(zip(ref, ours)):
                g = torch.randn(p.shape, device=dev, generator=gen(dev, 17000 + 1000 * k + i))
                g.mul_(1e-2 * 0.8 ** (k % 7))
                p.grad = g.clone()
                q.grad = g.clone()
            if action == "none_grad":
                j = rng.randrange(len(ref))
                ref[j].grad = None
                ours[j].grad = None
        elif action == "refill":
            for i, (p, q) in enumerate(zip(ref, ours)):
                g = torch.randn(p.shape, device=dev, generator=gen(dev, 19000 + 1000 * k + i))
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
        elif action == "stream":
            side.wait_stream(torch.cuda.current_stream())
            stream = side
        elif action == "checkpoint":
            oopt.load_state_dict(copy.deepcopy(topt.state_dict()))
        elif action == "place":
            rep = oopt.place_buffers(trials=2, launches=1, rounds=1, min_gain=0.0)
            what = f"place {rep['chosen']} {[s['chosen'] for s in rep['per_stream']]}"
            placed += 1
        elif action == "place_forced":
            what = f"forced {_forced(oopt, dev, rng)}"
            placed += 1
        # the placement changes no value: compare before the step as well
        if action.startswith("place"):
            torch.cuda.synchronize()
            assert _diff(ref, ours, topt, oopt) == 0, (k, what)
        # torch's clip_grads_with_norm_ scaled ref's gradients in place at the last step;
        # ours keep theirs, so ref's values are refreshed from ours
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
        d = _diff(ref, ours, topt, oopt)
        log.append((k, what, oopt.native_steps - before, d))
        assert d == 0, log[-5:]
        if k in (3, 4):
            assert log[-1][2] == 1, log                # the native path, after the placement
    if seed == 3:
        assert oopt.placement is not None          # place_trials placed after the first step
    native = sum(n for _, _, n, _ in log)
    if layout == "flat":
        fl = oopt._flat
        for q in ours:
            assert fl.is_param_view(q)
            st = oopt.state.get(q, {})
            if "exp_avg" in st:
                assert st["exp_avg"].data_ptr() == (fl.exp_avg.data_ptr()
                                                    + 4 * fl.offsets[id(q)])
    print(f"seed {seed} {layout} clip {clip}: {placed} placements, {native} of 30 steps "
          f"native; {[w for _, w, _, _ in log if w.startswith(('place', 'forced'))]}",
          flush=True)
    assert placed >= 1 and native >= 1
