"""2000 chained clipped steps under the reference's learning-rate schedule, against torch.

mini-megatron builds AdamW with lr 6e-4, weight decay 0.1 and the default betas and eps
(config.py:11,13; main.py:177), clips at 1.0 (config.py:16) and drives lr with LambdaLR
over a linear warm-up and a cosine decay (main.py:36-43,178-180; WARMUP_STEPS = 10,
config.py:14).  The per-step scalars (bias corrections 1 - beta**step in float64, the
scheduled lr, the step size) change every step, so a long chain pins them over the whole
range of step counts a run sees, including lr = 0 at the first step.  New gradient
tensors every step, as after zero_grad(); parameters and moments are compared with
torch.optim.AdamW(foreach=False) bit for bit every 100 steps.
"""
from __future__ import annotations

import gc
import math

import pytest
import torch

from _helpers import clone_params, gen, make_params, max_ulp_all

pytestmark = pytest.mark.gpu

SHAPES = [(96, 64), (64,), (64,), (192, 64), (4099,), (7, 5), (3,), (20001,)]


def _schedule(warmup: int, total: int):
    # the same function as main.py:36-43, restated
    def lr_at(step):
        if step < warmup:
            return step / max(warmup, 1)
        progress = (step - warmup) / max(total - warmup, 1)
        return 0.5 * (1.0 + math.cos(progress * math.pi))
    return lr_at


@pytest.fixture
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    yield torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("flat", [False, True])
def test_two_thousand_steps_of_the_reference_schedule(dev, flat):
    import mi_adamw
    total = 2000
    ref = make_params(SHAPES, dev, seed=77)
    ours = clone_params(ref)
    hp = dict(lr=6e-4, weight_decay=0.1)
    topt = torch.optim.AdamW(ref, foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(ours, **hp, max_grad_norm=1.0, flat_buffer=flat)
    tsch = torch.optim.lr_scheduler.LambdaLR(topt, _schedule(10, total))
    osch = torch.optim.lr_scheduler.LambdaLR(oopt, _schedule(10, total))
    for step in range(total):
        topt.zero_grad()
        oopt.zero_grad()
        scale = 3e-2 * (1.0 + 0.5 * math.sin(step / 37.0))
        for i, (p, q) in enumerate(zip(ref, ours)):
            g = torch.randn(p.shape, device=dev, generator=gen(dev, 5000 + 100 * step + i))
            g.mul_(scale)
            p.grad = g
            if flat:
                q.grad.copy_(g)          # the flat layout's gradients stay in its buffer
            else:
                q.grad = g.clone()
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
        tsch.step()
        osch.step()
        if step % 100 == 99 or step == total - 1:
            torch.cuda.synchronize()
            d = max(max_ulp_all(list(ref), list(ours)),
                    max_ulp_all([topt.state[p]["exp_avg"] for p in ref],
                                [oopt.state[q]["exp_avg"] for q in ours]),
                    max_ulp_all([topt.state[p]["exp_avg_sq"] for p in ref],
                                [oopt.state[q]["exp_avg_sq"] for q in ours]))
            assert d == 0, (step, d)
    assert topt.param_groups[0]["lr"] == oopt.param_groups[0]["lr"]
    assert all(float(oopt.state[q]["step"]) == float(total) for q in ours)
    print(f"flat {flat}: {total} steps bit-identical, {oopt.native_steps} on the native path",
          flush=True)
    assert oopt.native_steps >= total - 2
