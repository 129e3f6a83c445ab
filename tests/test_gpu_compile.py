"""The reference's --compile call site with FusedAdamW (main.py:81,174-180,202-210).

main.py wraps the model in torch.compile, then builds the optimizer on the compiled
model's parameters, and runs zero_grad, the forward (under bf16 autocast with --amp),
backward, optimizer.step() and the LambdaLR step (warm-up + cosine, main.py:36-43) every
iteration.  Here the tiny GPT is compiled with inductor and trained that way for 10
iterations with FusedAdamW (lr 6e-4, weight decay 0.1, config.py:11,13), with and without
bf16 autocast, in both layouts, and with --amp --fused (main.py:80: fused=True).  The
gradients inductor's backward hands to step() are also given, cloned, to
torch.optim.AdamW (foreach=False, or fused=True) over a shadow copy of the parameters with
its own LambdaLR: after every iteration the compiled model's parameters and FusedAdamW's
moments must equal torch's bit for bit.  (Two compiled models stepped
by the two optimizers would compare their backward passes too, and the embedding
gradient accumulates with atomics, which is not bit-reproducible from run to run.)
"""
from __future__ import annotations

import contextlib
import gc
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lr_at(warmup: int, total: int):
    # main.py:36-43, restated
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
    import torch._inductor.config as inductor_config
    threads = inductor_config.compile_threads
    inductor_config.compile_threads = 1        # compile in this process, no worker pool
    yield torch.device("cuda", 0)
    inductor_config.compile_threads = threads
    torch._dynamo.reset()
    gc.collect()
    torch.cuda.empty_cache()


def _bits(t):
    return t.detach().view(torch.int32)


@pytest.mark.parametrize("amp,flat,fused", [(False, False, False), (False, True, False),
                                            (True, False, False), (True, True, False),
                                            (True, False, True)])
def test_compiled_model_steps_as_torch_adamw(dev, amp, flat, fused):
    import mi_adamw
    import refgpt
    torch._dynamo.reset()
    model = refgpt.tiny(dev, seed=3)
    shadow = [torch.nn.Parameter(p.detach().clone()) for p in model.parameters()]
    cmodel = torch.compile(model)
    hp = dict(lr=6e-4, weight_decay=0.1)
    oopt = mi_adamw.FusedAdamW(cmodel.parameters(), **hp, fused=fused, flat_buffer=flat)
    topt = (torch.optim.AdamW(shadow, **hp, fused=True) if fused
            else torch.optim.AdamW(shadow, **hp, foreach=False))
    total = 10
    osch = torch.optim.lr_scheduler.LambdaLR(oopt, _lr_at(3, total))
    tsch = torch.optim.lr_scheduler.LambdaLR(topt, _lr_at(3, total))
    params = list(cmodel.parameters())
    ctx = torch.autocast("cuda", dtype=torch.bfloat16) if amp else contextlib.nullcontext()
    print(f"amp {amp} flat {flat} fused {fused}: compiling the tiny GPT (inductor)", flush=True)
    losses = []
    for it in range(total):
        ids, labels, mask = refgpt.batch(dev, seed=100 + it)
        oopt.zero_grad()
        topt.zero_grad()
        with ctx:
            _, loss = cmodel(ids, labels, mask)
        loss.backward()
        for p, q in zip(params, shadow):
            assert p.grad is not None and p.grad.dtype == torch.float32
            q.grad = p.grad.detach().clone()
        oopt.step()
        topt.step()
        osch.step()
        tsch.step()
        losses.append(loss.item())
        for p, q in zip(params, shadow):
            assert torch.equal(_bits(p), _bits(q)), it
            for key in ("exp_avg", "exp_avg_sq"):
                assert torch.equal(_bits(oopt.state[p][key]), _bits(topt.state[q][key])), (it, key)
        if it == 0:
            print(f"amp {amp} flat {flat} fused {fused}: first iteration done, "
                  f"loss {losses[0]:.4f}", flush=True)
    assert all(float(oopt.state[p]["step"]) == float(total) for p in params)
    assert oopt.param_groups[0]["lr"] == topt.param_groups[0]["lr"]
    print(f"amp {amp} flat {flat} fused {fused}: {total} compiled iterations bit-identical "
          f"to torch's AdamW, "
          f"loss {losses[0]:.4f} -> {losses[-1]:.4f}, {oopt.native_steps} native steps",
          flush=True)
    assert oopt.native_steps >= total - 2
