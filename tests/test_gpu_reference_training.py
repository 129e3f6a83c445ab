"""GPU: the reference's own training tests (tests/test_training.py:45-104), with FusedAdamW
in place of torch.optim.AdamW.

* A tiny GPT (vocab 64, 8 positions) trains 200 steps on a repeating token pattern at
  lr 1e-3; the loss on a held-out batch must drop by more than 1.0 and end below 3.5
  (the random-init loss is about ln 64 = 4.16).  Run with the default fp32 step, and with
  the fused clip, bf16 moments, the bf16 copy and the forward on the copies under bf16
  autocast.
* One step at lr 1e-2 changes every parameter that has a gradient.
"""
from __future__ import annotations

import pytest
import torch

import refgpt

pytestmark = pytest.mark.gpu

VOCAB, S, B = 64, 8, 4


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    return torch.device("cuda", 0)


def _model(dev, seed):
    torch.manual_seed(seed)
    return refgpt.GPT(vocab=VOCAB, h=64, heads=4, ffn=256, layers=2, seq=S).to(dev)


def _batch(dev):
    x = torch.tensor([[(i + 1) % VOCAB for i in range(S)]] * B, device=dev)
    y = torch.tensor([[(i + 2) % VOCAB for i in range(S)]] * B, device=dev)
    return x, y, torch.ones(B, S, device=dev)


@pytest.mark.parametrize("variant", ["fp32", "fp32-fused-true",
                                     "clip-bf16-state-copy-bf16-weights"])
def test_loss_decreases_with_the_fused_step(dev, variant):
    import mi_adamw
    model = _model(dev, 42)
    x, y, mask = _batch(dev)
    if variant.startswith("fp32"):
        # fp32-fused-true: the reference's --fused (main.py:80,177), torch's fused chain
        opt = mi_adamw.FusedAdamW(model.parameters(), lr=1e-3, fused=variant.endswith("true"))
    else:
        opt = mi_adamw.FusedAdamW(model.parameters(), lr=1e-3, max_grad_norm=1.0,
                                  state_dtype=torch.bfloat16, bf16_copy=True)
    with torch.no_grad():
        initial = model(x, y, mask)[1].item()
    for _ in range(200):
        opt.zero_grad()
        if variant.startswith("fp32"):
            loss = model(x, y, mask)[1]
        else:
            with torch.autocast("cuda", dtype=torch.bfloat16), mi_adamw.bf16_weights(opt, model):
                loss = model(x, y, mask)[1]
        loss.backward()
        opt.step()
    with torch.no_grad():
        final = model(x, y, mask)[1].item()
    print(f"{variant}: loss {initial:.3f} -> {final:.3f}", flush=True)
    assert final < initial - 1.0, (initial, final)
    assert final < 3.5, final


def test_one_step_updates_every_parameter(dev):
    import mi_adamw
    model = _model(dev, 0)
    x, y, mask = _batch(dev)
    opt = mi_adamw.FusedAdamW(model.parameters(), lr=1e-2)
    before = [p.detach().clone() for p in model.parameters()]
    opt.zero_grad()
    model(x, y, mask)[1].backward()
    opt.step()
    torch.cuda.synchronize()
    with_grad = [(p, p0) for p, p0 in zip(model.parameters(), before) if p.grad is not None]
    assert with_grad
    for p, p0 in with_grad:
        assert not torch.equal(p.detach(), p0)
