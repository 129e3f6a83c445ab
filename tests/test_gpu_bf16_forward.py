"""GPU: training with the step's bf16 copies as the forward's GEMM weights.

Reference loop: zero_grad, forward under bf16 autocast, backward, step
(main.py:202-209 with --amp).  Two identical models train side by side, one
with plain autocast (every F.linear casts its fp32 weight), one inside
mi_adamw.bf16_weights (the step's bf16 copies, no casts).  Loss, master
gradients, parameters and copies must agree bit for bit at every iteration:
the copy is round-to-nearest-even of the updated master, which is the value
autocast's cast produces, and the copy's backward widens the gradient exactly
as the cast's does.
"""
from __future__ import annotations

import pytest
import torch

import mi_adamw
import refgpt
from test_bf16_forward import _bits_equal, weight_casts

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    print("mi_adamw", mi_adamw.version(), flush=True)
    return torch.device("cuda", 0)


@pytest.mark.parametrize("placed", [False, True])
@pytest.mark.parametrize("flat", [False, True])
def test_training_on_bf16_copies_is_bit_identical(dev, flat, placed):
    """With `placed`, the bf16-weights model's optimizer places its streams after its first
    step (place_trials), again before its third (min_gain 0, so it moves whenever a
    candidate is any faster), and moves them before its fourth: the forward must read the
    copies where they are now."""
    a = refgpt.tiny(dev, seed=11)
    b = refgpt.tiny(dev, seed=11)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1, bf16_copy=True, max_grad_norm=1.0,
              flat_buffer=flat)
    oa = mi_adamw.FusedAdamW(a.parameters(), **hp)
    ob = mi_adamw.FusedAdamW(b.parameters(), **hp, place_trials=2 if placed else 0)
    for it in range(5):
        ids, labels, mask = refgpt.batch(dev, seed=100 + it)
        oa.zero_grad()
        ob.zero_grad()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, la = a(ids, labels, mask)
        la.backward()
        with torch.autocast("cuda", dtype=torch.bfloat16), mi_adamw.bf16_weights(ob, b):
            _, lb = b(ids, labels, mask)
        lb.backward()
        assert _bits_equal(la.detach(), lb.detach()), it
        for p, q in zip(a.parameters(), b.parameters()):
            assert _bits_equal(p.grad, q.grad), it
        if placed and it == 2:
            ob.place_buffers(trials=2, launches=1, rounds=1, min_gain=0.0)
        if placed and it == 3:
            # and a move forced through the layout's streams, whatever the timing says
            from mi_adamw import placement
            cls = placement._FlatStreams if flat else placement._TableStreams
            streams = cls(ob, dev)
            new = streams.allocate()
            streams.adopt(new)
            ob._launch_cache = None
            ob._fast = None
            assert ob.bf16_param(next(b.parameters())).data_ptr() == (
                new["copy"].data_ptr() if flat else new["copy"][0].data_ptr())
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for p, q in zip(a.parameters(), b.parameters()):
            assert _bits_equal(p.detach(), q.detach()), it
            assert _bits_equal(ob.bf16_param(q), q.detach().bfloat16()), it
        print(f"iteration {it}: loss {la.item():.6f} identical", flush=True)
    assert (ob.placement is not None) == placed


@pytest.mark.parametrize("flat", [False, True])
def test_gradient_accumulation_over_micro_batches_is_bit_identical(dev, flat):
    """Several forward/backward passes per step, as a pipeline schedule's micro-batches
    run them (parallel/pipeline_parallel.py): each backward's widened gradients add
    into the masters' .grad exactly as the cast's do under plain autocast."""
    a = refgpt.tiny(dev, seed=12)
    b = refgpt.tiny(dev, seed=12)
    hp = dict(lr=1e-3, weight_decay=0.1, bf16_copy=True, flat_buffer=flat)
    oa = mi_adamw.FusedAdamW(a.parameters(), **hp)
    ob = mi_adamw.FusedAdamW(b.parameters(), **hp)
    for it in range(3):
        oa.zero_grad()
        ob.zero_grad()
        for mb in range(3):
            ids, labels, mask = refgpt.batch(dev, seed=200 + 10 * it + mb)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                _, la = a(ids, labels, mask)
            (la / 3).backward()
            with torch.autocast("cuda", dtype=torch.bfloat16), mi_adamw.bf16_weights(ob, b):
                _, lb = b(ids, labels, mask)
            (lb / 3).backward()
            assert _bits_equal(la.detach(), lb.detach()), (it, mb)
        for p, q in zip(a.parameters(), b.parameters()):
            assert _bits_equal(p.grad, q.grad), it
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for p, q in zip(a.parameters(), b.parameters()):
            assert _bits_equal(p.detach(), q.detach()), it


def test_weight_casts_disappear_on_the_gpu(dev):
    model = refgpt.tiny(dev)
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    plain, swapped = weight_casts(model, opt, *refgpt.batch(dev), device_type="cuda")
    n_linear = sum(1 for m in model.modules() if isinstance(m, refgpt.ColumnLinear))
    print("aten::_to_copy per forward", plain, swapped, flush=True)
    assert plain - swapped == n_linear


def test_widen_every_bf16_pattern_like_torch(dev):
    """The one-launch widening of the weight gradients: all 2^16 bf16 bit patterns (NaN
    payloads, infinities, denormals, signed zeros) give torch's Tensor.to(float32) bits,
    through the vector path, a ragged tail and a 2-byte-misaligned view (scalar path)."""
    from mi_adamw.bf16_forward import _widen
    every = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    every = every.to(dev)
    srcs = [every, every[:4099], every[1:4098], every[5:8], every[:0],
            every.view(256, 256).t().contiguous()]
    outs = _widen(srcs)
    for s_, o in zip(srcs, outs):
        assert o.dtype == torch.float32 and o.shape == s_.shape
        assert torch.equal(o.view(torch.int32), s_.to(torch.float32).view(torch.int32))
    # a None gradient stays None, and a CPU tensor takes torch's cast
    cpu = every[:10].cpu()
    none, host = _widen([None, cpu])
    assert none is None and torch.equal(host.view(torch.int32), cpu.float().view(torch.int32))
