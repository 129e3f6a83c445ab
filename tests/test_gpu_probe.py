"""GPU: the update's memory-only twin (mi_adamw_probe, mi_adamw.probe.time_probe).

It must move the step's bytes without changing any value: after probe launches on an
optimizer's tensors, parameters, gradients, moments, amsgrad's maximum and the bf16
copies are bit-identical to what the step left, in the per-tensor, bf16-state,
flat and capturable layouts, through the vector path and the scalar path (a
misaligned view).
"""
from __future__ import annotations

import warnings

import pytest
import torch

from _helpers import make_params, set_grads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    return torch.device("cuda", 0)


def _snapshot(opt, params):
    snap = []
    for p in params:
        st = opt.state[p]
        snap.append([p.detach().clone(), p.grad.clone()]
                    + [st[k].clone() for k in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq")
                       if k in st])
    copies = [c.clone() for c in opt.bf16_params()] if opt.bf16_copy else []
    return snap, copies


@pytest.mark.parametrize("kw", [
    dict(max_grad_norm=1.0),
    dict(state_dtype=torch.bfloat16, bf16_copy=True, amsgrad=True, max_grad_norm=0.5,
         clip_write_grads=True),
    dict(flat_buffer=True, bf16_copy=True, max_grad_norm=1.0),
    dict(capturable=True),
], ids=["fp32-clip", "bf16-state-copy-amsgrad-writegrad", "flat-copy-clip", "capturable"])
def test_probe_keeps_every_value(dev, kw):
    import mi_adamw
    from mi_adamw.probe import time_probe
    params = make_params([(4096,), (33, 17), (5,), (70000,)], dev)
    if not kw.get("flat_buffer"):
        # a view at a 1-element offset: not 16-byte aligned, the scalar path
        store = torch.zeros(9000, device=dev)
        view = store[1:8193]
        view.copy_(torch.randn(8192, device=dev) * 0.02)
        params.append(torch.nn.Parameter(view))
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
        opt = mi_adamw.FusedAdamW(params, lr=1e-3, weight_decay=0.1, **kw)
        for step in (1, 2):
            set_grads(params, step, 1e-2)
            opt.step()
    torch.cuda.synchronize()
    before, copies = _snapshot(opt, params)
    ms = time_probe(opt, launches=3)
    torch.cuda.synchronize()
    assert ms is not None and ms > 0
    after, copies_after = _snapshot(opt, params)
    for i, (xs, ys) in enumerate(zip(before, after)):
        assert len(xs) == len(ys)
        for j, (x, y) in enumerate(zip(xs, ys)):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), (i, j)
    for p, c, d in zip(params, copies, copies_after):
        assert torch.equal(c.view(torch.int16), d.view(torch.int16))
        assert torch.equal(d, p.detach().to(torch.bfloat16))
