"""bf16_weights on the CPU: the optimizer's bf16 copies in place of autocast's weight casts.

CPU autocast casts F.linear's operands to bf16 as the GPU's does, so the
mechanism is checked here without a GPU: loss, logits and every master
gradient bit-identical to plain autocast; the copies are refreshed when a
master changes outside the optimizer; misuse raises.  (The copies are the ones
FusedAdamW writes at construction: RNE of the fp32 masters.)
"""
from __future__ import annotations

import pytest
import torch

import mi_adamw
import refgpt


def _autocast():
    return torch.autocast("cpu", dtype=torch.bfloat16)


def _run(model, ids, labels, mask, opt=None):
    model.zero_grad(set_to_none=True)
    if opt is None:
        with _autocast():
            logits, loss = model(ids, labels, mask)
    else:
        with _autocast(), mi_adamw.bf16_weights(opt, model):
            logits, loss = model(ids, labels, mask)
    loss.backward()
    return logits.detach(), loss.detach(), [p.grad.clone() for p in model.parameters()]


def _bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.dtype == torch.bfloat16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_forward_and_grads_bit_identical_to_autocast():
    dev = torch.device("cpu")
    a = refgpt.tiny(dev, seed=3)
    b = refgpt.tiny(dev, seed=3)
    opt = mi_adamw.FusedAdamW(b.parameters(), lr=1e-3, bf16_copy=True)
    ids, labels, mask = refgpt.batch(dev)
    la, fa, ga = _run(a, ids, labels, mask)
    lb, fb, gb = _run(b, ids, labels, mask, opt)
    assert la.dtype == torch.bfloat16          # autocast ran the lm_head GEMM in bf16
    assert _bits_equal(la, lb) and _bits_equal(fa, fb)
    assert all(_bits_equal(x, y) for x, y in zip(ga, gb))
    # the parameters are back in place and nothing else holds a swap
    for mod in b.modules():
        for p in mod._parameters.values():
            assert p is None or isinstance(p, torch.nn.Parameter)


def test_only_linear_layers_are_swapped():
    model = refgpt.tiny(torch.device("cpu"))
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    ctx = mi_adamw.bf16_weights(opt, model)
    swapped = {id(p) for _, _, p in ctx.swaps}
    linear = {id(m.weight) for m in model.modules() if isinstance(m, refgpt.ColumnLinear)}
    assert swapped == linear
    assert id(model.wte) not in swapped and id(model.wpe.weight) not in swapped
    assert all(id(p) not in swapped for m in model.modules() if isinstance(m, torch.nn.LayerNorm)
               for p in m.parameters())


def test_copy_refreshed_after_master_changes_in_place():
    dev = torch.device("cpu")
    a = refgpt.tiny(dev, seed=5)
    b = refgpt.tiny(dev, seed=5)
    opt = mi_adamw.FusedAdamW(b.parameters(), bf16_copy=True)
    ids, labels, mask = refgpt.batch(dev)
    _run(b, ids, labels, mask, opt)           # copies now tracked
    with torch.no_grad():                     # a change the optimizer did not make
        for m in (a, b):
            m.layers[0].fc1.weight.mul_(1.5)
            m.lm_head.weight.add_(0.01)
    la, fa, ga = _run(a, ids, labels, mask)
    lb, fb, gb = _run(b, ids, labels, mask, opt)
    assert _bits_equal(la, lb) and _bits_equal(fa, fb)
    assert all(_bits_equal(x, y) for x, y in zip(ga, gb))
    assert torch.equal(opt.bf16_param(b.lm_head.weight), b.lm_head.weight.detach().bfloat16())


def test_refresh_after_data_assignment():
    model = refgpt.tiny(torch.device("cpu"))
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    w = model.layers[1].o.weight
    w.data = torch.full_like(w, 0.25)
    opt.refresh_bf16_copies()
    assert torch.equal(opt.bf16_param(w), torch.full_like(w, 0.25, dtype=torch.bfloat16))


def test_misuse_raises():
    model = refgpt.tiny(torch.device("cpu"))
    ids, labels, mask = refgpt.batch(torch.device("cpu"))
    with pytest.raises(RuntimeError, match="bf16_copy"):
        mi_adamw.bf16_weights(mi_adamw.FusedAdamW(model.parameters()), model)
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    with pytest.raises(RuntimeError, match="autocast"):
        with mi_adamw.bf16_weights(opt, model):
            model(ids, labels, mask)
    # an exception inside the context restores the parameters too
    with pytest.raises(ValueError):
        with _autocast(), mi_adamw.bf16_weights(opt, model):
            assert model.lm_head.weight.dtype == torch.bfloat16
            raise ValueError("boom")
    # the failed forward left every parameter in place
    for mod in model.modules():
        for p in mod._parameters.values():
            assert p is None or isinstance(p, torch.nn.Parameter)


def test_complex_params_refuse_a_bf16_copy():
    p = torch.nn.Parameter(torch.zeros(8, dtype=torch.complex64))
    with pytest.raises(NotImplementedError, match="complex"):
        mi_adamw.FusedAdamW([p], bf16_copy=True)
    opt = mi_adamw.FusedAdamW([torch.nn.Parameter(torch.zeros(4))], bf16_copy=True)
    with pytest.raises(NotImplementedError, match="complex"):
        opt.add_param_group({"params": [p]})
    assert len(opt.param_groups) == 1


def test_the_gemm_reads_the_copy():
    """A copy altered behind the optimizer's back changes the output: the swap is real."""
    dev = torch.device("cpu")
    model = refgpt.tiny(dev, seed=7)
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    ids, labels, mask = refgpt.batch(dev)
    w = model.lm_head.weight                  # inside the context this name is the copy
    with _autocast(), mi_adamw.bf16_weights(opt, model):
        assert model.lm_head.weight.dtype == torch.bfloat16
        ref = model(ids, labels, mask)[0].detach()
    assert model.lm_head.weight is w
    opt.bf16_param(w).zero_()                    # the copy only; the master is untouched
    with _autocast(), mi_adamw.bf16_weights(opt, model):
        out = model(ids, labels, mask)[0].detach()
    assert not torch.equal(ref, out)
    assert torch.count_nonzero(out) == 0                 # lm_head GEMM ran on the zeroed copy


def weight_casts(model, opt, ids, labels, mask, device_type="cpu"):
    """aten::_to_copy calls in one bf16-autocast forward, plain and with bf16_weights."""
    out = []
    for use in (False, True):
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU],
                                    acc_events=True) as prof:
            with torch.autocast(device_type, dtype=torch.bfloat16):
                if use:
                    with mi_adamw.bf16_weights(opt, model):
                        model(ids, labels, mask)
                else:
                    model(ids, labels, mask)
        out.append(sum(1 for e in prof.events() if e.name == "aten::_to_copy"))
    return out


def test_weight_casts_disappear_from_the_forward():
    dev = torch.device("cpu")
    model = refgpt.tiny(dev)
    opt = mi_adamw.FusedAdamW(model.parameters(), bf16_copy=True)
    plain, swapped = weight_casts(model, opt, *refgpt.batch(dev))
    n_linear = sum(1 for m in model.modules() if isinstance(m, refgpt.ColumnLinear))
    assert plain - swapped == n_linear
