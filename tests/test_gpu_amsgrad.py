"""GPU parity of amsgrad: FusedAdamW(amsgrad=True) against torch.optim.AdamW(amsgrad=True,
foreach=False) and the oracle.

amsgrad keeps max_exp_avg_sq = maximum(max_exp_avg_sq, exp_avg_sq) and takes
the denominator from it (torch/optim/adam.py:538-543).  The gradients below
shrink from step to step, so exp_avg_sq decays under its running maximum and
the maximum, not v, drives most updates; each test checks that it did.
Tolerance: 0 ulp (the kernel follows torch-ROCm's op chain), as in the other
parity tests.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import (clone_params, load_states, make_params, max_ulp_all, midtrain_state,
                      set_grads, to_np)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (1,), (7, 5), (70001,), (65536 + 12,)]
HP = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    import mi_adamw
    print("mi_adamw", mi_adamw.version(), flush=True)
    return torch.device("cuda", 0)


def _shrinking_grads(params, step):
    # std 1e-2 * 0.5**step: v falls below its running maximum after the first steps
    set_grads(params, step, 1e-2 * 0.5 ** step, base=7000)


def _same(ref, ours, topt, oopt, keys=("exp_avg", "exp_avg_sq", "max_exp_avg_sq")):
    d = {"p": max_ulp_all(ref, ours)}
    for k in keys:
        d[k] = max_ulp_all([topt.state[p][k] for p in ref], [oopt.state[q][k] for q in ours])
    print("ulp", d, flush=True)
    assert all(v == 0 for v in d.values()), d


def _frac_max_above_v(opt, params):
    above = sum(int((opt.state[p]["max_exp_avg_sq"] > opt.state[p]["exp_avg_sq"]).sum())
                for p in params)
    return above / sum(p.numel() for p in params)


@pytest.mark.parametrize("clip", [None, 1.0])
def test_amsgrad_chained_matches_torch_bitwise(dev, clip):
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, amsgrad=True, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, amsgrad=True, max_grad_norm=clip, **HP)
    for step in range(1, 9):
        _shrinking_grads(ref, step)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        oopt.step()
        if clip is not None:
            # torch's clip, driven by our norm (the norms agree to 1e-6; the
            # coefficient is then the same fp32 value on both sides)
            torch.nn.utils.clip_grads_with_norm_(ref, clip, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        print(f"step {step}", flush=True)
        _same(ref, ours, topt, oopt)
    assert _frac_max_above_v(oopt, ours) > 0.5


def test_amsgrad_midtrain_and_checkpoint_interchange(dev):
    """A stored max_exp_avg_sq above v on part of the elements, loaded through
    load_state_dict; then the checkpoint goes back into torch and steps on."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    states = midtrain_state(ref, 1000.0)
    for i, (p, st) in enumerate(zip(ref, states)):
        other = (torch.randn(p.shape, device=dev, generator=torch.Generator(dev).manual_seed(900 + i))
                 * 1e-6).abs()
        st["max_exp_avg_sq"] = torch.maximum(st["exp_avg_sq"], other)
    hp = dict(HP, fused=False)
    topt = torch.optim.AdamW(ref, amsgrad=True, **hp)
    oopt = mi_adamw.FusedAdamW(ours, amsgrad=True, **hp)
    load_states(topt, ref, states)
    load_states(oopt, ours, states)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    _same(ref, ours, topt, oopt)
    frac = _frac_max_above_v(oopt, ours)
    print("fraction max > v", frac, flush=True)
    assert 0.05 < frac < 0.95
    sd = oopt.state_dict()
    assert set(sd["state"][0]) == set(topt.state_dict()["state"][0])
    t2 = torch.optim.AdamW(clone_params(ours), amsgrad=True, **hp)
    t2.load_state_dict(sd)
    o2 = mi_adamw.FusedAdamW(clone_params(ref), amsgrad=True, **hp)
    o2.load_state_dict(topt.state_dict())
    pt, po = t2.param_groups[0]["params"], o2.param_groups[0]["params"]
    for step in range(4, 6):
        set_grads(pt, step, 1e-3)
        for p, q in zip(pt, po):
            q.grad = p.grad.clone()
        t2.step()
        o2.step()
    torch.cuda.synchronize()
    _same(pt, po, t2, o2)


def test_amsgrad_mixed_groups(dev):
    """One amsgrad group, one plain group, and enough distinct step counts
    (more than 16 hyperparameter sets) to split each side over launches."""
    import mi_adamw
    shapes = [(37 + 5 * i,) for i in range(40)] + [(4096 * 3 + 1,)]
    ref = make_params(shapes, dev)
    ours = clone_params(ref)

    def groups(ps):
        return [dict(params=ps[0::2], amsgrad=True), dict(params=ps[1::2], amsgrad=False)]

    topt = torch.optim.AdamW(groups(ref), foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(groups(ours), **HP)
    states = midtrain_state(ref, 0.0)
    for i, st in enumerate(states):
        st["step"] = torch.tensor(float(10 + i))
    order_ref = topt.param_groups[0]["params"] + topt.param_groups[1]["params"]
    order_ours = oopt.param_groups[0]["params"] + oopt.param_groups[1]["params"]
    st_by_param = {id(p): st for p, st in zip(ref, states)}
    st_ordered = [st_by_param[id(p)] for p in order_ref]
    for st, p in zip(st_ordered, order_ref):
        if any(p is q for q in topt.param_groups[0]["params"]):
            st["max_exp_avg_sq"] = st["exp_avg_sq"] * 2
    load_states(topt, order_ref, st_ordered)
    load_states(oopt, order_ours, st_ordered)
    for step in range(1, 4):
        _shrinking_grads(ref, step)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    g0r, g0o = topt.param_groups[0]["params"], oopt.param_groups[0]["params"]
    g1r, g1o = topt.param_groups[1]["params"], oopt.param_groups[1]["params"]
    _same(g0r, g0o, topt, oopt)
    _same(g1r, g1o, topt, oopt, keys=("exp_avg", "exp_avg_sq"))
    assert all("max_exp_avg_sq" not in oopt.state[q] for q in g1o)


def test_amsgrad_bf16_state_matches_oracle(dev):
    """bf16 moments and bf16 running maximum against the oracle, bit for bit."""
    import mi_adamw
    params = make_params(SHAPES, dev)
    init = [to_np(p).copy() for p in params]
    opt = mi_adamw.FusedAdamW(params, amsgrad=True, state_dtype=torch.bfloat16, **HP)
    states = midtrain_state(params, 50.0)
    for i, (p, st) in enumerate(zip(params, states)):
        st["max_exp_avg_sq"] = st["exp_avg_sq"] * (1.0 + (i % 3))
    load_states(opt, params, states)
    for p in params:
        assert opt.state[p]["max_exp_avg_sq"].dtype == torch.bfloat16
    bits = [{k: O.to_bf16_bits(to_np(states[i][k])).reshape(-1)
             for k in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq")} for i in range(len(params))]
    pn = [x.reshape(-1).copy() for x in init]
    for step in (1, 2):
        _shrinking_grads(params, step)
        grads = [to_np(p.grad).reshape(-1).copy() for p in params]
        opt.step()
        for i in range(len(params)):
            O.adamw_step_bf16state(pn[i], grads[i], bits[i]["exp_avg"], bits[i]["exp_avg_sq"],
                                   step=50.0 + step, vmax_bits=bits[i]["max_exp_avg_sq"], **HP)
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        assert O.max_ulp(pn[i], to_np(p).reshape(-1))[0] == 0
        for k in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
            got = to_np(opt.state[p][k].view(torch.int16)).view(np.uint16).reshape(-1)
            assert np.array_equal(got, bits[i][k]), (i, k)


def test_amsgrad_flat_buffer_matches_torch(dev):
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, amsgrad=True, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, amsgrad=True, flat_buffer=True, max_grad_norm=1.0, **HP)
    for step in range(1, 6):
        oopt.zero_grad()
        _shrinking_grads(ref, step)
        for p, q in zip(ref, ours):
            q.grad.copy_(p.grad)
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        _same(ref, ours, topt, oopt)
    # every max_exp_avg_sq is a view of the one flat buffer
    buf = oopt._flat.max_exp_avg_sq
    for q in ours:
        x = oopt.state[q]["max_exp_avg_sq"]
        assert buf.data_ptr() <= x.data_ptr() < buf.data_ptr() + 4 * buf.numel()
    assert _frac_max_above_v(oopt, ours) > 0.5


def test_amsgrad_nonfinite_propagates_like_torch(dev):
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, amsgrad=True, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, amsgrad=True, **HP)
    set_grads(ref, 1, 1e-3)
    ref[0].grad[0, 0] = float("nan")
    ref[3].grad[5] = float("inf")
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()
    topt.step()
    oopt.step()
    torch.cuda.synchronize()
    for p, q in zip(ref, ours):
        for k in ("exp_avg_sq", "max_exp_avg_sq"):
            a, b = topt.state[p][k], oopt.state[q][k]
            assert torch.equal(torch.isnan(a), torch.isnan(b)), k
            assert torch.equal(torch.isinf(a), torch.isinf(b)), k
        assert torch.equal(torch.isnan(p), torch.isnan(q))
    _same(ref, ours, topt, oopt)
