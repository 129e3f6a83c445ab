"""GPU: FusedAdamW(fused=True) against torch.optim.AdamW(fused=True), bit for bit.

mini-megatron builds ``torch.optim.AdamW(..., fused=args.fused)`` (main.py:80,144,177);
with ``--fused`` torch runs ``_fused_adam`` (torch/optim/adam.py:803-895): the step
counts += 1 on the device, then ``torch._fused_adamw_``, whose per-element math is
``adam_math`` of ATen/native/hip/fused_adam_utils.cuh: float64 hyperparameters, m and v
formed in float64 and rounded once, per-step values formed from the step count in
float64 and handed over as fp32.  Its results differ from the ``foreach=False`` chain
(a quarter of the parameters by up to hundreds of ulp after one step), so
``fused=True`` selects the same chain here (mi_adamw_step*_fused_chain).

The oracle's restatement of that chain (``oracle.adamw_step_fused``) is pinned here
against torch's own kernel, and every FusedAdamW configuration is compared with torch
directly: p, exp_avg, exp_avg_sq (and max_exp_avg_sq) must be bit-identical.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from _helpers import (clone_params, gen, load_states, make_params, max_ulp, midtrain_state,
                      set_grads, to_np)

pytestmark = pytest.mark.gpu

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (65536 + 12,)]
HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


@pytest.fixture(scope="module")
def dev():
    import mi_adamw  # noqa: F401  (loads the library; raises without it)
    return torch.device("cuda", 0)


def _fused_torch(p, g, m, v, step, *, lr, betas, eps, weight_decay, maximize=False, vmax=None):
    st = torch.tensor(float(step), dtype=torch.float32, device=p.device)
    torch._fused_adamw_([p], [g], [m], [v], [vmax] if vmax is not None else [], [st], lr=lr,
                        beta1=betas[0], beta2=betas[1], weight_decay=weight_decay, eps=eps,
                        maximize=maximize, amsgrad=vmax is not None, grad_scale=None,
                        found_inf=None)


@pytest.mark.parametrize("case", [
    dict(step=1, zero_state=True), dict(step=3, betas=(0.9, 0.999)), dict(step=50, betas=(0.3, 0.95)),
    dict(step=1000), dict(step=1000, maximize=True), dict(step=7, weight_decay=0.0),
    dict(step=1000, amsgrad=True), dict(step=123456), dict(step=1000, lr=0.0),
])
def test_torch_fused_matches_oracle(dev, case):
    """Pins the oracle's fused=True chain: torch's own _fused_adamw_ equals it bit for bit."""
    n = (1 << 20) + 3
    hp = dict(HP)
    hp.update({k: case[k] for k in ("betas", "weight_decay", "lr") if k in case})
    maximize = case.get("maximize", False)
    p = torch.randn(n, device=dev, generator=gen(dev, 1)) * 0.02
    g = torch.randn(n, device=dev, generator=gen(dev, 2)) * 1e-3
    if case.get("zero_state"):
        m, v = torch.zeros_like(p), torch.zeros_like(p)
    else:
        m = torch.randn(n, device=dev, generator=gen(dev, 3)) * 1e-3
        v = (torch.randn(n, device=dev, generator=gen(dev, 4)) * 1e-6).abs()
    x = (v * 1.5).clone() if case.get("amsgrad") else None
    if x is not None:
        x[::2] = 0
    pn, gn, mn, vn = to_np(p).copy(), to_np(g).copy(), to_np(m).copy(), to_np(v).copy()
    xn = None if x is None else to_np(x).copy()
    _fused_torch(p, g, m, v, case["step"], maximize=maximize, vmax=x, **hp)
    O.adamw_step_fused(pn, gn, mn, vn, step=case["step"], maximize=maximize, vmax=xn, **hp)
    assert O.max_ulp(pn, to_np(p))[0] == 0
    assert O.max_ulp(mn, to_np(m))[0] == 0
    assert O.max_ulp(vn, to_np(v))[0] == 0
    if x is not None:
        assert O.max_ulp(xn, to_np(x))[0] == 0


@pytest.mark.parametrize("beta", [0.9, 0.95, 0.999, 0.99, 0.98, 0.3, 0.5])
def test_host_per_step_values_match_the_device(dev, beta):
    """The library forms bc1 = f32(1 - pow(beta1, step)) and bc2_sqrt = f32(sqrt(1 -
    pow(beta2, step))) on the host with libm pow; torch's kernel forms them on the device.
    The two pow differ in the last float64 bit at some steps; after the roundings to fp32
    the values must agree at every step 1 .. 1e6."""
    steps = np.arange(1, 1_000_001, dtype=np.float32)
    host_bc1, host_bc2s = O.fused_scalars_many(beta, beta, steps)
    st = torch.from_numpy(steps.astype(np.float64)).to(dev)
    dpow = torch.pow(torch.full_like(st, beta), st)
    dev_bc1 = to_np((1 - dpow).float())
    dev_bc2s = to_np(torch.sqrt(1 - dpow).float())
    assert int((host_bc1 != dev_bc1).sum()) == 0
    assert int((host_bc2s != dev_bc2s).sum()) == 0


def _compare(ours, ref, opt, topt, ams=False):
    for a, b in zip(ours, ref):
        assert max_ulp(a, b) == 0
        sa, sb = opt.state[a], topt.state[b]
        assert max_ulp(sa["exp_avg"], sb["exp_avg"]) == 0
        assert max_ulp(sa["exp_avg_sq"], sb["exp_avg_sq"]) == 0
        assert float(sa["step"]) == float(sb["step"])
        if ams:
            assert max_ulp(sa["max_exp_avg_sq"], sb["max_exp_avg_sq"]) == 0


@pytest.mark.parametrize("flat", [False, True])
@pytest.mark.parametrize("variant", ["plain", "no_wd", "maximize", "amsgrad", "lr_cpu_tensor",
                                     "lr_device_tensor", "midtrain"])
def test_fused_true_matches_torch_fused(dev, flat, variant):
    """Six chained steps with gradients that move every step (as after zero_grad), so
    every step after the first goes through the native host path."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    hp = dict(HP)
    if variant == "no_wd":
        hp["weight_decay"] = 0.0
    lr_ref = lr_ours = hp.pop("lr")
    if variant == "lr_cpu_tensor":
        lr_ref, lr_ours = torch.tensor(lr_ref), torch.tensor(lr_ours)
    elif variant == "lr_device_tensor":
        lr_ref = torch.tensor(lr_ref, device=dev)
        lr_ours = torch.tensor(lr_ours, device=dev)
    kw = dict(maximize=variant == "maximize", amsgrad=variant == "amsgrad")
    topt = torch.optim.AdamW(ref, lr=lr_ref, fused=True, **hp, **kw)
    opt = mi_adamw.FusedAdamW(ours, lr=lr_ours, fused=True, flat_buffer=flat, **hp, **kw)
    if variant == "midtrain":
        states = midtrain_state(ref, 1000.0)
        load_states(topt, ref, states)
        load_states(opt, ours, states)
    for step in range(6):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            if flat and q.grad is not None:
                q.grad.copy_(p.grad)          # the flat layout keeps its gradient views
            else:
                q.grad = p.grad.clone()
        topt.step()
        opt.step()
        _compare(ours, ref, opt, topt, ams=kw["amsgrad"])
        if not flat:
            opt.zero_grad()
            topt.zero_grad()
    if not flat:
        assert opt.native_steps >= 4


def test_fused_true_with_clip(dev):
    """fused=True with the fused clip, against torch's clip_grads_with_norm_ at the kernel's
    own norm and then torch's fused AdamW: bit-identical, over five chained steps."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, fused=True, **HP)
    opt = mi_adamw.FusedAdamW(ours, fused=True, max_grad_norm=1.0, **HP)
    states = midtrain_state(ref, 1000.0)
    load_states(topt, ref, states)
    load_states(opt, ours, states)
    for step in range(5):
        set_grads(ref, step, 1e-1)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        opt.step()
        norm = opt.last_grad_norm
        assert norm.item() > 1.0
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, norm.clone())
        topt.step()
        _compare(ours, ref, opt, topt)


@pytest.mark.filterwarnings("ignore:This instance was constructed with capturable=True")
@pytest.mark.parametrize("capturable", [False, True])
@pytest.mark.parametrize("flat", [False, True])
def test_fused_true_clip_write_grads_matches_torch(dev, flat, capturable):
    """fused=True with the clip storing the clipped gradients (clip_write_grads) and the
    bf16 copy: the stored gradients equal torch's clip_grads_with_norm_ at the kernel's own
    norm, and p, m, v equal torch's fused AdamW after it, over three chained steps; the
    copy is the bf16 of p.  capturable=True runs the chain's device-step kernel."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, fused=True, capturable=capturable, **HP)
    opt = mi_adamw.FusedAdamW(ours, fused=True, capturable=capturable, max_grad_norm=1.0,
                              clip_write_grads=True, bf16_copy=True, flat_buffer=flat, **HP)
    states = midtrain_state(ref, 1000.0)
    load_states(topt, ref, states)
    load_states(opt, ours, states)
    for step in range(3):
        set_grads(ref, step, 1e-1)
        for p, q in zip(ref, ours):
            if flat and q.grad is not None:
                q.grad.copy_(p.grad)
            else:
                q.grad = p.grad.clone()
        opt.step()
        norm = opt.last_grad_norm
        assert norm.item() > 1.0
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, norm.clone())
        topt.step()
        _compare(ours, ref, opt, topt)
        for p, q in zip(ref, ours):
            assert max_ulp(q.grad, p.grad) == 0
            assert torch.equal(opt.bf16_param(q).view(torch.int16),
                               q.detach().to(torch.bfloat16).view(torch.int16))


@pytest.mark.filterwarnings("ignore:This instance was constructed with capturable=True")
def test_fused_true_capturable_replayed_from_a_graph(dev):
    """capturable=True with fused=True: torch runs the fused kernel on device step counts;
    here the fused chain forms the per-step values from the device counts.  Two eager
    steps, then a graph of one step replayed three times: bit-identical throughout."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, fused=True, capturable=True, **HP)
    opt = mi_adamw.FusedAdamW(ours, fused=True, capturable=True, **HP)
    for p, q in zip(ref, ours):
        p.grad = torch.zeros_like(p)
        q.grad = torch.zeros_like(q)

    def fill(step):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad.copy_(p.grad)

    for step in range(2):
        fill(step)
        topt.step()
        opt.step()
        _compare(ours, ref, opt, topt)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            opt.step()
    torch.cuda.current_stream().wait_stream(s)
    for step in range(2, 5):
        fill(step)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        topt.step()
        _compare(ours, ref, opt, topt)


def test_fused_true_bf16_state_matches_oracle(dev):
    """bf16 moments with the fused=True chain (no torch counterpart: its fused kernel keeps
    the moments in the parameters' dtype): against the oracle's fused chain on bf16-stored
    moments, fp32 math, round-to-nearest-even stores."""
    import mi_adamw
    ps = make_params(SHAPES, dev)
    opt = mi_adamw.FusedAdamW(ps, fused=True, state_dtype=torch.bfloat16, max_grad_norm=1.0,
                              **HP)
    pn = [to_np(p).copy() for p in ps]
    mb = [np.zeros(p.numel(), np.uint16) for p in ps]
    vb = [np.zeros(p.numel(), np.uint16) for p in ps]
    for step in range(1, 4):
        set_grads(ps, step, 3e-2)
        gn = [to_np(p.grad).reshape(-1).copy() for p in ps]
        opt.step()
        coef = float(O.clip_coef(O.total_norm(gn), 1.0))
        for i in range(len(ps)):
            pi = pn[i].reshape(-1)
            O.adamw_step_fused_bf16state(pi, gn[i], mb[i], vb[i], lr=HP["lr"], betas=HP["betas"],
                                         eps=HP["eps"], weight_decay=HP["weight_decay"],
                                         step=step, grad_scale=coef)
            st = opt.state[ps[i]]
            assert O.max_ulp(pi, to_np(ps[i]).reshape(-1))[0] == 0
            assert np.array_equal(mb[i], to_np(st["exp_avg"].view(torch.int16)).view(np.uint16)
                                  .reshape(-1))
            assert np.array_equal(vb[i], to_np(st["exp_avg_sq"].view(torch.int16))
                                  .view(np.uint16).reshape(-1))


def test_fused_true_range_step_equals_the_flat_step(dev):
    """ZeroRangeStep over a fused=True optimizer: every rank's slice in the fused chain,
    bit-identical to opt.step() on a copy (world 3, clip, bf16 copy)."""
    import mi_adamw
    from mi_adamw.zero import ZeroRangeStep
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    kw = dict(fused=True, flat_buffer=True, max_grad_norm=1.0, bf16_copy=True, **HP)
    oa = mi_adamw.FusedAdamW(a, **kw)
    ob = mi_adamw.FusedAdamW(b, **kw)
    zr = ZeroRangeStep(ob, 3)
    for step in range(3):
        set_grads(a, step, 3e-2)
        for p, q in zip(a, b):
            if q.grad is None:
                q.grad = p.grad.clone()
            else:
                q.grad.copy_(p.grad)
        oa.step()
        zr.step()
        for p, q in zip(a, b):
            assert max_ulp(p, q) == 0
            for k in ("exp_avg", "exp_avg_sq"):
                assert max_ulp(oa.state[p][k], ob.state[q][k]) == 0
        for x, y in zip(oa.bf16_params(), ob.bf16_params()):
            assert torch.equal(x, y)


def test_mixed_groups_each_take_their_chain(dev):
    """One group with fused=True and one without: each steps in its own chain, as torch
    steps each group with its own setting."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    half = len(SHAPES) // 2

    def groups(ps):
        return [{"params": ps[:half], "fused": True},
                {"params": ps[half:], "fused": False, "foreach": False}]

    topt = torch.optim.AdamW(groups(ref), **HP)
    opt = mi_adamw.FusedAdamW(groups(ours), **HP)
    for step in range(3):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        opt.step()
        _compare(ours, ref, opt, topt)


def test_reference_schedule_and_checkpoint_interchange(dev):
    """The reference's warm-up + cosine LambdaLR (main.py:178-180) over 40 steps with
    fused=True; at step 20 each optimizer's state_dict is loaded into the other kind and
    both pairs continue bit-identical."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    hp = dict(lr=6e-4, weight_decay=0.1)
    topt = torch.optim.AdamW(ref, fused=True, **hp)
    opt = mi_adamw.FusedAdamW(ours, fused=True, **hp)
    warm, total = 10, 40

    def lam(it):
        if it < warm:
            return it / warm
        return 0.5 * (1 + math.cos(math.pi * (it - warm) / (total - warm)))

    ts = torch.optim.lr_scheduler.LambdaLR(topt, lam)
    os_ = torch.optim.lr_scheduler.LambdaLR(opt, lam)
    for step in range(total):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        opt.step()
        ts.step()
        os_.step()
        _compare(ours, ref, opt, topt)
        if step == 20:
            sd_t, sd_o = topt.state_dict(), opt.state_dict()
            opt.load_state_dict(sd_t)
            topt.load_state_dict(sd_o)
            _compare(ours, ref, opt, topt)
        opt.zero_grad()
        topt.zero_grad()


def test_fused_true_refuses_complex_params_as_torch_does(dev):
    """torch's fused kernel takes real floating-point params only: AdamW(fused=True) raises
    at a complex parameter's first step, with this message, and so does FusedAdamW."""
    import mi_adamw
    msgs = []
    for cls in (torch.optim.AdamW, mi_adamw.FusedAdamW):
        p = torch.nn.Parameter(torch.randn(8, dtype=torch.complex64, device=dev))
        p.grad = torch.randn_like(p)
        opt = cls([p], fused=True, **HP)
        with pytest.raises(RuntimeError) as e:
            opt.step()
        msgs.append(str(e.value))
    assert msgs[0] == msgs[1] and "`fused=True` requires" in msgs[0]


SPECIALS = [0.0, -0.0, 1e-45, -1e-45, 1e-40, -3e-39, 1.17e-38, 1e-30, -1e-20, 1e-8, 1.0, -1.0,
            3e4, -1e15, 1e30, 3.4e38, float("inf"), float("-inf"), float("nan")]


def _grid(specials):
    """Every combination of a special p, g, m and |v| (v >= 0 as in real state)."""
    s = torch.tensor(specials, dtype=torch.float32)
    idx = torch.cartesian_prod(*(torch.arange(s.numel()) for _ in range(4)))
    pv, gv, mv, vv = (s[idx[:, j]] for j in range(4))
    return pv, gv, mv, vv.abs()


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Equal NaN positions and identical bits elsewhere (signed zeros told apart)."""
    a, b = a.reshape(-1), b.reshape(-1)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                          b[~nb].view(np.uint32)))


@pytest.mark.parametrize("case", [
    dict(betas=(0.9, 0.95), step=1.0, maximize=False, weight_decay=0.1),
    dict(betas=(0.3, 0.999), step=7.0, maximize=True, weight_decay=0.1),
    dict(betas=(0.9, 0.95), step=1000.0, maximize=False, weight_decay=0.0),
    dict(betas=(0.9, 0.999), step=20.0, maximize=False, weight_decay=0.1, amsgrad=True),
])
def test_fused_true_special_values_match_torch_fused(dev, case):
    """Denormals, signed zeros, tiny and huge magnitudes, inf and NaN in p, g, m, v (and the
    amsgrad maximum): FusedAdamW(fused=True) equals torch.optim.AdamW(fused=True) bit for
    bit, and the oracle's fused chain equals both (which pins it on these values)."""
    import mi_adamw
    pv, gv, mv, vv = _grid(SPECIALS)
    ams = case.get("amsgrad", False)
    xv = vv.roll(1) if ams else None          # a maximum unrelated to v, specials included
    hp = dict(lr=1e-3, betas=case["betas"], eps=1e-8, weight_decay=case["weight_decay"],
              maximize=case["maximize"], amsgrad=ams)
    st = {"step": torch.tensor(case["step"] - 1), "exp_avg": mv.clone(), "exp_avg_sq": vv.clone()}
    if ams:
        st["max_exp_avg_sq"] = xv.clone()
    out = []
    for cls in (torch.optim.AdamW, mi_adamw.FusedAdamW):
        p = torch.nn.Parameter(pv.clone().to(dev))
        p.grad = gv.clone().to(dev)
        opt = cls([p], fused=True, **hp)
        load_states(opt, [p], [st])
        opt.step()
        torch.cuda.synchronize()
        s = opt.state[p]
        out.append([to_np(t) for t in (p, s["exp_avg"], s["exp_avg_sq"])]
                   + ([to_np(s["max_exp_avg_sq"])] if ams else []))
    pn, mn, vn = pv.numpy().copy(), mv.numpy().copy(), vv.numpy().copy()
    xn = xv.numpy().copy() if ams else None
    O.adamw_step_fused(pn, gv.numpy().copy(), mn, vn, lr=hp["lr"], betas=hp["betas"],
                       eps=hp["eps"], weight_decay=hp["weight_decay"], step=case["step"],
                       maximize=hp["maximize"], vmax=xn)
    oracle = [pn, mn, vn] + ([xn] if ams else [])
    for what, t, o, orc in zip("pmvx", out[0], out[1], oracle):
        assert _same_bits(t, o), (what, case)
        assert _same_bits(t, orc), (what, case, "oracle")
    print(f"{pv.numel()} special combinations, {case}: identical", flush=True)


def test_fused_true_special_values_bf16_state_match_oracle(dev):
    """The special-value grid with bf16 moments and the bf16 copy in the fused=True chain,
    against the oracle's fused chain on bf16-stored moments: bf16 rounding of inf, NaN,
    denormals and overflow to inf."""
    import mi_adamw
    pv, gv, mv, vv = _grid([0.0, -0.0, 1e-45, -1e-40, 9.2e-41, 1.17e-38, 1e-30, -1e-20, 1e-8,
                            1.0, -1.0, 3e4, 3.3961e38, 3.4e38, float("inf"), float("-inf"),
                            float("nan")])
    p = torch.nn.Parameter(pv.clone().to(dev))
    p.grad = gv.clone().to(dev)
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    opt = mi_adamw.FusedAdamW([p], fused=True, state_dtype=torch.bfloat16, bf16_copy=True, **hp)
    load_states(opt, [p], [{"step": torch.tensor(4.0), "exp_avg": mv.clone(),
                            "exp_avg_sq": vv.clone()}])
    opt.step()
    torch.cuda.synchronize()
    pn = pv.numpy().copy()
    mb = O.to_bf16_bits(mv.numpy())
    vb = O.to_bf16_bits(vv.numpy())
    O.adamw_step_fused_bf16state(pn, gv.numpy().copy(), mb, vb, step=5.0, **hp)
    assert _same_bits(pn, to_np(p))
    got_m = to_np(opt.state[p]["exp_avg"].view(torch.int16)).view(np.uint16)
    got_v = to_np(opt.state[p]["exp_avg_sq"].view(torch.int16)).view(np.uint16)
    assert np.array_equal(got_m, mb) and np.array_equal(got_v, vb)
    copy = to_np(opt.bf16_param(p).view(torch.int16)).view(np.uint16)
    assert np.array_equal(copy, O.to_bf16_bits(pn))
    print(f"{pv.numel()} special combinations with bf16 state: identical to the oracle",
          flush=True)
