"""The native host path of FusedAdamW.step() (csrc/host.cpp) against torch, on the GPU.

After the first step, steps whose only change is where the gradients live (the
reference loop: zero_grad() frees them, backward allocates new ones, main.py:204-209)
go through the C++ path: it checks every parameter, state entry and step count, patches
the moved gradient pointers into the device table and launches.  Everything else must
fall back to the general path before anything is changed.  Each test runs chained
steps with gradients that move every step and compares with torch.optim.AdamW
(foreach=False), bit for bit, and checks that the native path did take the steps it
should.
"""
from __future__ import annotations

import copy
import gc

import pytest
import torch

from _helpers import (clone_params, gen, load_states, make_params, max_ulp_all, midtrain_state,
                      rel_err)

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SHAPES = [(64, 48), (48,), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (0,),
          (65536 + 12,), (1024,)]


@pytest.fixture
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    yield torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()


def _fresh_grads(params, step, std=3e-2):
    """New gradient tensors, as backward allocates them after zero_grad(set_to_none=True);
    a spacer allocation between steps keeps the allocator from handing back the same
    blocks, so the addresses move."""
    out = []
    for i, p in enumerate(params):
        out.append(torch.randn(p.shape, device=p.device,
                               generator=gen(p.device, 4000 + 10000 * step + i)) * std)
    return out


def _assign(ref, ours, grads, spacer, inplace=False):
    """ref gets new gradient tensors; ours too, or (inplace: the flat layout, whose
    gradients are views of its buffer that backward accumulates into) the values are
    written into its gradient views."""
    for p, q, g in zip(ref, ours, grads):
        p.grad = g.clone()
        spacer.append(torch.empty(1 << 16, device=g.device))
        if inplace and q.grad is not None:
            q.grad.copy_(g)
        else:
            q.grad = g.clone()


def _same(ref, ours, topt, oopt):
    d = (max_ulp_all(list(ref), list(ours)),
         max_ulp_all([topt.state[p]["exp_avg"] for p in ref if p.numel()],
                     [oopt.state[q]["exp_avg"] for q in ours if q.numel()]),
         max_ulp_all([topt.state[p]["exp_avg_sq"] for p in ref if p.numel()],
                     [oopt.state[q]["exp_avg_sq"] for q in ours if q.numel()]))
    return max(d)


def _groups(params, two):
    if not two:
        return params
    return [{"params": params[:5]}, {"params": params[5:], "lr": 1e-3, "weight_decay": 0.0}]


@pytest.mark.parametrize("clip", [False, True])
@pytest.mark.parametrize("layout,two_groups", [("tables", False), ("tables", True),
                                               ("flat", False), ("flat", True),
                                               ("single", False)])
def test_native_path_matches_torch_with_moving_gradients(dev, clip, layout, two_groups):
    import mi_adamw
    shapes = [(4099,)] if layout == "single" else SHAPES
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(_groups(ref, two_groups), foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(_groups(ours, two_groups), **HP,
                               max_grad_norm=1.0 if clip else None,
                               flat_buffer=layout == "flat")
    states = midtrain_state(ref, 1000.0)
    load_states(topt, ref, states)
    load_states(oopt, ours, states)
    spacer = []
    for step in range(8):
        topt.zero_grad(set_to_none=True)
        oopt.zero_grad(set_to_none=True)
        _assign(ref, ours, _fresh_grads(ref, step), spacer, inplace=layout == "flat")
        oopt.step()
        if clip:
            torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    assert _same(ref, ours, topt, oopt) == 0
    assert all(float(oopt.state[q]["step"]) == 1008.0 for q in ours)
    print(f"clip {clip} {layout} two_groups {two_groups}: native steps {oopt.native_steps} of 8",
          flush=True)
    assert oopt.native_steps == 7


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_native_path_bf16_copy_and_state(dev, state_dtype):
    """bf16 copy (and bf16 moments) through the native path equal the general path's."""
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=True, state_dtype=state_dtype)
    oa = mi_adamw.FusedAdamW(a, **kw)
    ob = mi_adamw.FusedAdamW(b, **kw)
    spacer = []
    for step in range(6):
        _assign(a, b, _fresh_grads(a, step), spacer)
        oa._fast = None              # the general path every step
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert oa.native_steps == 0 and ob.native_steps == 5
    for p, q in zip(a, b):
        assert torch.equal(p, q)
        if p.numel():
            for k in ("exp_avg", "exp_avg_sq"):
                assert torch.equal(oa.state[p][k], ob.state[q][k])
        assert torch.equal(oa.bf16_param(p), ob.bf16_param(q))


def test_native_path_falls_back_on_every_other_change(dev):
    """Changes the native path must not take: a gradient set to None, a state tensor
    replaced, p.data replaced, another stream, a checkpoint loaded.  Each step still
    equals torch's."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(_groups(ref, True), foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(_groups(ours, True), **HP, max_grad_norm=1.0)
    spacer = []
    log = []

    def step(k, note):
        before = oopt.native_steps
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(
            [p for p in ref if p.grad is not None], 1.0, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        d = _same(ref, ours, topt, oopt)
        log.append((k, note, oopt.native_steps - before, d))
        assert d == 0, log[-1]

    k = 0
    for note in ("first", "native", "native"):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        step(k, note)
        k += 1
    # a state tensor replaced in the dict
    for opt, p in ((topt, ref[3]), (oopt, ours[3])):
        opt.state[p]["exp_avg"] = opt.state[p]["exp_avg"].clone() * 0.5
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    step(k, "state replaced")
    k += 1
    # p.data replaced with new storage
    with torch.no_grad():
        ref[0].data = ref[0].data.clone()
        ours[0].data = ours[0].data.clone()
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    step(k, "p.data replaced")
    k += 1
    # another stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        step(k, "side stream")
        k += 1
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        step(k, "side stream native")
        k += 1
    torch.cuda.current_stream().wait_stream(side)
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    step(k, "back on the default stream")
    k += 1
    # a checkpoint of torch's state loaded into ours
    # (copied: load_state_dict keeps same-device tensors, as torch's does, and both
    # optimizers would then update one set of moments)
    oopt.load_state_dict(copy.deepcopy(topt.state_dict()))
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    step(k, "after load_state_dict")
    k += 1
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    step(k, "native")
    k += 1
    # a parameter without a gradient is skipped (torch semantics); its step count then
    # lags its group's, which needs two hyperparameter sets from then on: general path
    _assign(ref, ours, _fresh_grads(ref, k), spacer)
    ref[2].grad = None
    ours[2].grad = None
    step(k, "grad None")
    k += 1
    for _ in range(2):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        step(k, "two step counts in a group")
        k += 1
    for row in log:
        print(row, flush=True)
    native = {note: n for _, note, n, _ in log}
    assert native["grad None"] == 0 and native["state replaced"] == 0
    assert native["two step counts in a group"] == 0
    assert native["p.data replaced"] == 0 and native["after load_state_dict"] == 0
    assert native["side stream"] == 0 and native["side stream native"] == 1
    assert native["native"] == 1


@pytest.mark.parametrize("layout", ["tables", "flat"])
@pytest.mark.parametrize("view", ["strided", "transposed", "restrided_in_place"])
def test_state_replaced_by_a_non_dense_view(dev, view, layout):
    """A moment put into the state dict as a view that is not dense (every other element
    of a larger buffer, or a transposed matrix), or re-strided in place through .data
    (same object and address, its elements read in another order, done to torch's state
    too) after the native path has a plan: the step falls back, replaces the entry by a
    dense copy with the same values and steps it like torch (whose per-tensor ops take any
    strides); the next steps are native again.  In the flat layout the values go into
    the tensor's slice of the moment buffer (its own memory, when re-strided in place).
    The buffer around the strided view is never written."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    flat = layout == "flat"
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, flat_buffer=flat)
    spacer = []
    for k in range(2):
        _assign(ref, ours, _fresh_grads(ref, k), spacer, inplace=flat)
        oopt.step()
        topt.step()
    j = 7 if view == "strided" else 3          # (70001,) or (144, 48)
    st = oopt.state[ours[j]]
    if view == "restrided_in_place":
        for opt, ps in ((oopt, ours), (topt, ref)):
            v = opt.state[ps[j]]["exp_avg_sq"]
            ptr = v.data_ptr()
            v.data = v.data.as_strided((144, 48), (1, 144))
            assert v.data_ptr() == ptr and not v.is_contiguous()
    elif view == "strided":
        guard = torch.full((2 * ours[j].numel(),), 7.0, device=dev)
        t = guard[::2]
        t.copy_(st["exp_avg"])
        st["exp_avg"] = t
    else:
        v = st["exp_avg_sq"]
        st["exp_avg_sq"] = v.t().contiguous().t()
        assert not st["exp_avg_sq"].is_contiguous()
    before = oopt.native_steps
    for k in range(2, 5):
        _assign(ref, ours, _fresh_grads(ref, k), spacer, inplace=flat)
        oopt.step()
        topt.step()
        torch.cuda.synchronize()
        assert _same(ref, ours, topt, oopt) == 0, k
    assert oopt.native_steps - before == 2
    for key in ("exp_avg", "exp_avg_sq"):
        assert st[key].is_contiguous()
    if view == "strided":
        assert torch.equal(guard[1::2], torch.full_like(guard[1::2], 7.0))


def test_native_path_follows_the_lr_schedule(dev):
    """LambdaLR rewrites group["lr"] every iteration (main.py:178-180,210): the native path
    forms the scalars from the groups at every step."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, lr=6e-4, weight_decay=0.1)
    oopt = mi_adamw.FusedAdamW(ours, lr=6e-4, weight_decay=0.1, fused=False)
    fn = lambda it: min(1.0, (it + 1) / 5)          # noqa: E731
    ts = torch.optim.lr_scheduler.LambdaLR(topt, fn)
    os_ = torch.optim.lr_scheduler.LambdaLR(oopt, fn)
    spacer = []
    for step in range(10):
        _assign(ref, ours, _fresh_grads(ref, step), spacer)
        oopt.step()
        topt.step()
        ts.step()
        os_.step()
    torch.cuda.synchronize()
    assert _same(ref, ours, topt, oopt) == 0
    assert oopt.native_steps == 9


def test_native_path_grad_prescale_and_norm(dev):
    import mi_adamw
    world = 6
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0,
                               grad_prescale=mi_adamw.dp_prescale(world))
    spacer = []
    for step in range(5):
        _assign(ref, ours, _fresh_grads(ref, step, 0.2), spacer)
        oopt.step()
        for p in ref:
            p.grad.div_(world)
        tn = torch.nn.utils.get_total_norm([p.grad for p in ref])
        assert rel_err(oopt.last_grad_norm, tn) <= 1e-6
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    assert _same(ref, ours, topt, oopt) == 0
    assert oopt.native_steps == 4


def test_amsgrad_switched_off_for_one_group(dev):
    """Two amsgrad groups, then amsgrad switched off for the second and on again (the
    state keeps its max_exp_avg_sq, as torch's does).  The split into launches follows
    the groups' setting at every step: a cached launch made for another split is never
    reused, on the native or the general path."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(_groups(ref, True), foreach=False, amsgrad=True, **HP)
    oopt = mi_adamw.FusedAdamW(_groups(ours, True), amsgrad=True, **HP, max_grad_norm=1.0)
    spacer = []
    schedule = [True, True, True, False, False, False, True, True]
    for k, flag in enumerate(schedule):
        topt.param_groups[1]["amsgrad"] = flag
        oopt.param_groups[1]["amsgrad"] = flag
        # shrinking gradients, so the running maximum differs from v
        _assign(ref, ours, _fresh_grads(ref, k, 3e-2 * 0.5 ** k), spacer)
        before = oopt.native_steps
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        d = _same(ref, ours, topt, oopt)
        dx = max_ulp_all([topt.state[p]["max_exp_avg_sq"] for p in ref if p.numel()],
                         [oopt.state[q]["max_exp_avg_sq"] for q in ours if q.numel()])
        print(f"step {k} amsgrad(group 1) {flag}: native {oopt.native_steps - before}, "
              f"ulp {d}, max_exp_avg_sq ulp {dx}", flush=True)
        assert d == 0 and dx == 0
        # one launch while both groups agree (native from the second such step); two
        # launches while they differ, which only the general path makes
        assert oopt.native_steps == before + (1 if k in (1, 2, 7) else 0)


def test_parameter_swapped_into_a_group_in_place(dev):
    """A parameter replaced inside a group's list (same list object, same length): both
    paths notice it, and the new parameter starts from fresh state, as torch's does."""
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0)
    spacer = []
    for k in range(3):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    new_ref = torch.nn.Parameter(torch.randn(SHAPES[4], device=dev))
    new_ours = torch.nn.Parameter(new_ref.detach().clone())
    topt.param_groups[0]["params"][4] = new_ref
    oopt.param_groups[0]["params"][4] = new_ours
    ref[4], ours[4] = new_ref, new_ours
    before = oopt.native_steps
    for k in range(3, 6):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    assert _same(ref, ours, topt, oopt) == 0
    assert float(oopt.state[new_ours]["step"]) == 3.0
    # the new parameter's step count differs from the others: two hyperparameter sets in
    # one group, which only the general path launches
    assert oopt.native_steps == before


def test_parameter_swapped_into_a_flat_group_is_refused(dev):
    """The flat layout's buffers have no slice for a parameter put into a group's list
    after construction: the step refuses it before anything is launched or changed."""
    import mi_adamw
    ours = make_params(SHAPES, dev)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0, flat_buffer=True)
    spacer = []
    for k in range(2):
        _assign(ours, ours, _fresh_grads(ours, k), spacer, inplace=True)
        oopt.step()
    before = oopt._flat.param.clone()
    new = torch.nn.Parameter(torch.randn(SHAPES[4], device=dev))
    new.grad = torch.randn_like(new)
    oopt.param_groups[0]["params"][4] = new
    with pytest.raises(NotImplementedError, match="after construction"):
        oopt.step()
    torch.cuda.synchronize()
    assert torch.equal(oopt._flat.param, before)


@pytest.mark.parametrize("layout", ["tables", "single"])
def test_parameter_restrided_in_place_is_refused(dev, layout):
    """p.data replaced by a transposed view of its own storage (same address and element
    count, another element order) with a dense gradient of the new shape: the kernels
    step by memory position, so both step paths must refuse it rather than pair p's
    elements with the wrong gradients."""
    import mi_adamw
    shapes = [(65, 63)] if layout == "single" else SHAPES
    ours = make_params(shapes, dev)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0)
    spacer = []
    for k in range(3):
        _assign(ours, ours, _fresh_grads(ours, k), spacer)
        oopt.step()
    assert oopt.native_steps == 2
    p = ours[0]
    ptr = p.data_ptr()
    with torch.no_grad():
        p.data = p.data.t()
    assert p.data_ptr() == ptr and not p.is_contiguous()
    before = [q.detach().clone() for q in ours]
    _assign(ours, ours, _fresh_grads(ours, 3), spacer)
    with pytest.raises(NotImplementedError, match="contiguous"):
        oopt.step()
    torch.cuda.synchronize()
    assert oopt.native_steps == 2
    assert all(torch.equal(q, b) for q, b in zip(ours, before))


@pytest.mark.parametrize("layout", ["tables", "single"])
def test_parameter_narrowed_in_place_is_refused(dev, layout):
    """p.data narrowed to a view at the same address, then a gradient of the new size:
    torch's AdamW raises at the size mismatch with exp_avg, and so must both step paths,
    before any kernel reads the old row size from the smaller gradient."""
    import mi_adamw
    shapes = [(4099,)] if layout == "single" else SHAPES
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0)
    spacer = []
    for k in range(3):
        _assign(ref, ours, _fresh_grads(ref, k), spacer)
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    assert oopt.native_steps == 2
    j = 0 if layout == "single" else 4
    for p in (ref[j], ours[j]):
        ptr = p.data_ptr()
        with torch.no_grad():
            p.data = p.data[:1000]
        assert p.data_ptr() == ptr
    _assign(ref, ours, _fresh_grads(ref, 3), spacer)
    with pytest.raises(RuntimeError):
        topt.step()
    with pytest.raises(RuntimeError, match="elements"):
        oopt.step()
    torch.cuda.synchronize()
    assert oopt.native_steps == 2
