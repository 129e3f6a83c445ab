"""ZeRO-1 range sharding and the data-parallel gradient pre-scale, on the GPU.

1. The pre-scale: ``FusedAdamW(grad_prescale=dp_prescale(world))`` on summed gradients
   equals torch's ``grad.div_(world)`` (parallel/data_parallel.py:15), then
   ``clip_grads_with_norm_`` with the same norm, then ``AdamW(foreach=False).step()``,
   bit for bit, over chained steps; the norm within 1e-6 of torch's over the divided
   gradients; with clip_write_grads the stored gradients equal torch's.
2. Range sharding: ``ZeroRangeStep(opt, R).step()`` (R ranks' partial sums, the
   finalize over them, every rank's slice) equals the unsharded flat step bit for bit:
   parameters, moments, bf16 copy and norm, with slices that cut through tensors and
   param groups, fp32 and bf16 moments; and at the 6.7B GPT shape for R = 2, 4, 8.
"""
from __future__ import annotations

import gc

import pytest
import torch

from _helpers import (clone_params, gen, gpt_params, load_states, make_params, max_ulp_all,
                      midtrain_state, rel_err, set_grads)

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SHAPES = [(64, 48), (48,), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (65536 + 12,),
          (1024,), (33,)]


@pytest.fixture
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    yield torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()


def _state_ulps(ref, ours, topt, oopt):
    return (max_ulp_all(list(ref), list(ours)),
            max_ulp_all([topt.state[p]["exp_avg"] for p in ref],
                        [oopt.state[q]["exp_avg"] for q in ours]),
            max_ulp_all([topt.state[p]["exp_avg_sq"] for p in ref],
                        [oopt.state[q]["exp_avg_sq"] for q in ours]))


@pytest.mark.parametrize("world", [2, 3, 6, 8])
@pytest.mark.parametrize("clip", [False, True])
@pytest.mark.parametrize("flat", [False, True])
def test_prescale_equals_torch_div_then_adamw(dev, world, clip, flat):
    import mi_adamw
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0 if clip else None,
                               flat_buffer=flat, grad_prescale=mi_adamw.dp_prescale(world))
    states = midtrain_state(ref, 1000.0)
    load_states(topt, ref, states)
    load_states(oopt, ours, states)
    worst_norm = 0.0
    for step in range(3):
        # the all-reduced (summed) gradients of `world` ranks, scaled so the clip triggers
        set_grads(ref, step, 3e-2 * world)
        for p, q in zip(ref, ours):
            q.grad.copy_(p.grad) if q.grad is not None else setattr(q, "grad", p.grad.clone())
        oopt.step()
        for p in ref:
            p.grad.div_(world)                              # parallel/data_parallel.py:15
        if clip:
            tn = torch.nn.utils.get_total_norm([p.grad for p in ref])
            worst_norm = max(worst_norm, rel_err(oopt.last_grad_norm, tn))
            torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    d = _state_ulps(ref, ours, topt, oopt)
    print(f"world {world} clip {clip} flat {flat}: ulp (p, m, v) {d}, norm rel {worst_norm:.3g}",
          flush=True)
    assert max(d) == 0
    assert worst_norm <= 1e-6
    if clip:
        assert float(oopt.last_grad_norm) > 1.0       # the clip did scale


def test_prescale_with_clip_write_grads_stores_torchs_gradients(dev):
    import mi_adamw
    world = 3
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    oopt = mi_adamw.FusedAdamW(ours, **HP, max_grad_norm=1.0, clip_write_grads=True,
                               grad_prescale=mi_adamw.dp_prescale(world))
    set_grads(ref, 0, 1e-1)
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()
    oopt.step()
    for p in ref:
        p.grad.div_(world)
    torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
    topt.step()
    torch.cuda.synchronize()
    assert max(_state_ulps(ref, ours, topt, oopt)) == 0
    assert max_ulp_all([p.grad for p in ref], [q.grad for q in ours]) == 0


def _flat_pair(dev, shapes, state_dtype, groups, prescale):
    """Two flat-layout optimizers over identical params, grads and states."""
    import mi_adamw
    a = make_params(shapes, dev)
    b = clone_params(a)

    def split(ps):
        if groups == 1:
            return ps
        cut = len(ps) // 2
        return [{"params": ps[:cut]}, {"params": ps[cut:], "weight_decay": 0.0, "lr": 1e-3}]
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=True, flat_buffer=True, state_dtype=state_dtype,
              grad_prescale=prescale)
    oa = mi_adamw.FusedAdamW(split(a), **kw)
    ob = mi_adamw.FusedAdamW(split(b), **kw)
    states = midtrain_state(a, 1000.0)
    load_states(oa, a, states)
    load_states(ob, b, states)
    return a, b, oa, ob


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("groups", [1, 2])
def test_range_step_equals_flat_step(dev, state_dtype, groups):
    import mi_adamw
    for world in (1, 2, 3, 4, 8):
        prescale = mi_adamw.dp_prescale(world)
        a, b, oa, ob = _flat_pair(dev, SHAPES, state_dtype, groups, prescale)
        zs = mi_adamw.ZeroRangeStep(ob, world, grad_prescale=prescale)
        bounds = zs.bounds
        assert bounds[0][0] == 0 and bounds[-1][1] == ob._flat.total
        assert all(lo % 32 == 0 for lo, _ in bounds)
        cuts_inside = sum(1 for lo, _ in bounds[1:]
                          if lo not in {off for off in ob._flat.offsets.values()})
        for step in range(3):
            set_grads(a, step, 3e-2 * world)
            for p, q in zip(a, b):
                q.grad.copy_(p.grad)
            oa.step()
            nb = zs.step()
            torch.cuda.synchronize()
            assert torch.equal(oa.last_grad_norm.view(torch.int32), nb.view(torch.int32)), \
                (world, step, float(oa.last_grad_norm), float(nb))
        for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
            x, y = getattr(oa._flat, key), getattr(ob._flat, key)
            assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else
                               x.view(torch.int32),
                               y.view(torch.int16) if y.dtype == torch.bfloat16 else
                               y.view(torch.int32)), (world, key)
        assert all(float(oa.state[p]["step"]) == float(ob.state[q]["step"]) == 1003.0
                   for p, q in zip(a, b))
        assert zs.native_begins == 2          # the first begin() makes the native plan
        print(f"world {world} groups {groups} {state_dtype}: bit-identical, {cuts_inside} "
              f"slice boundaries inside tensors", flush=True)
        del a, b, oa, ob, zs


def test_range_step_takes_the_optimizers_prescale(dev):
    """An optimizer built with grad_prescale, driven by ZeroRangeStep without one: the
    range step pre-scales as the optimizer's own step does, bit for bit."""
    import mi_adamw
    world = 4
    prescale = mi_adamw.dp_prescale(world)
    a, b, oa, ob = _flat_pair(dev, SHAPES, torch.float32, 2, prescale)
    zs = mi_adamw.ZeroRangeStep(ob, world)
    assert zs.grad_prescale == ob.grad_prescale == prescale
    with pytest.raises(ValueError, match="differs"):
        mi_adamw.ZeroRangeStep(ob, world, grad_prescale=1.0)
    for step in range(2):
        set_grads(a, step, 3e-2 * world)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad)
        oa.step()
        nb = zs.step()
        torch.cuda.synchronize()
        assert torch.equal(oa.last_grad_norm.view(torch.int32), nb.view(torch.int32))
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        assert torch.equal(getattr(oa._flat, key), getattr(ob._flat, key)), key


def test_range_step_split_calls_match_step(dev):
    """The per-rank calls in the order a multi-GPU rank makes them: each rank's sum into its
    own float64, the sums combined (the all-reduce), the finalize from the one total."""
    import mi_adamw
    world = 4
    a, b, oa, ob = _flat_pair(dev, SHAPES, torch.float32, 2, 1.0)
    zs = mi_adamw.ZeroRangeStep(ob, world)
    set_grads(a, 0, 3e-2)
    for p, q in zip(a, b):
        q.grad.copy_(p.grad)
    oa.step()
    hypers = zs.begin()
    sums = torch.zeros(world, dtype=torch.float64, device=dev)
    for r in range(world):
        zs.grad_sumsq(r, sums[r:r + 1])
    exact = sum(float(p.grad.double().pow(2).sum()) for p in b)
    total = sums.sum().reshape(1)                       # what an all-reduce would deliver
    norm, coef = zs.finalize(total)
    for r in range(world):
        zs.update(r, hypers, coef)
    torch.cuda.synchronize()
    assert abs(float(total) - exact) <= 1e-12 * exact
    assert torch.equal(norm.view(torch.int32), oa.last_grad_norm.view(torch.int32))
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        x, y = getattr(oa._flat, key), getattr(ob._flat, key)
        assert torch.equal(x, y), key



def test_range_step_takes_back_replaced_tensors(dev):
    """p.data and a moment replaced between steps (new tensors, same sizes): the range
    step copies them into their slices as the flat step does, and both stay bit-identical."""
    import mi_adamw
    a, b, oa, ob = _flat_pair(dev, SHAPES, torch.float32, 2, 1.0)
    zs = mi_adamw.ZeroRangeStep(ob, 3)
    for step in range(3):
        set_grads(a, step, 3e-2)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad)
        if step == 1:
            with torch.no_grad():
                for ps, opt in ((a, oa), (b, ob)):
                    ps[3].data = ps[3].data.clone() * 0.5
                    opt.state[ps[7]]["exp_avg"] = opt.state[ps[7]]["exp_avg"].clone() * 0.25
        oa.step()
        zs.step()
    torch.cuda.synchronize()
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        assert torch.equal(getattr(oa._flat, key), getattr(ob._flat, key)), key
    for ps, opt in ((a, oa), (b, ob)):
        assert opt._flat.is_param_view(ps[3])
        assert opt.state[ps[7]]["exp_avg"].data_ptr() == (opt._flat.exp_avg.data_ptr()
                                                          + 4 * opt._flat.offsets[id(ps[7])])
    assert torch.equal(a[3], b[3])
    # step 0 made the plan, step 1 saw the replaced tensors and took the Python begin()
    assert zs.native_begins == 1


def test_range_step_native_begin_changes(dev):
    """Between range steps: a learning-rate change (read from the group each step, natively),
    a checkpoint loaded into the optimizer and a moved gradient.  The results stay the
    unsharded flat step's; a gradient that is no longer the buffer's view is refused as
    before, with the step counts unchanged."""
    import copy
    import mi_adamw
    a, b, oa, ob = _flat_pair(dev, SHAPES, torch.float32, 2, 1.0)
    zs = mi_adamw.ZeroRangeStep(ob, 4)
    log = []
    for step in range(6):
        set_grads(a, step, 3e-2)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad)
        if step == 2:
            for opt in (oa, ob):
                opt.param_groups[1]["lr"] = 7e-4
        if step == 4:
            sd = copy.deepcopy(oa.state_dict())
            ob.load_state_dict(sd)
        before = zs.native_begins
        oa.step()
        zs.step()
        log.append(zs.native_begins - before)
    torch.cuda.synchronize()
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        assert torch.equal(getattr(oa._flat, key), getattr(ob._flat, key)), key
    # native from the second step; the checkpoint load replaces the state dicts
    assert log == [0, 1, 1, 1, 0, 1], log
    counts = [float(ob.state[q]["step"]) for q in b]
    b[2].grad = b[2].grad.clone()
    with pytest.raises(RuntimeError, match="gradient view"):
        zs.begin()
    assert [float(ob.state[q]["step"]) for q in b] == counts


def test_range_step_rejects_bad_arguments(dev):
    """Ranks out of range and device buffers of the wrong type are refused on the host,
    before any launch (the kernels would read 8-byte sums from a 4-byte buffer)."""
    import mi_adamw
    _, b, _, ob = _flat_pair(dev, SHAPES, torch.float32, 1, 1.0)
    zs = mi_adamw.ZeroRangeStep(ob, 2)
    set_grads(b, 0, 3e-2)
    for bad in (-1, 2):
        with pytest.raises(ValueError):
            zs.grad_sumsq(bad)
        with pytest.raises(ValueError):
            zs.segments(bad)
    for bad in (torch.zeros(1, dtype=torch.float32, device=dev),
                torch.zeros(0, dtype=torch.float64, device=dev),
                torch.zeros(1, dtype=torch.float64),
                torch.zeros(4, dtype=torch.float64, device=dev)[::2]):
        with pytest.raises(ValueError):
            zs.grad_sumsq(0, bad)
        with pytest.raises(ValueError):
            zs.finalize(bad)
    hypers = zs.begin()
    with pytest.raises(ValueError):
        zs.update(0, hypers, torch.ones(1, dtype=torch.float64, device=dev))
    with pytest.raises(ValueError):
        zs.update(5, hypers, None)
    torch.cuda.synchronize()

def _fill_6p7b(params, opt, step: float) -> None:
    """Seeded parameters, gradients and moments (per-tensor seeds) in the flat buffers."""
    from mi_adamw.workloads import GPT_6P7B, init_kind
    names = [n for n, _ in GPT_6P7B.tensors()]
    with torch.no_grad():
        for i, p in enumerate(params):
            kind = init_kind(names[i])
            if kind == "ones":
                p.fill_(1.0)
            elif kind == "zeros":
                p.zero_()
            else:
                p.copy_(torch.randn(p.shape, device=p.device, generator=gen(p.device, 1000 + i)))
                p.mul_(0.02)
            m = torch.randn(p.shape, device=p.device, generator=gen(p.device, 2000 + i)).mul_(1e-3)
            v = torch.randn(p.shape, device=p.device, generator=gen(p.device, 3000 + i))
            opt.set_state(p, step, m, v.mul_(1e-6).abs_())
            del m, v
    set_grads(params, 0, 1e-3)
    opt.refresh_bf16_copies()


def test_range_step_6p7b_equals_flat_step(dev):
    import mi_adamw
    from mi_adamw.workloads import GPT_6P7B
    params = gpt_params(GPT_6P7B, dev)
    prescale = mi_adamw.dp_prescale(8)
    opt = mi_adamw.FusedAdamW(params, **HP, max_grad_norm=1.0, bf16_copy=True, flat_buffer=True,
                              grad_prescale=prescale)
    flat = opt._flat
    _fill_6p7b(params, opt, 1000.0)
    opt.step()
    torch.cuda.synchronize()
    ref_norm = opt.last_grad_norm.clone()
    ref = {k: getattr(flat, k).clone() for k in ("param", "exp_avg", "exp_avg_sq", "copy")}
    print(f"6.7B unsharded flat step: norm {float(ref_norm):.9g}", flush=True)
    for world in (2, 4, 8):
        _fill_6p7b(params, opt, 1000.0)
        zs = mi_adamw.ZeroRangeStep(opt, world, grad_prescale=prescale)
        norm = zs.step()
        torch.cuda.synchronize()
        same_norm = torch.equal(norm.view(torch.int32), ref_norm.view(torch.int32))
        diff = {}
        for k, t in ref.items():
            cur = getattr(flat, k)
            n_diff = 0
            for lo in range(0, cur.numel(), 1 << 30):
                n_diff += int((cur[lo:lo + (1 << 30)].view(torch.int16 if cur.dtype ==
                               torch.bfloat16 else torch.int32)
                               != t[lo:lo + (1 << 30)].view(torch.int16 if t.dtype ==
                               torch.bfloat16 else torch.int32)).sum())
            diff[k] = n_diff
        print(f"6.7B {world} ranks {[hi - lo for lo, hi in zs.bounds][:2]}...: norm "
              f"{float(norm):.9g} (same bits: {same_norm}), differing elements {diff}",
              flush=True)
        assert same_norm
        assert all(v == 0 for v in diff.values())
        assert all(float(opt.state[p]["step"]) == 1001.0 for p in params)


def test_bench_range_shard_rows_step_as_the_flat_step(dev):
    """bench.py's range_shard row steps the flat buffers as `world` ranks: after its steps
    the buffers equal an unsharded flat optimizer's after as many steps, bit for bit."""
    import importlib.util
    import os
    import mi_adamw
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    world = 4
    a, b, oa, ob = _flat_pair(dev, SHAPES, torch.float32, 2, mi_adamw.dp_prescale(world))
    set_grads(a, 0, 3e-2)
    for p, q in zip(a, b):
        q.grad.copy_(p.grad)
    rs = bench.range_shard_rows(ob, world, steps=2, warmup=1)
    for _ in range(3):
        oa.step()
    torch.cuda.synchronize()
    lo, hi = mi_adamw.shard_bounds(ob._flat.total, world)[0]
    assert rs["world"] == world and rs["slice_params"] == hi - lo
    assert rs["rank_ms_mean"] > 0 and rs["update_gbs_mean"] > 0
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        assert torch.equal(getattr(oa._flat, key), getattr(ob._flat, key)), key
    assert all(float(oa.state[p]["step"]) == float(ob.state[q]["step"]) == 1003.0
               for p, q in zip(a, b))


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_range_step_after_placement(dev, state_dtype):
    """The range step over buffers that place_buffers (min_gain 0, so it moves whenever a
    candidate is any faster) and a forced move of the parameter and copy buffers put
    elsewhere between steps: it reads the buffers where they are now, stays bit-identical
    to the unplaced flat step, and its native begin() resumes after each move."""
    import mi_adamw
    from mi_adamw import placement
    a, b, oa, ob = _flat_pair(dev, SHAPES, state_dtype, 2, 1.0)
    zs = mi_adamw.ZeroRangeStep(ob, 3)
    moved = []
    for step in range(6):
        set_grads(a, step, 3e-2)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad)
        if step == 2:
            rep = ob.place_buffers(trials=2, launches=1, rounds=1, min_gain=0.0)
            moved.append((rep["chosen"], [s["chosen"] for s in rep["per_stream"]]))
        if step == 4:
            streams = placement._FlatStreams(ob, dev)
            before = ob._flat.param.data_ptr()
            streams.adopt(streams.allocate(["param", "copy"]))
            assert ob._flat.param.data_ptr() != before
            assert all(ob._flat.is_param_view(q) for q in b)
        oa.step()
        zs.step()
    torch.cuda.synchronize()
    for key in ("param", "exp_avg", "exp_avg_sq", "copy"):
        assert torch.equal(getattr(oa._flat, key), getattr(ob._flat, key)), key
    assert torch.equal(oa.last_grad_norm.view(torch.int32), ob.last_grad_norm.view(torch.int32))
    for p, q in zip(a, b):
        assert torch.equal(p, q)
    # begin() natively at steps 1, 3 and 5; the Python body at 0 and after each move
    assert zs.native_begins == 3, moved
