"""FusedAdamW.place_buffers on the GPU: moving the written streams changes no result.

place_buffers times the update's memory-only twin on the optimizer's current streams and
on newly allocated sets, and moves the values into the fastest set.  Which set wins
depends on the box, so the move itself is also forced through the layout's stream
classes.  Either way, the steps that follow must be bit-identical to those of the same
optimizer left where it was (parameters, moments, bf16 copy, clip norm), the native host
path must take the steps after the move, and a checkpoint must still interchange with
torch.optim.AdamW.
"""
from __future__ import annotations

import gc
import io

import pytest
import torch

from _helpers import clone_params, load_states, make_params, midtrain_state, set_grads

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


def _pair(dev, state_dtype, flat, copy=True):
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=copy, state_dtype=state_dtype,
              flat_buffer=flat)
    oa, ob = mi_adamw.FusedAdamW(a, **kw), mi_adamw.FusedAdamW(b, **kw)
    states = midtrain_state(a, 1000.0)
    load_states(oa, a, states)
    load_states(ob, b, states)
    return a, b, oa, ob


def _bits(t):
    t = t.detach()
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def _assert_same(a, b, oa, ob):
    for p, q in zip(a, b):
        assert torch.equal(_bits(p), _bits(q))
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(_bits(oa.state[p][key]), _bits(ob.state[q][key])), key
        if oa.bf16_copy:
            assert torch.equal(_bits(oa.bf16_param(p)), _bits(ob.bf16_param(q)))
    assert torch.equal(_bits(oa.last_grad_norm), _bits(ob.last_grad_norm))


def _steps(a, b, oa, ob, first, n):
    for k in range(first, first + n):
        set_grads(a, k, 3e-2)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad) if q.grad is not None else setattr(q, "grad", p.grad.clone())
        oa.step()
        ob.step()
    torch.cuda.synchronize()


@pytest.mark.parametrize("flat", [False, True])
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_forced_move_changes_no_result(dev, flat, state_dtype):
    from mi_adamw import placement
    a, b, oa, ob = _pair(dev, state_dtype, flat)
    _steps(a, b, oa, ob, 0, 2)
    streams = (placement._FlatStreams(oa, dev) if flat else placement._TableStreams(oa, dev))
    def ptrs():
        # an empty tensor reports data_ptr() 0 wherever it lives: only non-empty ones count
        return {n: [t.data_ptr() for t in (v if isinstance(v, list) else [v]) if t.numel()]
                for n, v in streams.current().items()}
    before = ptrs()
    cand = streams.allocate()
    streams.adopt(cand)
    oa._launch_cache = None
    oa._fast = None
    after = ptrs()
    assert all(x != y for n in before for x, y in zip(before[n], after[n])), "nothing moved"
    if flat:
        assert all(oa._flat.is_param_view(p) for p in a if p.numel())
        assert oa._flat.param.data_ptr() == cand["param"].data_ptr()
    else:
        # every state entry and copy is a view of its stream's block, in order
        blk = oa.state[a[0]]["exp_avg"].untyped_storage().data_ptr()
        assert all(oa.state[p]["exp_avg"].untyped_storage().data_ptr() == blk for p in a)
    _assert_same(a, b, oa, ob)                     # the move itself changes no value
    native = oa.native_steps
    _steps(a, b, oa, ob, 2, 4)
    _assert_same(a, b, oa, ob)
    assert oa.native_steps >= native + 2           # rebuilt once, then native again


@pytest.mark.parametrize("flat", [False, True])
def test_place_buffers_report_and_parity(dev, flat):
    a, b, oa, ob = _pair(dev, torch.bfloat16, flat)
    _steps(a, b, oa, ob, 0, 1)
    rep = oa.place_buffers(trials=3)
    print(f"place_buffers ({'flat' if flat else 'tables'}): {rep}", flush=True)
    assert rep["layout"] == ("flat" if flat else "tables")
    assert rep["candidates"] == 4 and len(rep["twin_ms"]) == 4
    tw = rep["twin_ms"]
    assert tw[rep["fastest"]] == min(tw) and rep["min_gain"] == 0.01
    # the fastest set is taken only if it beats the current one by min_gain
    if tw[0] / tw[rep["fastest"]] - 1 >= 0.01:
        assert rep["chosen"] == rep["fastest"]
    else:
        assert rep["chosen"] == 0 and rep["twin_gain"] == 0
    names = ["param", "exp_avg", "exp_avg_sq", "copy"] if flat else ["exp_avg", "exp_avg_sq",
                                                                     "copy"]
    assert rep["streams"] == names
    assert rep["transient_bytes"] == 3 * rep["set_bytes"]
    # then each stream alone: 3 new allocations of it beside the current one, the same
    # rule, in sweeps over the streams; another sweep follows only one that moved a stream
    sweeps = rep["sweeps"]
    assert 1 <= sweeps <= 3
    by_sweep = [[st for st in rep["per_stream"] if st["sweep"] == k] for k in range(1, sweeps + 1)]
    assert sum(map(len, by_sweep)) == len(rep["per_stream"])
    for k, sw in enumerate(by_sweep, 1):
        assert [st["stream"] for st in sw] == names
        moved = any(st["chosen"] != 0 for st in sw)
        assert moved == (k < sweeps) or (moved and k == sweeps == 3)
    for st in rep["per_stream"]:
        t = st["twin_ms"]
        assert st["candidates"] == 4 and t[st["fastest"]] == min(t)
        assert st["chosen"] in (0, st["fastest"])
        assert (st["chosen"] != 0) == (t[0] / t[st["fastest"]] - 1 >= 0.01)
    assert rep["peak_transient_bytes"] >= rep["transient_bytes"]
    _assert_same(a, b, oa, ob)
    _steps(a, b, oa, ob, 1, 3)
    _assert_same(a, b, oa, ob)


def test_checkpoint_after_a_move_interchanges_with_torch(dev):
    """Tables, fp32 state: after a forced move the state entries are views of the blocks;
    a state_dict taken then loads into torch.optim.AdamW and both step alike."""
    import mi_adamw
    from mi_adamw import placement
    ref = make_params(SHAPES, dev)
    ours = clone_params(ref)
    oopt = mi_adamw.FusedAdamW(ours, **HP)
    states = midtrain_state(ref, 1000.0)
    load_states(oopt, ours, states)
    set_grads(ours, 0, 3e-2)
    oopt.step()
    streams = placement._TableStreams(oopt, dev)
    streams.adopt(streams.allocate())
    oopt._launch_cache = None
    oopt._fast = None
    with torch.no_grad():
        for p, q in zip(ref, ours):
            p.copy_(q)
    topt = torch.optim.AdamW(ref, foreach=False, **HP)
    buf = io.BytesIO()
    torch.save(oopt.state_dict(), buf)
    buf.seek(0)
    topt.load_state_dict(torch.load(buf, weights_only=True))
    for k in range(1, 4):
        set_grads(ref, k, 3e-2)
        set_grads(ours, k, 3e-2)
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    for p, q in zip(ref, ours):
        assert torch.equal(_bits(p), _bits(q))
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(_bits(topt.state[p][key]), _bits(oopt.state[q][key]))


def test_place_buffers_refusals(dev):
    import mi_adamw
    ps = make_params(SHAPES[:3], dev)
    with pytest.raises(RuntimeError, match="no parameter has optimizer state"):
        mi_adamw.FusedAdamW(ps, **HP).place_buffers(trials=1)
    with pytest.raises(NotImplementedError, match="amsgrad"):
        mi_adamw.FusedAdamW(ps, **HP, amsgrad=True).place_buffers(trials=1)
    opt = mi_adamw.FusedAdamW(ps, **HP)
    set_grads(ps, 0, 1e-2)
    opt.step()
    for p in ps:
        p.grad = None
    with pytest.raises(RuntimeError, match="gradient"):
        opt.place_buffers(trials=1)
    # no memory for a candidate: only the current set is timed, nothing moves
    set_grads(ps, 1, 1e-2)
    rep = opt.place_buffers(trials=4, reserve_bytes=1 << 50)
    assert rep["candidates"] == 1 and rep["chosen"] == 0 and rep["transient_bytes"] == 0
    # min_gain 0 takes the fastest of the candidates, whatever the margin
    rep = opt.place_buffers(trials=2, min_gain=0.0)
    assert rep["chosen"] == rep["fastest"]


@pytest.mark.parametrize("flat", [False, True])
def test_place_trials_option_places_once_after_the_first_step(dev, flat):
    """FusedAdamW(place_trials=K) runs place_buffers(K) once, after the first step (the
    one that creates every parameter's state): results equal an optimizer without it."""
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=True, state_dtype=torch.bfloat16,
              flat_buffer=flat)
    oa = mi_adamw.FusedAdamW(a, **kw, place_trials=2)
    ob = mi_adamw.FusedAdamW(b, **kw)
    assert oa.placement is None
    _steps(a, b, oa, ob, 0, 1)
    rep = oa.placement
    assert rep is not None and rep["candidates"] == 3
    assert rep["layout"] == ("flat" if flat else "tables")
    _steps(a, b, oa, ob, 1, 3)
    assert oa.placement is rep                     # once only
    _assert_same(a, b, oa, ob)


def test_placement_with_groups_and_a_parameter_without_gradient(dev):
    """Two param groups with their own hyperparameters; one parameter has no gradient at the
    first step, so place_trials places the others and that one's state, created when its
    gradient arrives, keeps its own allocation.  Every step equals an unplaced optimizer's."""
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)

    def groups(ps):
        return [{"params": ps[:5]}, {"params": ps[5:], "lr": 1e-3, "weight_decay": 0.0,
                                     "betas": (0.8, 0.99)}]
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=True, state_dtype=torch.bfloat16)
    oa = mi_adamw.FusedAdamW(groups(a), **kw, place_trials=3)
    ob = mi_adamw.FusedAdamW(groups(b), **kw)
    late = 3
    for k in range(4):
        set_grads(a, k, 3e-2)
        if k == 0:
            a[late].grad = None
        for p, q in zip(a, b):
            q.grad = None if p.grad is None else p.grad.clone()
        oa.step()
        ob.step()
        if k == 0:
            rep = oa.placement
            assert rep is not None and rep["candidates"] == 4
            assert "exp_avg" not in oa.state[a[late]]
    torch.cuda.synchronize()
    assert oa.placement is rep
    for p, q in zip(a, b):
        assert torch.equal(_bits(p), _bits(q))
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(_bits(oa.state[p][key]), _bits(ob.state[q][key])), key
        assert torch.equal(_bits(oa.bf16_param(p)), _bits(ob.bf16_param(q)))
    assert float(oa.state[a[late]]["step"]) == 3.0 and float(oa.state[a[0]]["step"]) == 4.0


def test_capturable_placed_before_capture_replays_bit_identically(dev):
    """capturable=True with place_trials: the first (eager) step places the streams; a step
    recorded into a HIP graph afterwards, replayed with new gradients in the same tensors,
    is bit-identical to an unplaced capturable optimizer's eager steps.  place_buffers after
    the capture raises: the graph keeps the addresses it recorded."""
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    kw = dict(**HP, max_grad_norm=1.0, bf16_copy=True, capturable=True)
    oa = mi_adamw.FusedAdamW(a, **kw, place_trials=2)
    ob = mi_adamw.FusedAdamW(b, **kw)
    for p in a + b:
        p.grad = torch.zeros_like(p)

    def fill(k):
        set_grads(a, k, 3e-2)
        for p, q in zip(a, b):
            q.grad.copy_(p.grad)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(3):
            fill(k)
            oa.step()
            ob.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert oa.placement is not None and oa.placement["candidates"] == 3
    _assert_same(a, b, oa, ob)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        oa.step()
    assert oa.captured
    for k in range(3, 7):
        fill(k)
        graph.replay()
        ob.step()
        torch.cuda.synchronize()
        _assert_same(a, b, oa, ob)
        torch.randn(1 << 20, device=dev).sum().item()     # other eager work between replays
    assert float(oa.state[a[0]]["step"]) == 7.0
    with pytest.raises(RuntimeError, match="recorded into a graph"):
        oa.place_buffers(trials=1)


def test_twin_leaves_out_rows_that_are_not_dense(dev):
    """A state entry put into the dict as a strided view (not dense, more storage than its
    elements) is left out of the twin's rows, so the twin never touches memory beyond the
    tensors; the next step converts it and every step equals an unplaced optimizer's."""
    import mi_adamw
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    oa = mi_adamw.FusedAdamW(a, **HP, max_grad_norm=1.0)
    ob = mi_adamw.FusedAdamW(b, **HP, max_grad_norm=1.0)
    _steps(a, b, oa, ob, 0, 1)
    j = 7                                   # the (70001,) parameter
    guard = torch.full((2 * a[j].numel(),), 7.0, device=dev)
    strided = guard[::2]
    strided.copy_(oa.state[a[j]]["exp_avg"])
    oa.state[a[j]]["exp_avg"] = strided
    from mi_adamw import placement
    streams = placement._TableStreams(oa, dev)
    launch = streams._launch(streams.current())
    dense = sum(1 for p in a if p.numel())
    assert launch.n_rows == dense - 1                # the strided entry's row is left out
    assert int(launch.host_rows["numel"].sum()) == sum(p.numel() for p in a) - a[j].numel()
    before = guard[1::2].clone()
    rep = oa.place_buffers(trials=2)
    assert rep["candidates"] == 3
    torch.cuda.synchronize()
    assert torch.equal(guard[1::2], before)          # the gaps were never written
    _steps(a, b, oa, ob, 1, 2)
    _assert_same(a, b, oa, ob)


def test_twin_leaves_out_host_and_narrower_state(dev):
    """A state entry in host memory, and one of a narrower type than the state dtype, are
    left out of the twin's rows for every candidate (the twin would read host memory, or
    past the narrower tensor's end); the move converts them as the step would, and every
    step equals that of an unplaced optimizer given the same entries."""
    import mi_adamw
    from mi_adamw import placement
    a = make_params(SHAPES, dev)
    b = clone_params(a)
    oa = mi_adamw.FusedAdamW(a, **HP, max_grad_norm=1.0, bf16_copy=True)
    ob = mi_adamw.FusedAdamW(b, **HP, max_grad_norm=1.0, bf16_copy=True)
    _steps(a, b, oa, ob, 0, 1)
    for o, ps in ((oa, a), (ob, b)):
        o.state[ps[7]]["exp_avg"] = o.state[ps[7]]["exp_avg"].cpu()           # (70001,)
        o.state[ps[3]]["exp_avg_sq"] = o.state[ps[3]]["exp_avg_sq"].bfloat16()  # (144, 48)
    streams = placement._TableStreams(oa, dev)
    for cand in (streams.current(), streams.allocate()):
        launch = streams._launch(cand)
        assert launch.n_rows == sum(1 for p in a if p.numel()) - 2
        assert int(launch.host_rows["numel"].sum()) == (sum(p.numel() for p in a)
                                                        - a[7].numel() - a[3].numel())
    oa.place_buffers(trials=2, min_gain=0.0)
    _steps(a, b, oa, ob, 1, 2)
    _assert_same(a, b, oa, ob)
    assert oa.state[a[7]]["exp_avg"].device == dev
    assert oa.state[a[3]]["exp_avg_sq"].dtype == torch.float32
