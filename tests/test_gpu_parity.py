"""GPU parity: FusedAdamW / the C ABI against torch.optim.AdamW(foreach=False) and the oracle.

Tolerances (fp32): parameters and moments within 2 ulp of torch after one
step; relative error 1e-5 after chained steps; clip norm relative 1e-6.  The
kernels follow torch-ROCm's op chain, so the observed distance is 0 ulp and
the tests also assert bit-equality with the oracle's ROCm op model.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import (clone_params, close_rel, gen, load_states, make_params, max_ulp,
                      max_ulp_all, midtrain_state, rel_err, rms, set_grads, to_np)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

# A miniature of the GPT layout: LayerNorm vectors, ragged matrices, sizes that
# are not multiples of 4 (scalar tail) or of the chunk size (partial chunks).
MINI_SHAPES = [(64, 48), (48,), (48,), (144, 48), (48, 48), (4099,), (3,), (1,), (7, 5),
               (70001,), (1024,), (65536 + 12,)]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    import mi_adamw
    print("mi_adamw", mi_adamw.version(), flush=True)
    return torch.device("cuda", 0)


def _pair(dev, shapes=MINI_SHAPES, **kw):
    import mi_adamw
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    hp = dict(lr=kw.pop("lr", 3e-4), betas=kw.pop("betas", (0.9, 0.95)), eps=kw.pop("eps", 1e-8),
              weight_decay=kw.pop("weight_decay", 0.1), maximize=kw.pop("maximize", False))
    topt = torch.optim.AdamW(ref, foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(ours, **hp, **kw)
    return ref, ours, topt, oopt


def _assert_same(ref, ours, topt, oopt, max_allowed=0):
    du = max_ulp_all([p for p in ref], [p for p in ours])
    dm = max_ulp_all([topt.state[p]["exp_avg"] for p in ref], [oopt.state[p]["exp_avg"] for p in ours])
    dv = max_ulp_all([topt.state[p]["exp_avg_sq"] for p in ref],
                     [oopt.state[p]["exp_avg_sq"] for p in ours])
    print(f"ulp p={du} m={dm} v={dv}", flush=True)
    assert du <= max_allowed and dm <= max_allowed and dv <= max_allowed
    for p, q in zip(ref, ours):
        assert float(topt.state[p]["step"]) == float(oopt.state[q]["step"])


@pytest.mark.parametrize("betas,lr,wd,maximize", [
    ((0.9, 0.95), 3e-4, 0.1, False),     # the benchmark workloads' hyperparameters
    ((0.9, 0.999), 6e-4, 0.1, False),    # mini-megatron's defaults (config.py:11,13)
    ((0.9, 0.999), 6e-4, 0.0, False),    # no weight decay: first op is skipped
    ((0.3, 0.95), 1e-3, 0.01, False),    # lerp weight 0.7: the other Lerp.h branch
    ((0.9, 0.95), 3e-4, 0.1, True),      # maximize
    ((0.9, 0.95), 0.0, 0.1, False),      # lr = 0, the reference's first step (main.py:39-40)
    ((0.0, 0.0), 1e-3, 0.1, False),      # lerp weight 1 and beta2 0: bias corrections exactly 1
    ((0.0, 0.999), 1e-3, 0.0, True),
])
def test_chained_steps_match_torch_bitwise(dev, betas, lr, wd, maximize):
    """Steps 1..10 from zero state: bias corrections change every step."""
    ref, ours, topt, oopt = _pair(dev, betas=betas, lr=lr, weight_decay=wd, maximize=maximize)
    for step in range(1, 11):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        oopt.step()
        torch.cuda.synchronize()
        print(f"step {step}", flush=True)
        _assert_same(ref, ours, topt, oopt, max_allowed=0)


def test_eps_zero_matches_torch_including_its_nans(dev):
    """eps = 0: where v is 0 the denominator is 0 and torch produces inf/NaN; so must we."""
    ref, ours, topt, oopt = _pair(dev, eps=0.0)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        for p in ref:
            p.grad.view(-1)[::7] = 0.0          # v stays 0 there on the first step
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    assert any(bool(torch.isnan(p).any()) for p in ref)
    _assert_same(ref, ours, topt, oopt, max_allowed=0)


def test_kernel_matches_oracle_bitwise(dev):
    """The HIP update equals the oracle's ROCm op model, element for element."""
    import mi_adamw
    shapes = [(1,), (3,), (5,), (1023,), (1025,), (4096,), (65537,)]
    params = make_params(shapes, dev)
    init = [to_np(p).copy() for p in params]
    states = midtrain_state(params, step=7.0)
    opt = mi_adamw.FusedAdamW(params, lr=6e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    load_states(opt, params, states)
    set_grads(params, 8, 1e-3)
    grads = [to_np(p.grad).copy() for p in params]
    opt.step()
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        pn, mn, vn = init[i].copy(), to_np(states[i]["exp_avg"]).copy(), to_np(states[i]["exp_avg_sq"]).copy()
        O.adamw_step(pn, grads[i], mn, vn, lr=6e-4, betas=(0.9, 0.999), eps=1e-8,
                     weight_decay=0.1, step=8.0, opmodel=O.OPMODEL_TORCH_ROCM)
        assert O.max_ulp(pn.reshape(-1), to_np(p).reshape(-1))[0] == 0
        assert O.max_ulp(mn.reshape(-1), to_np(opt.state[p]["exp_avg"]).reshape(-1))[0] == 0
        assert O.max_ulp(vn.reshape(-1), to_np(opt.state[p]["exp_avg_sq"]).reshape(-1))[0] == 0


def test_torch_rocm_matches_oracle_opmodel(dev):
    """Pins the oracle's ROCm op model: torch's own GPU AdamW equals it bit for bit."""
    n = 1 << 20
    for betas, step in (((0.9, 0.95), 1), ((0.9, 0.999), 3), ((0.3, 0.95), 50), ((0.9, 0.95), 1000)):
        p = torch.nn.Parameter(torch.randn(n, device=dev, generator=gen(dev, 1)) * 0.02)
        st = midtrain_state([p], step=float(step - 1))[0]
        p.grad = torch.randn(n, device=dev, generator=gen(dev, 2)) * 1e-3
        pn, gn = to_np(p).copy(), to_np(p.grad).copy()
        mn, vn = to_np(st["exp_avg"]).copy(), to_np(st["exp_avg_sq"]).copy()
        opt = torch.optim.AdamW([p], lr=3e-4, betas=betas, eps=1e-8, weight_decay=0.1, foreach=False)
        load_states(opt, [p], [st])
        opt.step()
        O.adamw_step(pn, gn, mn, vn, lr=3e-4, betas=betas, eps=1e-8, weight_decay=0.1,
                     step=float(step), opmodel=O.OPMODEL_TORCH_ROCM)
        assert O.max_ulp(pn, to_np(p))[0] == 0, (betas, step)
        assert O.max_ulp(mn, to_np(opt.state[p]["exp_avg"]))[0] == 0, (betas, step)
        assert O.max_ulp(vn, to_np(opt.state[p]["exp_avg_sq"]))[0] == 0, (betas, step)


def test_clip_matches_torch(dev):
    """Fused clip + AdamW, 5 chained mid-training steps, against two torch references.

    A: torch.nn.utils.clip_grad_norm_ then AdamW(foreach=False) -- the norm may
       differ by an ulp (torch sums fp32 per-tensor norms; the kernel sums
       squares in float64), so p, m, v are compared elementwise with
       |d| <= 1e-6 (|ref| + rms(ref)).
    B: torch.nn.utils.clip_grads_with_norm_ with the kernel's norm, then AdamW --
       the same coefficient, so everything must be bit-identical.
    """
    import mi_adamw
    ref_a = make_params(MINI_SHAPES, dev)
    ref_b = clone_params(ref_a)
    ours = clone_params(ref_a)
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    ta = torch.optim.AdamW(ref_a, foreach=False, **hp)
    tb = torch.optim.AdamW(ref_b, foreach=False, **hp)
    oo = mi_adamw.FusedAdamW(ours, max_grad_norm=1.0, **hp)
    states = midtrain_state(ref_a, 1000.0)
    for opt, ps in ((ta, ref_a), (tb, ref_b), (oo, ours)):
        load_states(opt, ps, states)
    for step in range(5):
        set_grads(ref_a, step, 1e-2)
        for p, q, r in zip(ref_a, ref_b, ours):
            q.grad = p.grad.clone()
            r.grad = p.grad.clone()
        oo.step()
        on = oo.last_grad_norm
        tn = torch.nn.utils.clip_grad_norm_(ref_a, 1.0)
        ta.step()
        torch.nn.utils.clip_grads_with_norm_(ref_b, 1.0, on.clone())
        tb.step()
        torch.cuda.synchronize()
        exact = O.total_norm([to_np(p.grad) for p in ours])
        print(f"norm torch={tn.item():.9g} ours={on.item():.9g} float64={float(exact):.9g}",
              flush=True)
        assert rel_err(on, tn) <= 1e-6
        assert on.item() == float(exact)
        _assert_same(ref_b, ours, tb, oo, max_allowed=0)
        for p, q in zip(ref_a, ours):
            assert close_rel(q, p, 1e-6, 1e-6 * rms(p)) <= 1
            for k in ("exp_avg", "exp_avg_sq"):
                r = ta.state[p][k]
                assert close_rel(oo.state[q][k], r, 1e-6, 1e-6 * rms(r)) <= 1


def test_clip_grad_norm_dropin(dev):
    import mi_adamw
    ref = make_params(MINI_SHAPES, dev)
    set_grads(ref, 3, 1e-2)
    ours = clone_params(ref)
    tn = torch.nn.utils.clip_grad_norm_(ref, 1.0)
    on = mi_adamw.clip_grad_norm_(ours, 1.0)
    assert rel_err(on, tn) <= 1e-6
    exact = float(np.sqrt(sum(float((to_np(p.grad).astype(np.float64) ** 2).sum()) for p in ours)))
    print("norm", tn.item(), on.item(), exact, flush=True)
    assert max_ulp_all([p.grad for p in ref], [q.grad for q in ours]) <= 1


def test_clip_grad_norm_with_moving_gradients(dev):
    """clip_grad_norm_ in a training loop: new gradient tensors every call (their tables
    are refreshed, the chunk table kept), each result against torch's on the same grads."""
    import mi_adamw
    from mi_adamw import clip as C
    ref = make_params(MINI_SHAPES, dev)
    ours = clone_params(ref)
    held = []
    for step in range(1, 5):
        set_grads(ref, step, 1e-2)
        held.append([q.grad for q in ours if q.grad is not None])   # force new addresses
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        tn = torch.nn.utils.clip_grad_norm_(ref, 1.0)
        on = mi_adamw.clip_grad_norm_(ours, 1.0)
        assert rel_err(on, tn) <= 1e-6
        for p, q in zip(ref, ours):
            # each scaled by its own coefficient (the two norms may differ by an ulp)
            assert close_rel(q.grad, p.grad, 1e-6, 1e-12) <= 1.0
    keys = [k for k in C._cache if k[0] == dev]
    assert len(keys) == 1, "one chunk table for one set of sizes"


def test_clip_grad_norm_on_two_streams(dev):
    """Two clip_grad_norm_ calls on two streams with no ordering between them (their
    scratch is per stream): each norm and each scaled gradient as torch's alone."""
    import mi_adamw
    sets = []
    for k, shapes in enumerate((MINI_SHAPES, MINI_SHAPES[::-1])):
        ref = make_params(shapes, dev, seed=1000 + 100 * k)
        set_grads(ref, 7 + k, 1e-2 * (k + 1))
        sets.append((ref, clone_params(ref)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s_ in streams:
        s_.wait_stream(torch.cuda.current_stream())
    norms = []
    for (ref, ours), s_ in zip(sets, streams):
        with torch.cuda.stream(s_):
            norms.append(mi_adamw.clip_grad_norm_(ours, 1.0))
    torch.cuda.synchronize()
    for (ref, ours), on in zip(sets, norms):
        tn = torch.nn.utils.clip_grad_norm_(ref, 1.0)
        assert rel_err(on, tn) <= 1e-6
        for p, q in zip(ref, ours):
            assert close_rel(q.grad, p.grad, 1e-6, 1e-12) <= 1.0


def test_clip_grad_norm_same_sizes_on_two_streams(dev):
    """Gradient lists of the same sizes, clipped on two streams with no ordering between
    them, twice (the second round rewrites the rows): each stream has its own tables, so
    neither call reads or frees rows the other is using."""
    import mi_adamw
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rnd in range(2):
        sets = []
        for k in range(2):
            ref = make_params(MINI_SHAPES, dev, seed=1000 + 100 * k + 10 * rnd)
            set_grads(ref, 3 * rnd + k, 1e-2 * (k + 1))
            sets.append((ref, clone_params(ref)))
        for s_ in streams:
            s_.wait_stream(torch.cuda.current_stream())
        norms = []
        for (ref, ours), s_ in zip(sets, streams):
            with torch.cuda.stream(s_):
                norms.append(mi_adamw.clip_grad_norm_(ours, 1.0))
        torch.cuda.synchronize()
        for (ref, ours), on in zip(sets, norms):
            tn = torch.nn.utils.clip_grad_norm_(ref, 1.0)
            assert rel_err(on, tn) <= 1e-6
            for p, q in zip(ref, ours):
                assert close_rel(q.grad, p.grad, 1e-6, 1e-12) <= 1.0


def test_bf16_copy_and_state(dev):
    import mi_adamw
    params = make_params(MINI_SHAPES, dev)
    ref = clone_params(params)
    opt = mi_adamw.FusedAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                              state_dtype=torch.bfloat16, bf16_copy=True, max_grad_norm=1.0)
    states = midtrain_state(params, 1000.0)
    load_states(opt, params, states)
    for p in params:
        assert opt.state[p]["exp_avg"].dtype == torch.bfloat16
    set_grads(params, 0, 1e-3)
    grads = [to_np(p.grad).copy() for p in params]
    opt.step()
    torch.cuda.synchronize()
    coef = float(opt.last_grad_norm.item())
    coef = O.clip_coef(np.float32(coef), 1.0)
    for i, p in enumerate(params):
        pn = to_np(ref[i]).copy()
        mb = O.to_bf16_bits(to_np(states[i]["exp_avg"]))
        vb = O.to_bf16_bits(to_np(states[i]["exp_avg_sq"]))
        O.adamw_step_bf16state(pn.reshape(-1), grads[i].reshape(-1), mb.reshape(-1), vb.reshape(-1),
                               lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                               step=1001.0, grad_scale=coef)
        assert O.max_ulp(pn, to_np(p))[0] == 0
        got_m = to_np(opt.state[p]["exp_avg"].view(torch.int16)).view(np.uint16)
        got_v = to_np(opt.state[p]["exp_avg_sq"].view(torch.int16)).view(np.uint16)
        assert np.array_equal(got_m, mb) and np.array_equal(got_v, vb)
        copy = opt.bf16_param(p)
        assert torch.equal(copy, p.detach().to(torch.bfloat16))


def test_flat_buffer_matches_per_tensor(dev):
    """Flat-buffer mode (one contiguous range per group) against torch with the same norm.

    Flat mode keeps gradients allocated, which is torch's zero_grad(set_to_none=False).
    """
    import mi_adamw
    ref, ours, topt, oopt = _pair(dev, flat_buffer=True, max_grad_norm=1.0, bf16_copy=True)
    states = midtrain_state(ref, 1000.0)
    load_states(topt, ref, states)
    load_states(oopt, ours, states)
    for step in range(3):
        oopt.zero_grad()
        set_grads(ref, step, 1e-2)
        for p, q in zip(ref, ours):
            q.grad.copy_(p.grad)
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        exact = O.total_norm([to_np(p.grad) for p in ours])
        assert oopt.last_grad_norm.item() == float(exact)
        _assert_same(ref, ours, topt, oopt, max_allowed=0)
    for p in ours:
        assert torch.equal(oopt.bf16_param(p), p.detach().to(torch.bfloat16))
    assert oopt._copies == {}          # the copies live in the flat buffer only


def test_state_dict_roundtrip_with_torch(dev):
    """A FusedAdamW checkpoint loads into torch.optim.AdamW and back (checkpoint.py:9,19).

    Both optimizers are built as main.py:177 builds its AdamW, with fused=False:
    the saved param_groups carry that flag, which keeps torch on its
    per-tensor path after loading (with fused=foreach=None torch would pick its
    foreach path, whose rounding differs).
    """
    import mi_adamw
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=False)
    ref = make_params(MINI_SHAPES, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, **hp)
    oopt = mi_adamw.FusedAdamW(ours, **hp)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        topt.step()
        oopt.step()
    _assert_same(ref, ours, topt, oopt)
    sd = oopt.state_dict()
    # Independent step tensors, torch's keys and layout.
    steps = [st["step"] for st in sd["state"].values()]
    assert len({id(s) for s in steps}) == len(steps)
    assert all(s.device.type == "cpu" and s.dtype == torch.float32 for s in steps)
    assert set(sd["param_groups"][0]) == set(topt.state_dict()["param_groups"][0])
    assert set(sd["state"][0]) == set(topt.state_dict()["state"][0])
    t2 = torch.optim.AdamW(clone_params(ours), **hp)
    t2.load_state_dict(sd)
    o2 = mi_adamw.FusedAdamW(clone_params(ref), **hp)
    o2.load_state_dict(topt.state_dict())
    p_t2 = t2.param_groups[0]["params"]
    p_o2 = o2.param_groups[0]["params"]
    for step in range(4, 6):
        set_grads(p_t2, step, 1e-3)
        for p, q in zip(p_t2, p_o2):
            q.grad = p.grad.clone()
        t2.step()
        o2.step()
    torch.cuda.synchronize()
    _assert_same(p_t2, p_o2, t2, o2)
    for p, q in zip(p_t2, p_o2):
        assert float(t2.state[p]["step"]) == float(o2.state[q]["step"]) == 5.0


def test_params_without_grad_are_skipped(dev):
    ref, ours, topt, oopt = _pair(dev)
    set_grads(ref, 1, 1e-3)
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()
    for i in (1, 5):
        ref[i].grad = None
        ours[i].grad = None
    topt.step()
    oopt.step()
    torch.cuda.synchronize()
    assert len(oopt.state[ours[1]]) == 0
    _assert_same([p for i, p in enumerate(ref) if i not in (1, 5)],
                 [p for i, p in enumerate(ours) if i not in (1, 5)], topt, oopt)
    # A later step with every grad: the skipped params start at step 1.
    set_grads(ref, 2, 1e-3)
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()
    topt.step()
    oopt.step()
    torch.cuda.synchronize()
    _assert_same(ref, ours, topt, oopt)


def test_nonfinite_grads_propagate_like_torch(dev):
    ref, ours, topt, oopt = _pair(dev, max_grad_norm=1.0)
    set_grads(ref, 1, 1e-3)
    ref[3].grad[0, 0] = float("inf")
    ref[5].grad[7] = float("nan")
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()
    tn = torch.nn.utils.clip_grad_norm_(ref, 1.0)
    topt.step()
    oopt.step()
    torch.cuda.synchronize()
    assert torch.isnan(tn) == torch.isnan(oopt.last_grad_norm)
    for p, q in zip(ref, ours):
        assert torch.equal(torch.isnan(p), torch.isnan(q))


def test_misaligned_views_take_scalar_path(dev):
    """Params that are views at odd offsets (not 16-byte aligned) still match torch."""
    import mi_adamw
    base = torch.randn(10007, device=dev, generator=gen(dev, 5)) * 0.02
    ref_views = [torch.nn.Parameter(base[1:4001].clone()), torch.nn.Parameter(base[3:1030].clone())]
    store = torch.zeros(10007, device=dev)
    ours = []
    for off, p in ((1, ref_views[0]), (4003, ref_views[1])):
        v = store[off:off + p.numel()]
        v.copy_(p.detach())
        q = torch.nn.Parameter(v)
        ours.append(q)
    topt = torch.optim.AdamW(ref_views, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, foreach=False)
    oopt = mi_adamw.FusedAdamW(ours, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    for step in range(1, 4):
        set_grads(ref_views, step, 1e-3)
        gstore = torch.zeros(10007, device=dev)
        for (off, p), q in zip(((1, ref_views[0]), (4003, ref_views[1])), ours):
            gv = gstore[off:off + p.numel()]
            gv.copy_(p.grad)
            q.grad = gv
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    assert ours[0].data_ptr() % 16 != 0
    _assert_same(ref_views, ours, topt, oopt)


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_chunk_size_and_grid_shape_do_not_change_results(dev, state_dtype):
    """The update is elementwise: chunk size (one 4096-element tile per workgroup, or
    pipelined multi-tile chunks) and grid shape (one chunk per workgroup, or a capped
    grid striding over chunks) must give the same bits.  The clip norm's float64
    partial sums do depend on the chunk assignment; its fp32 result is compared to
    1 ulp, with max_norm so large that the coefficient is exactly 1."""
    import mi_adamw
    results, norms = [], []
    for chunk, max_blocks in ((4096, 0), (8192, 0), (65536, 0), (1 << 20, 0), (4096, 64),
                              (65536, 7)):
        params = make_params(MINI_SHAPES, dev)
        # max_grad_norm 1e9: the norm pass runs under this chunking, the coefficient is 1
        opt = mi_adamw.FusedAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                                  chunk_elems=chunk, state_dtype=state_dtype, bf16_copy=True,
                                  max_grad_norm=1e9)
        opt.max_blocks = max_blocks
        load_states(opt, params, midtrain_state(params, 10.0))
        for step in (1, 2):
            set_grads(params, step, 1e-3)
            opt.step()
        copies = [c.clone() for c in opt.bf16_params()]
        normed = opt.last_grad_norm
        torch.cuda.synchronize()
        results.append(([p.detach().clone() for p in params],
                        [opt.state[p]["exp_avg"].clone() for p in params],
                        [opt.state[p]["exp_avg_sq"].clone() for p in params], copies))
        norms.append(normed.clone())
        print(f"chunk {chunk} max_blocks {max_blocks} done", flush=True)
    base = results[0]
    for other in results[1:]:
        for xs, ys in zip(base, other):
            for x, y in zip(xs, ys):
                assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x.view(torch.int32),
                                   y.view(torch.int16) if y.dtype == torch.bfloat16 else y.view(torch.int32))
    for n in norms[1:]:
        assert max_ulp(n, norms[0]) <= 1


def test_chunk_size_changed_between_steps(dev):
    """chunk_elems and max_blocks changed on a live optimizer between steps: the chunk
    tables are cut again at the new size (a table cut at the old size would step some
    elements twice), and every step equals an untouched optimizer's.  The norm pass runs
    under each chunking, with max_norm so large that the coefficient is exactly 1 (the
    float64 partial sums, and so the last bit of the norm, depend on the chunking)."""
    import mi_adamw
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=1e9)
    a = make_params(MINI_SHAPES, dev)
    b = clone_params(a)
    oa = mi_adamw.FusedAdamW(a, **hp)
    ob = mi_adamw.FusedAdamW(b, **hp)
    for step, (chunk, blocks) in enumerate(((4096, 0), (65536, 0), (8192, 7), (4096, 0))):
        oa.chunk_elems, oa.max_blocks = chunk, blocks
        set_grads(a, step, 1e-2)
        for p, q in zip(a, b):
            q.grad = p.grad.clone()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for p, q in zip(a, b):
            assert max_ulp(p, q) == 0, (step, chunk)
            for k in ("exp_avg", "exp_avg_sq"):
                assert max_ulp(oa.state[p][k], ob.state[q][k]) == 0, (step, k)


def test_clip_step_is_deterministic(dev):
    """Two runs on the same inputs give the same bits, norm included (fixed reduction order)."""
    import mi_adamw
    runs = []
    for _ in range(2):
        params = make_params(MINI_SHAPES, dev)
        opt = mi_adamw.FusedAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                                  max_grad_norm=1.0)
        load_states(opt, params, midtrain_state(params, 1000.0))
        norms = []
        for step in range(3):
            set_grads(params, step, 1e-2)
            opt.step()
            norms.append(opt.last_grad_norm.clone())
        torch.cuda.synchronize()
        runs.append(([p.detach().clone() for p in params], norms))
    for a, b in zip(runs[0][0], runs[1][0]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_step_on_a_side_stream(dev):
    """step() enqueues on the current stream, tables and clip included: a side stream
    gives the same bits as the default one (ordering against the grads' producer is the
    caller's, as for any torch op)."""
    import mi_adamw
    runs = []
    for use_side in (False, True):
        params = make_params(MINI_SHAPES, dev)
        opt = mi_adamw.FusedAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                                  max_grad_norm=1.0, bf16_copy=True)
        load_states(opt, params, midtrain_state(params, 100.0))
        side = torch.cuda.Stream(device=dev)
        for step in range(3):
            set_grads(params, step, 1e-2)
            if use_side:
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    opt.step()
                    norm = opt.last_grad_norm.clone()
                torch.cuda.current_stream(dev).wait_stream(side)
            else:
                opt.step()
                norm = opt.last_grad_norm.clone()
        torch.cuda.synchronize()
        runs.append(([p.detach().clone() for p in params], [c.clone() for c in opt.bf16_params()],
                     norm))
    for a, b in zip(runs[0][0], runs[1][0]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(runs[0][2], runs[1][2])


def test_special_values_match_torch(dev):
    """Denormals, signed zeros, tiny and huge magnitudes, inf and NaN in p, g, m and v:
    the kernel keeps fp32 denormals and follows torch's per-op chain through all of them."""
    import mi_adamw
    specials = torch.tensor([0.0, -0.0, 1e-45, -1e-45, 1e-40, -3e-39, 1.17e-38, 1e-30, -1e-20,
                             1e-8, 1.0, -1.0, 3e4, -1e15, 1e30, 3.4e38, float("inf"),
                             float("-inf"), float("nan")], dtype=torch.float32)
    k = specials.numel()
    # every combination of a special p, g, m and |v| (v >= 0 as in real state)
    idx = torch.cartesian_prod(*(torch.arange(k) for _ in range(4)))
    pv, gv, mv, vv = (specials[idx[:, j]] for j in range(4))
    vv = vv.abs()
    n = idx.shape[0]
    for betas, step, maximize in (((0.9, 0.95), 1.0, False), ((0.3, 0.999), 7.0, True)):
        ref = [torch.nn.Parameter(pv.clone().to(dev))]
        ours = [torch.nn.Parameter(pv.clone().to(dev))]
        ref[0].grad = gv.clone().to(dev)
        ours[0].grad = gv.clone().to(dev)
        hp = dict(lr=1e-3, betas=betas, eps=1e-8, weight_decay=0.1, maximize=maximize)
        topt = torch.optim.AdamW(ref, foreach=False, **hp)
        oopt = mi_adamw.FusedAdamW(ours, **hp)
        st = [{"step": torch.tensor(step - 1), "exp_avg": mv.clone().to(dev),
               "exp_avg_sq": vv.clone().to(dev)}]
        load_states(topt, ref, st)
        load_states(oopt, ours, st)
        topt.step()
        oopt.step()
        torch.cuda.synchronize()
        for a, b, what in ((ref[0], ours[0], "p"),
                           (topt.state[ref[0]]["exp_avg"], oopt.state[ours[0]]["exp_avg"], "m"),
                           (topt.state[ref[0]]["exp_avg_sq"], oopt.state[ours[0]]["exp_avg_sq"], "v")):
            a, b = a.detach(), b.detach()
            nan_a, nan_b = torch.isnan(a), torch.isnan(b)
            assert torch.equal(nan_a, nan_b), what
            same = torch.equal(a[~nan_a].view(torch.int32), b[~nan_b].view(torch.int32))
            assert same, (what, betas, int((a[~nan_a] != b[~nan_b]).sum()))
        print(f"{n} special combinations, betas {betas}: identical", flush=True)


def _rne_bf16_bits(bits: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even fp32 -> bf16 on int32 bit patterns, in int64 arithmetic
    (u + 0x7fff + ((u >> 16) & 1)) >> 16, every NaN -> 0x7FC0: the conversion torch's
    c10::BFloat16 performs, restated on the integers."""
    u = bits.to(torch.int64) & 0xFFFFFFFF
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    return torch.where(nan, torch.full_like(r, 0x7FC0), r)


@pytest.mark.parametrize("offset", [0, 1])
def test_bf16_copy_of_every_fp32_pattern(dev, offset):
    """The bf16 copy the update stores, for all 2^32 fp32 bit patterns as parameters, in
    16 slices of 2^28: lr 0, no weight decay and g = m = v = 0 leave p as it is, so the
    copy is the conversion of the input.  It must equal round-to-nearest-even with every
    NaN stored as 0x7FC0 (restated on the integers) and, for every non-NaN input, torch's
    own Tensor.to(torch.bfloat16) on the GPU.  offset 0: 16-byte aligned parameters, the
    four-lane stores; offset 1: a parameter one element into its buffer, the scalar path."""
    import mi_adamw
    n = 1 << 28
    store = torch.zeros(n + 8, device=dev)
    p = torch.nn.Parameter(store[offset:offset + n])
    p.grad = torch.zeros(n, device=dev)
    opt = mi_adamw.FusedAdamW([p], lr=0.0, weight_decay=0.0, bf16_copy=True)
    base = torch.arange(n, dtype=torch.int64, device=dev)
    for k in range(16):
        bits = (base + (k * n - (1 << 31))).to(torch.int32)
        with torch.no_grad():
            p.view(torch.int32).copy_(bits)
        opt.step()
        torch.cuda.synchronize()
        got = opt.bf16_param(p).view(torch.int16).to(torch.int64) & 0xFFFF
        assert torch.equal(got, _rne_bf16_bits(bits)), (k, offset)
        ok = ~torch.isnan(p.detach())
        assert torch.equal(p.detach().view(torch.int32)[ok], bits[ok]), (k, offset)
        ref = p.detach()[ok].to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
        assert torch.equal(got[ok], ref), (k, offset)
        del got, ok, ref
    print(f"2^32 patterns, offset {offset}: the copy is RNE with NaN -> 0x7FC0", flush=True)


def test_special_values_bf16_state_match_oracle(dev):
    """The special-value grid with bf16 moments (and a bf16 copy), against the oracle's
    bf16-state model: bf16 rounding of inf, NaN (0x7FC0), denormals and overflow to inf."""
    import mi_adamw
    specials = torch.tensor([0.0, -0.0, 1e-45, -1e-40, 9.2e-41, 1.17e-38, 1e-30, -1e-20, 1e-8,
                             1.0, -1.0, 3e4, 3.3961e38, 3.4e38, float("inf"), float("-inf"),
                             float("nan")], dtype=torch.float32)
    k = specials.numel()
    idx = torch.cartesian_prod(*(torch.arange(k) for _ in range(4)))
    pv, gv, mv, vv = (specials[idx[:, j]] for j in range(4))
    vv = vv.abs()
    p = torch.nn.Parameter(pv.clone().to(dev))
    p.grad = gv.clone().to(dev)
    opt = mi_adamw.FusedAdamW([p], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                              state_dtype=torch.bfloat16, bf16_copy=True)
    load_states(opt, [p], [{"step": torch.tensor(4.0), "exp_avg": mv.clone(),
                            "exp_avg_sq": vv.clone()}])
    opt.step()
    torch.cuda.synchronize()
    pn = pv.numpy().copy()
    mb = O.to_bf16_bits(mv.numpy())
    vb = O.to_bf16_bits(vv.numpy())
    O.adamw_step_bf16state(pn, gv.numpy().copy(), mb, vb, lr=1e-3, betas=(0.9, 0.95), eps=1e-8,
                           weight_decay=0.1, step=5.0)
    assert O.max_ulp(pn, to_np(p))[0] == 0
    got_m = to_np(opt.state[p]["exp_avg"].view(torch.int16)).view(np.uint16)
    got_v = to_np(opt.state[p]["exp_avg_sq"].view(torch.int16)).view(np.uint16)
    assert np.array_equal(got_m, mb) and np.array_equal(got_v, vb)
    copy = to_np(opt.bf16_param(p).view(torch.int16)).view(np.uint16)
    assert np.array_equal(copy, O.to_bf16_bits(pn))
    print(f"{idx.shape[0]} special combinations with bf16 state: identical to the oracle", flush=True)


def test_mismatched_checkpoint_state_raises_before_any_launch(dev):
    """A state dict from another model (moments of the wrong size) makes step() raise, as
    torch's own AdamW does, and nothing is written: no pointer of a too-small buffer ever
    reaches a kernel."""
    import mi_adamw
    params = make_params([(64, 48), (4099,)], dev)
    other = make_params([(64, 48), (4000,)], dev)
    for p in other:
        p.grad = torch.ones_like(p)
    donor = torch.optim.AdamW(other, lr=1e-3, fused=False)
    donor.step()
    ref_opt = torch.optim.AdamW(clone_params(params), lr=1e-3, fused=False)
    ref_opt.load_state_dict(donor.state_dict())
    for p in ref_opt.param_groups[0]["params"]:
        p.grad = torch.ones_like(p)
    with pytest.raises(RuntimeError):
        ref_opt.step()                                   # torch refuses too
    opt = mi_adamw.FusedAdamW(params, lr=1e-3, fused=False)
    opt.load_state_dict(donor.state_dict())
    for p in params:
        p.grad = torch.ones_like(p)
    before = [p.detach().clone() for p in params]
    with pytest.raises(RuntimeError, match="elements"):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b.detach()) for a, b in zip(before, params))


def test_thousands_of_ragged_tensors_with_clip(dev):
    """3,000 parameters of random sizes (most with a scalar tail, many smaller than one
    lane's vector) and two large ones: one table launch of thousands of rows, bit-identical
    to torch given the same clip norm."""
    import mi_adamw
    rng = np.random.default_rng(11)
    shapes = [(int(n),) for n in rng.integers(1, 5000, 3000)] + [(70001,), (262147,)]
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    topt = torch.optim.AdamW(ref, foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(ours, **hp, max_grad_norm=1.0)
    for step in range(1, 3):
        set_grads(ref, step, 1e-2)
        for p, q in zip(ref, ours):
            q.grad = p.grad.clone()
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    launch = oopt._launch_cache.launches[0]
    assert launch.n_rows == len(shapes) and launch.tables
    exact = O.total_norm([to_np(p.grad) for p in ours])
    print("rows", launch.n_rows, "chunks", launch.n_chunks, "norm", oopt.last_grad_norm.item(),
          float(exact), flush=True)
    _assert_same(ref, ours, topt, oopt, max_allowed=0)
