"""GPU: FusedAdamW(capturable=True) against torch.optim.AdamW(capturable=True, foreach=False),
and its step recorded into a HIP graph (torch.cuda.graph) and replayed.

torch's capturable chain keeps the step counts on the device and forms the
per-step values there in fp32 (adam.py:480-527): ``beta ** step`` by the device
pow, ``lr / bc1`` (a float lr as ``bc1.reciprocal() * lr``), ``sqrt(bc2) *
-step_size`` and ``eps / -step_size``, then ``p += m / (sqrt(v) / (sqrt(bc2) *
-step_size) + eps / -step_size)``.  A launch before the update forms the same values
once per tensor from its device step count, so parameters, moments and step counts
must be bit-identical step after step, eager or replayed from a graph.
"""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from _helpers import clone_params, make_params, max_ulp, max_ulp_all, set_grads

pytestmark = [
    pytest.mark.gpu,
    # torch warns once per optimizer that capturable=True runs uncaptured
    pytest.mark.filterwarnings("ignore:This instance was constructed with capturable=True"),
]

SHAPES = [(64, 48), (48,), (144, 48), (4099,), (3,), (7, 5), (70001,), (65536 + 12,)]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    return torch.device("cuda", 0)


def _pair(dev, shapes=SHAPES, opt_kw=None, lr=6e-4, lr_ours=None, **hp):
    import mi_adamw
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    topt = torch.optim.AdamW(ref, lr=lr, foreach=False, capturable=True, **hp)
    # foreach=False on both sides: a state dict carries it to whichever optimizer loads it
    oopt = mi_adamw.FusedAdamW(ours, lr=lr if lr_ours is None else lr_ours, foreach=False,
                               capturable=True, **hp, **(opt_kw or {}))
    return ref, ours, topt, oopt


def _copy_grads(ref, ours):
    for p, q in zip(ref, ours):
        q.grad = p.grad.clone()


def _same(ref, ours, topt, oopt):
    torch.cuda.synchronize()
    assert max_ulp_all(ref, ours) == 0
    for p, q in zip(ref, ours):
        ts, os_ = topt.state[p], oopt.state[q]
        assert os_["step"].device == q.device and os_["step"].dtype == torch.float32
        assert torch.equal(ts["step"], os_["step"])
        assert max_ulp(ts["exp_avg"], os_["exp_avg"]) == 0
        assert max_ulp(ts["exp_avg_sq"], os_["exp_avg_sq"]) == 0
        if "max_exp_avg_sq" in ts:
            assert max_ulp(ts["max_exp_avg_sq"], os_["max_exp_avg_sq"]) == 0


@pytest.mark.parametrize("betas,lr,wd,maximize,amsgrad", [
    ((0.9, 0.999), 6e-4, 0.1, False, False),   # mini-megatron's defaults (config.py:11,13)
    ((0.9, 0.95), 3e-4, 0.1, True, False),     # maximize
    ((0.3, 0.95), 1e-3, 0.0, False, False),    # lerp weight 0.7 (other Lerp.h branch), no decay
    ((0.9, 0.999), 6e-4, 0.1, False, True),    # amsgrad
    ((0.9, 0.95), 0.0, 0.1, False, False),     # lr 0: step_size 0, both denominator terms -inf
])
def test_capturable_chained_matches_torch_bitwise(dev, betas, lr, wd, maximize, amsgrad):
    ref, ours, topt, oopt = _pair(dev, lr=lr, betas=betas, weight_decay=wd, maximize=maximize,
                                  amsgrad=amsgrad)
    for step in range(1, 11):
        set_grads(ref, step, 1e-3)
        _copy_grads(ref, ours)
        topt.step()
        oopt.step()
        _same(ref, ours, topt, oopt)


@pytest.mark.parametrize("where", ["cuda", "cpu"])
def test_capturable_tensor_lr_with_scheduler(dev, where):
    """A tensor lr, driven by LambdaLR (which fill_()s it) with warm-up from 0
    (main.py:36-43): on the device the kernel reads it, on the host the step passes
    its value; both divide lr / bc1 truly, as torch does for a tensor lr."""
    d = dev if where == "cuda" else torch.device("cpu")
    ref, ours, topt, oopt = _pair(dev, lr=torch.tensor(6e-4, device=d),
                                  lr_ours=torch.tensor(6e-4, device=d), weight_decay=0.1)
    lam = lambda s: min(1.0, s / 3) * (0.5 + 0.5 / (1 + s))   # noqa: E731
    tsch = torch.optim.lr_scheduler.LambdaLR(topt, lam)
    osch = torch.optim.lr_scheduler.LambdaLR(oopt, lam)
    for step in range(1, 8):
        set_grads(ref, step, 1e-3)
        _copy_grads(ref, ours)
        topt.step()
        oopt.step()
        tsch.step()
        osch.step()
        _same(ref, ours, topt, oopt)
    assert float(oopt.param_groups[0]["lr"]) == float(topt.param_groups[0]["lr"]) > 0


def test_capturable_clip_copy_and_flat(dev):
    """The fused clip, the bf16 copy and the flat layout in the capturable chain,
    against torch's capturable step after clip_grads_with_norm_ with the same norm."""
    for flat in (False, True):
        ref, ours, topt, oopt = _pair(dev, weight_decay=0.1, opt_kw=dict(
            max_grad_norm=1.0, bf16_copy=True, flat_buffer=flat))
        for step in range(1, 6):
            set_grads(ref, step, 1e-2)
            for p, q in zip(ref, ours):
                if flat:
                    q.grad.copy_(p.grad)
                else:
                    q.grad = p.grad.clone()
            oopt.step()
            want = torch.nn.utils.get_total_norm([p.grad for p in ref])
            assert abs(oopt.last_grad_norm.item() - want.item()) <= 1e-6 * want.item()
            torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
            topt.step()
            _same(ref, ours, topt, oopt)
        for q in ours:
            assert torch.equal(oopt.bf16_param(q), q.detach().to(torch.bfloat16))


def test_capturable_state_dict_interchange(dev):
    """Checkpoints move between torch's capturable AdamW, FusedAdamW(capturable=True)
    and a non-capturable torch AdamW (host step counts), mid-training.  Each state
    dict is deep-copied, as torch.save / torch.load hand it over: load_state_dict
    keeps the very tensors of a live state dict whose dtype and device already fit."""
    import mi_adamw
    ref, ours, topt, oopt = _pair(dev, weight_decay=0.1)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        _copy_grads(ref, ours)
        topt.step()
        oopt.step()
    # torch -> ours, into a fresh capturable FusedAdamW
    ours2 = clone_params(ref)
    o2 = mi_adamw.FusedAdamW(ours2, lr=6e-4, weight_decay=0.1, foreach=False, capturable=True)
    o2.load_state_dict(copy.deepcopy(topt.state_dict()))
    # ours -> torch capturable
    ref2 = clone_params(ours)
    t2 = torch.optim.AdamW(ref2, lr=6e-4, weight_decay=0.1, foreach=False, capturable=True)
    t2.load_state_dict(copy.deepcopy(oopt.state_dict()))
    for step in range(4, 7):
        set_grads(ref, step, 1e-3)
        for group in (ours, ours2, ref2):
            _copy_grads(ref, group)
        for o in (topt, oopt, o2, t2):
            o.step()
    _same(ref, ours, topt, oopt)
    _same(ref, ours2, topt, o2)
    _same(ref, ref2, topt, t2)
    # a non-capturable checkpoint (host steps) into a capturable FusedAdamW
    tn = torch.optim.AdamW(clone_params(ref), lr=6e-4, weight_decay=0.1, foreach=False)
    sd = copy.deepcopy(topt.state_dict())
    for st in sd["state"].values():
        st["step"] = st["step"].cpu()
    tn.load_state_dict(sd)
    ours3 = clone_params(ref)
    o3 = mi_adamw.FusedAdamW(ours3, lr=6e-4, weight_decay=0.1, foreach=False, capturable=True)
    o3.load_state_dict(copy.deepcopy(tn.state_dict()))
    assert all(o3.state[q]["step"].device == dev for q in ours3)
    set_grads(ref, 7, 1e-3)
    _copy_grads(ref, ours3)
    topt.step()
    o3.step()
    _same(ref, ours3, topt, o3)


def test_graph_capture_replays_match_eager(dev):
    """step() (clip, bf16 copy) recorded once into a HIP graph after eager warm-up
    steps, then replayed with new gradients in the same tensors: every replay is
    bit-identical to torch's eager capturable step, with other eager work and
    synchronisation between replays."""
    ref, ours, topt, oopt = _pair(dev, weight_decay=0.1,
                                  opt_kw=dict(max_grad_norm=1.0, bf16_copy=True))
    for p in ref + ours:
        p.grad = torch.zeros_like(p)

    def fill(step):
        set_grads(ref, step, 1e-2)
        for p, q in zip(ref, ours):
            q.grad.copy_(p.grad)

    def torch_step():
        torch.nn.utils.clip_grads_with_norm_(ref, 1.0, oopt.last_grad_norm.clone())
        topt.step()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for step in range(1, 4):
            fill(step)
            oopt.step()
            torch_step()
    torch.cuda.current_stream().wait_stream(side)
    _same(ref, ours, topt, oopt)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        oopt.step()
    captured_norm = oopt.last_grad_norm
    for step in range(4, 10):
        fill(step)
        graph.replay()
        assert oopt.last_grad_norm is captured_norm
        torch_step()
        _same(ref, ours, topt, oopt)
        for q in ours:
            assert torch.equal(oopt.bf16_param(q), q.detach().to(torch.bfloat16))
        # unrelated eager work between replays
        torch.randn(1 << 20, device=dev).sum().item()
    assert float(oopt.state[ours[0]]["step"]) == 9.0


def test_capture_refuses_moved_gradients(dev):
    """A step under capture must find the tables of an earlier eager step: with a
    gradient moved to a new tensor it raises instead of recording an upload."""
    ref, ours, topt, oopt = _pair(dev)
    set_grads(ours, 1, 1e-3)
    oopt.step()
    torch.cuda.synchronize()
    ours[0].grad = ours[0].grad.clone()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="under graph capture"):
        with torch.cuda.graph(graph):
            oopt.step()
    torch.cuda.synchronize()
    oopt.step()          # eager again: the rows are refreshed and the step runs
    torch.cuda.synchronize()
    assert float(oopt.state[ours[0]]["step"]) == 2.0


def _torch_den(b1, b2, lr, eps, step, dev, lr_tensor=False):
    """torch's own per-step values of the capturable chain (adam.py:480-522), run as
    the same 0-d tensor ops on the GPU: (sqrt(bc2) * -step_size, eps / -step_size)."""
    step_t = torch.tensor(float(step), device=dev)
    bc1 = 1 - b1 ** step_t
    bc2 = 1 - b2 ** step_t
    lr_v = torch.tensor(lr, device=dev) if lr_tensor else lr
    step_size = lr_v / bc1
    neg = step_size.neg()
    return float(bc2.sqrt() * neg), float(eps / neg)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_oracle_capturable_chain_matches_torch_on_the_gpu(dev, amsgrad):
    """Pins the oracle's capturable chain: with torch's per-step values, its
    ROCm op model reproduces torch.optim.AdamW(capturable=True, foreach=False)
    on the MI355X bit for bit, mid-training, over several steps."""
    from oracle import oracle as O
    n = 70001
    gen_ = torch.Generator(device=dev).manual_seed(5)
    p = torch.nn.Parameter(torch.randn(n, device=dev, generator=gen_) * 0.02)
    t = torch.optim.AdamW([p], lr=6e-4, betas=(0.9, 0.999), weight_decay=0.1, foreach=False,
                          capturable=True, amsgrad=amsgrad)
    pn = p.detach().cpu().numpy().copy()
    mn, vn = np.zeros(n, np.float32), np.zeros(n, np.float32)
    xn = np.zeros(n, np.float32) if amsgrad else None
    for step in range(1, 6):
        p.grad = torch.randn(n, device=dev, generator=gen_) * 1e-3
        gn = p.grad.cpu().numpy().copy()
        t.step()
        O.adamw_step_capt(pn, gn, mn, vn, lr=6e-4, betas=(0.9, 0.999), eps=1e-8,
                          weight_decay=0.1, step=step, vmax=xn,
                          den=_torch_den(0.9, 0.999, 6e-4, 1e-8, step, dev))
        st = t.state[p]
        assert O.max_ulp(pn, p.detach().cpu().numpy())[0] == 0
        assert np.array_equal(mn, st["exp_avg"].cpu().numpy())
        assert np.array_equal(vn, st["exp_avg_sq"].cpu().numpy())
        if amsgrad:
            assert np.array_equal(xn, st["max_exp_avg_sq"].cpu().numpy())


@pytest.mark.parametrize("amsgrad,clip", [(False, True), (True, False)])
def test_capturable_bf16_state_matches_oracle(dev, amsgrad, clip):
    """bf16 moments in the capturable chain (torch has no such mode): the kernel
    against the oracle's capturable bf16-state step, bit for bit, with torch's
    per-step values, over several steps from a mid-training state."""
    import mi_adamw
    from oracle import oracle as O
    shapes = [(4099,), (64, 48), (70001,)]
    ps = make_params(shapes, dev)
    opt = mi_adamw.FusedAdamW(ps, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, capturable=True,
                              state_dtype=torch.bfloat16, amsgrad=amsgrad,
                              max_grad_norm=1.0 if clip else None)
    gen_ = torch.Generator(device=dev).manual_seed(9)
    host = []
    for q in ps:
        m0 = (torch.randn(q.numel(), device=dev, generator=gen_) * 1e-3).bfloat16()
        v0 = (torch.randn(q.numel(), device=dev, generator=gen_) * 1e-6).abs().bfloat16()
        x0 = (v0.float() * 1.5).bfloat16() if amsgrad else None
        opt.set_state(q, 40.0, m0.view(q.shape), v0.view(q.shape),
                      None if x0 is None else x0.view(q.shape))
        host.append([q.detach().cpu().numpy().reshape(-1).copy(),
                     m0.view(torch.int16).cpu().numpy().view(np.uint16).copy(),
                     v0.view(torch.int16).cpu().numpy().view(np.uint16).copy(),
                     None if x0 is None else x0.view(torch.int16).cpu().numpy().view(np.uint16).copy()])
    for step in range(41, 45):
        set_grads(ps, step, 1e-2)
        opt.step()
        coef = O.clip_coef(np.float32(opt.last_grad_norm.item()), 1.0) if clip else None
        den = _torch_den(0.9, 0.95, 3e-4, 1e-8, step, dev)
        for q, (pn, mb, vb, xb) in zip(ps, host):
            O.adamw_step_capt_bf16state(pn, q.grad.detach().cpu().numpy().reshape(-1).copy(),
                                        mb, vb, lr=3e-4, betas=(0.9, 0.95), eps=1e-8,
                                        weight_decay=0.1, step=step, grad_scale=coef,
                                        vmax_bits=xb, den=den)
            st = opt.state[q]
            assert O.max_ulp(pn, q.detach().cpu().numpy().reshape(-1))[0] == 0
            assert np.array_equal(mb, st["exp_avg"].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))
            assert np.array_equal(vb, st["exp_avg_sq"].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))
            if amsgrad:
                assert np.array_equal(xb, st["max_exp_avg_sq"].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1))


def test_capturable_params_without_grads_and_many_groups(dev):
    """Tensors of one launch at different device step counts (some params skip steps:
    the counts advance by index_add_ over the stepped ones), over 18 param groups, more
    than one launch's 16 constant sets."""
    import mi_adamw
    shapes = [(37,), (4099,), (64, 48), (5,)] * 9
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    groups = lambda ps: [dict(params=ps[2 * i:2 * i + 2], lr=1e-4 * (i + 1),   # noqa: E731
                              weight_decay=0.01 * (i % 3)) for i in range(18)]
    topt = torch.optim.AdamW(groups(ref), foreach=False, capturable=True)
    oopt = mi_adamw.FusedAdamW(groups(ours), foreach=False, capturable=True)
    for step in range(1, 7):
        set_grads(ref, step, 1e-3)
        for i, (p, q) in enumerate(zip(ref, ours)):
            if (i % 5 == 0 and step % 2 == 0) or (i % 3 == 1 and step == 3):   # skips
                p.grad = None
                q.grad = None
            else:
                q.grad = p.grad.clone()
        topt.step()
        oopt.step()
        torch.cuda.synchronize()
        assert max_ulp_all(ref, ours) == 0
        for p, q in zip(ref, ours):
            if p in topt.state:
                assert torch.equal(topt.state[p]["step"], oopt.state[q]["step"])
                assert max_ulp(topt.state[p]["exp_avg_sq"], oopt.state[q]["exp_avg_sq"]) == 0
    steps = {float(oopt.state[q]["step"]) for q in ours}
    assert len(steps) > 1


@pytest.mark.parametrize("fused", [False, True])
def test_capturable_more_rows_than_one_prep_workgroup(dev, fused):
    """300 tensors in one launch: the launch that forms each table row's per-step values
    runs 256 rows per workgroup, so rows 256-299 come from its second workgroup.  Row i
    and row i - 256 differ in shape, group (lr) and device step count (steps 2-7 each skip
    the tensors with i mod 7 == step - 1), so a row reading another row's slot changes
    bits; the last step skips none, so its launch has all 300 rows.
    Both capturable chains: torch's capturable AdamW (foreach=False) and fused=True."""
    import mi_adamw
    cycle = [(37,), (4099,), (64, 48), (5,), (129,)]
    shapes = [cycle[i % len(cycle)] for i in range(300)]
    ref = make_params(shapes, dev)
    ours = clone_params(ref)

    def groups(ps):
        return [dict(params=ps[75 * k:75 * (k + 1)], lr=1e-4 * (k + 1),
                     weight_decay=0.05 * k) for k in range(4)]

    kw = dict(fused=True) if fused else dict(foreach=False)
    topt = torch.optim.AdamW(groups(ref), capturable=True, **kw)
    oopt = mi_adamw.FusedAdamW(groups(ours), capturable=True, **kw)
    for step in range(1, 9):
        set_grads(ref, step, 1e-3)
        for i, (p, q) in enumerate(zip(ref, ours)):
            if 1 < step < 8 and i % 7 == step - 1:
                p.grad = None
                q.grad = None
            else:
                q.grad = p.grad.clone()
        topt.step()
        oopt.step()
        torch.cuda.synchronize()
        assert max_ulp_all(ref, ours) == 0
        for p, q in zip(ref, ours):
            ts, os_ = topt.state[p], oopt.state[q]
            assert torch.equal(ts["step"], os_["step"])
            assert max_ulp(ts["exp_avg"], os_["exp_avg"]) == 0
            assert max_ulp(ts["exp_avg_sq"], os_["exp_avg_sq"]) == 0
    assert max(l.n_rows for l in oopt._launch_cache.launches) > 256
    assert float(oopt.state[ours[0]]["step"]) != float(oopt.state[ours[256]]["step"])


def test_capturable_deepcopy_mid_training(dev):
    """copy.deepcopy of a capturable FusedAdamW mid-training: the copy's device step
    counts and moments continue exactly as the original's."""
    ref, ours, topt, oopt = _pair(dev, weight_decay=0.1)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        _copy_grads(ref, ours)
        topt.step()
        oopt.step()
    twin = copy.deepcopy({"params": ours, "opt": oopt})
    ours2, o2 = twin["params"], twin["opt"]
    assert all(o2.state[q]["step"].device == dev for q in ours2)
    for step in range(4, 7):
        set_grads(ref, step, 1e-3)
        _copy_grads(ref, ours)
        _copy_grads(ref, ours2)
        topt.step()
        oopt.step()
        o2.step()
    _same(ref, ours, topt, oopt)
    _same(ref, ours2, topt, o2)


def test_whole_training_iteration_in_one_graph(dev):
    """zero_grad, a bf16-autocast forward and backward of a reference-shaped GPT and the
    capturable step (flat layout, clip), recorded into one HIP graph: every replay, with
    new batches copied into the static inputs and eager work in between, is bit-identical
    to the same iteration run eagerly on a twin model (loss, gradients, parameters).  The
    model's forward and backward kernels are deterministic on the MI355X (30 repeated
    passes bit-identical, at this size and at gpt-125m), so any difference is the graph's."""
    import mi_adamw
    import refgpt

    def build():
        model = refgpt.tiny(dev, seed=4)
        opt = mi_adamw.FusedAdamW(model.parameters(), lr=6e-4, weight_decay=0.1,
                                  capturable=True, flat_buffer=True, max_grad_norm=1.0)
        return model, opt

    def iteration(model, opt, ids, labels, mask):
        opt.zero_grad()
        with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            _, loss = model(ids, labels, mask)
        loss.backward()
        opt.step()
        return loss

    eager, graphed = build(), build()
    data = [refgpt.batch(dev, seed=s) for s in range(10)]
    static = [t.clone() for t in data[0]]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(3):
            for t, src in zip(static, data[k]):
                t.copy_(src)
            iteration(*graphed, *static)
            iteration(*eager, *data[k])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = iteration(*graphed, *static)
    for k in range(3, 10):
        for t, src in zip(static, data[k]):
            t.copy_(src)
        graph.replay()
        loss = iteration(*eager, *data[k])
        torch.cuda.synchronize()
        assert torch.equal(static_loss, loss)
        for p, q in zip(eager[0].parameters(), graphed[0].parameters()):
            assert torch.equal(p.grad, q.grad) and torch.equal(p, q)
        torch.randn(1 << 16, device=dev).sum().item()
    assert float(graphed[1].state[next(graphed[0].parameters())]["step"]) == 10.0
