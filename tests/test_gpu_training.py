"""GPU: FusedAdamW in a training loop shaped like mini-megatron's (main.py:177-211).

A small pre-LN GPT in the reference's parameter order (token and position
embeddings, per layer ln1 / qkv / o / ln2 / fc1 / fc2 with bias-free linears,
ln_f, an untied lm_head) trains with torch.optim.AdamW(fused=False) in one copy
and FusedAdamW in another, both driven by LambdaLR with warm-up (lr is 0 at
iteration 0, main.py:36-43), zero_grad -> forward -> backward -> step.  The
two runs see identical forward/backward kernels, so parameters, moments and
losses must stay bit-identical step after step.  Also: param groups with
different hyperparameters (decay / no-decay), more distinct hyperparameter
sets than one launch holds, a tensor lr, clip write-back (in every update
variant) and complex params.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from _helpers import clone_params, gen, make_params, max_ulp, max_ulp_all, set_grads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    return torch.device("cuda", 0)


class TinyGPT(torch.nn.Module):
    def __init__(self, vocab=512, hidden=64, heads=4, ffn=256, layers=2, positions=64):
        super().__init__()
        self.heads = heads
        self.tok = torch.nn.Embedding(vocab, hidden)
        self.pos = torch.nn.Embedding(positions, hidden)
        self.blocks = torch.nn.ModuleList()
        for _ in range(layers):
            self.blocks.append(torch.nn.ModuleDict(dict(
                ln1=torch.nn.LayerNorm(hidden),
                qkv=torch.nn.Linear(hidden, 3 * hidden, bias=False),
                o=torch.nn.Linear(hidden, hidden, bias=False),
                ln2=torch.nn.LayerNorm(hidden),
                fc1=torch.nn.Linear(hidden, ffn, bias=False),
                fc2=torch.nn.Linear(ffn, hidden, bias=False))))
        self.ln_f = torch.nn.LayerNorm(hidden)
        self.lm_head = torch.nn.Linear(hidden, vocab, bias=False)

    def forward(self, tokens):
        b, s = tokens.shape
        x = self.tok(tokens) + self.pos(torch.arange(s, device=tokens.device))
        for blk in self.blocks:
            h = blk["ln1"](x)
            q, k, v = blk["qkv"](h).view(b, s, 3, self.heads, -1).unbind(2)
            q, k, v = (t.transpose(1, 2) for t in (q, k, v))
            att = (q @ k.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
            mask = torch.ones(s, s, device=tokens.device, dtype=torch.bool).tril()
            att = att.masked_fill(~mask, float("-inf")).softmax(-1)
            x = x + blk["o"]((att @ v).transpose(1, 2).reshape(b, s, -1))
            x = x + blk["fc2"](F.gelu(blk["fc1"](blk["ln2"](x))))
        return self.lm_head(self.ln_f(x))


def _lr_lambda(warmup, total):
    # Cosine schedule with linear warm-up, as main.py:36-43 defines it.
    def f(step):
        if step < warmup:
            return step / max(warmup, 1)
        progress = (step - warmup) / max(total - warmup, 1)
        return 0.5 * (1.0 + math.cos(progress * math.pi))
    return f


def test_training_loop_bit_identical(dev):
    import mi_adamw
    torch.manual_seed(0)
    ref = TinyGPT().to(dev)
    ours = TinyGPT().to(dev)
    ours.load_state_dict(ref.state_dict())
    topt = torch.optim.AdamW(ref.parameters(), lr=6e-4, weight_decay=0.1, fused=False)
    oopt = mi_adamw.AdamW(ours.parameters(), lr=6e-4, weight_decay=0.1, fused=False)
    tsch = torch.optim.lr_scheduler.LambdaLR(topt, _lr_lambda(3, 20))
    osch = torch.optim.lr_scheduler.LambdaLR(oopt, _lr_lambda(3, 20))
    g = gen(dev, 7)
    for step in range(12):
        tokens = torch.randint(0, 512, (4, 32), device=dev, generator=g)
        losses = []
        for model, opt in ((ref, topt), (ours, oopt)):
            opt.zero_grad()
            logits = model(tokens)
            loss = F.cross_entropy(logits.view(-1, logits.shape[-1]), tokens.view(-1))
            loss.backward()
            losses.append(loss.item())
        # Same parameters in, same kernels: forward and backward agree bitwise, so
        # any later difference comes from the optimizer step.
        assert losses[0] == losses[1]
        assert max_ulp_all([p.grad for p in ref.parameters()], [q.grad for q in ours.parameters()]) == 0
        topt.step()
        oopt.step()
        tsch.step()
        osch.step()
        print(f"step {step}: lr {topt.param_groups[0]['lr']:.3g} loss {losses[0]:.6f}", flush=True)
        assert max_ulp_all(list(ref.parameters()), list(ours.parameters())) == 0
    for p, q in zip(ref.parameters(), ours.parameters()):
        assert max_ulp(topt.state[p]["exp_avg"], oopt.state[q]["exp_avg"]) == 0
        assert max_ulp(topt.state[p]["exp_avg_sq"], oopt.state[q]["exp_avg_sq"]) == 0


def test_decay_and_no_decay_groups(dev):
    import mi_adamw
    params = make_params([(128, 64), (64,), (64,), (300, 64), (7,)], dev)
    ours = clone_params(params)
    groups = lambda ps: [{"params": [ps[0], ps[3]], "weight_decay": 0.1},
                         {"params": [ps[1], ps[2], ps[4]], "weight_decay": 0.0, "lr": 1e-3}]
    topt = torch.optim.AdamW(groups(params), lr=3e-4, betas=(0.9, 0.95), fused=False)
    oopt = mi_adamw.FusedAdamW(groups(ours), lr=3e-4, betas=(0.9, 0.95), fused=False)
    for step in range(1, 6):
        set_grads(params, step, 1e-3)
        for p, q in zip(params, ours):
            q.grad = p.grad.clone()
        topt.param_groups[1]["lr"] *= 0.5
        oopt.param_groups[1]["lr"] *= 0.5
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    assert max_ulp_all(params, ours) == 0


def test_more_hyper_sets_than_one_launch(dev):
    """20 groups with different lr: 20 distinct hyperparameter sets, two launches."""
    import mi_adamw
    params = make_params([(257,)] * 20, dev)
    ours = clone_params(params)
    tg = [{"params": [p], "lr": 1e-4 * (i + 1)} for i, p in enumerate(params)]
    og = [{"params": [p], "lr": 1e-4 * (i + 1)} for i, p in enumerate(ours)]
    topt = torch.optim.AdamW(tg, fused=False)
    oopt = mi_adamw.FusedAdamW(og, fused=False, max_grad_norm=1.0)
    for step in range(1, 4):
        set_grads(params, step, 1e-1)
        for p, q in zip(params, ours):
            q.grad = p.grad.clone()
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(params, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    assert max_ulp_all(params, ours) == 0


def test_tensor_lr(dev):
    import mi_adamw
    params = make_params([(1000,)], dev)
    ours = clone_params(params)
    topt = torch.optim.AdamW(params, lr=torch.tensor(3e-4), foreach=False)
    oopt = mi_adamw.FusedAdamW(ours, lr=torch.tensor(3e-4))
    for step in range(1, 4):
        set_grads(params, step, 1e-3)
        ours[0].grad = params[0].grad.clone()
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    assert max_ulp_all(params, ours) == 0


def test_clip_write_grads_matches_clip_grad_norm(dev):
    import mi_adamw
    params = make_params([(4096,), (33, 17), (5,)], dev)
    ours = clone_params(params)
    topt = torch.optim.AdamW(params, lr=3e-4, foreach=False)
    oopt = mi_adamw.FusedAdamW(ours, lr=3e-4, max_grad_norm=0.5, clip_write_grads=True)
    set_grads(params, 1, 1e-1)
    for p, q in zip(params, ours):
        q.grad = p.grad.clone()
    oopt.step()
    torch.nn.utils.clip_grads_with_norm_(params, 0.5, oopt.last_grad_norm.clone())
    topt.step()
    torch.cuda.synchronize()
    assert max_ulp_all([p.grad for p in params], [q.grad for q in ours]) == 0
    assert max_ulp_all(params, ours) == 0


@pytest.mark.parametrize("state_dtype,copy,flat,capt", [
    (torch.bfloat16, True, False, False),
    (torch.float32, True, True, False),
    (torch.bfloat16, False, True, False),
    (torch.float32, False, False, True),
])
def test_clip_write_grads_in_every_update_variant(dev, state_dtype, copy, flat, capt):
    """The clipped-gradient store in the bf16-state, bf16-copy, flat and capturable
    update variants, three chained steps: the stored gradients equal
    clip_grads_with_norm_'s, and parameters, moments and copies equal those of the
    same optimizer without the store (which the other tests pin to torch)."""
    import warnings
    import mi_adamw
    shapes = [(4096,), (33, 17), (5,), (8192,)]
    a = make_params(shapes, dev)
    b = clone_params(a)
    kw = dict(lr=3e-4, weight_decay=0.1, max_grad_norm=0.5, state_dtype=state_dtype,
              bf16_copy=copy, flat_buffer=flat, capturable=capt)
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
        stored = mi_adamw.FusedAdamW(a, clip_write_grads=True, **kw)
        plain = mi_adamw.FusedAdamW(b, **kw)
        for step in range(1, 4):
            grads = [torch.randn(s, device=dev, generator=gen(dev, 4000 + 10000 * step + i)) * 1e-1
                     for i, s in enumerate(shapes)]
            for p, q, g in zip(a, b, grads):
                p.grad = g.clone()
                q.grad = g.clone()
            stored.step()
            plain.step()
            holders = [torch.nn.Parameter(torch.empty_like(g)) for g in grads]
            for h, g in zip(holders, grads):
                h.grad = g.clone()
            torch.nn.utils.clip_grads_with_norm_(holders, 0.5, stored.last_grad_norm.clone())
            torch.cuda.synchronize()
            assert torch.equal(stored.last_grad_norm, plain.last_grad_norm)
            assert max_ulp_all([p.grad for p in a], [h.grad for h in holders]) == 0, step
            assert max_ulp_all([q.grad for q in b], grads) == 0, step   # no store: unchanged
            assert max_ulp_all(a, b) == 0, step
            for p, q in zip(a, b):
                for key in ("exp_avg", "exp_avg_sq"):
                    assert torch.equal(stored.state[p][key], plain.state[q][key]), (step, key)
            if copy:
                for x, y in zip(stored.bf16_params(), plain.bf16_params()):
                    assert torch.equal(x, y), step


def test_complex_params_follow_view_as_real(dev):
    import mi_adamw
    base = torch.randn(300, 2, device=dev, generator=gen(dev, 3)) * 0.02
    p = torch.nn.Parameter(torch.view_as_complex(base.clone()))
    q = torch.nn.Parameter(torch.view_as_complex(base.clone()))
    topt = torch.optim.AdamW([p], lr=3e-4, foreach=False)
    oopt = mi_adamw.FusedAdamW([q], lr=3e-4)
    for step in range(1, 4):
        g = torch.randn(300, 2, device=dev, generator=gen(dev, 10 + step)) * 1e-3
        p.grad = torch.view_as_complex(g.clone())
        q.grad = torch.view_as_complex(g.clone())
        topt.step()
        oopt.step()
    torch.cuda.synchronize()
    assert max_ulp(torch.view_as_real(p), torch.view_as_real(q)) == 0


def test_flat_buffer_training_loop(dev):
    """flat_buffer=True in a real backward: grads accumulate into the flat views.

    Flat mode keeps gradients allocated, so the torch reference runs
    zero_grad(set_to_none=False)."""
    import mi_adamw
    torch.manual_seed(1)
    ref = TinyGPT().to(dev)
    ours = TinyGPT().to(dev)
    ours.load_state_dict(ref.state_dict())
    topt = torch.optim.AdamW(ref.parameters(), lr=6e-4, weight_decay=0.1, fused=False)
    oopt = mi_adamw.AdamW(ours.parameters(), lr=6e-4, weight_decay=0.1, fused=False,
                          flat_buffer=True, max_grad_norm=1.0, bf16_copy=True)
    tsch = torch.optim.lr_scheduler.LambdaLR(topt, _lr_lambda(2, 10))
    osch = torch.optim.lr_scheduler.LambdaLR(oopt, _lr_lambda(2, 10))
    grad_base = oopt._flat.grad.data_ptr()
    g = gen(dev, 11)
    for step in range(8):
        tokens = torch.randint(0, 512, (4, 32), device=dev, generator=g)
        for model, opt in ((ref, topt), (ours, oopt)):
            opt.zero_grad(set_to_none=False)
            logits = model(tokens)
            F.cross_entropy(logits.view(-1, logits.shape[-1]), tokens.view(-1)).backward()
        assert max_ulp_all([p.grad for p in ref.parameters()], [q.grad for q in ours.parameters()]) == 0
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(list(ref.parameters()), 1.0, oopt.last_grad_norm.clone())
        topt.step()
        tsch.step()
        osch.step()
        assert max_ulp_all(list(ref.parameters()), list(ours.parameters())) == 0
    # backward wrote into the flat buffer: every grad is still a view of it
    assert all(oopt._flat.is_grad_view(q, q.grad) for q in ours.parameters())
    assert oopt._flat.grad.data_ptr() == grad_base
    for q in ours.parameters():
        assert torch.equal(oopt.bf16_param(q), q.detach().to(torch.bfloat16))


@pytest.mark.parametrize("flat", [False, True])
def test_checkpoint_interchange_with_torch(dev, flat):
    """save_checkpoint / load_checkpoint (checkpoint.py:5-21: torch.save, then
    torch.load(weights_only=True)) across FusedAdamW and torch.optim.AdamW."""
    import io
    import mi_adamw
    shapes = [(96, 64), (64,), (200,), (33, 7)]
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=False)
    ours = make_params(shapes, dev)
    ref = clone_params(ours)
    oopt = mi_adamw.FusedAdamW(ours, flat_buffer=flat, **hp)
    topt = torch.optim.AdamW(ref, **hp)
    for step in range(1, 4):
        set_grads(ref, step, 1e-3)
        for p, q in zip(ref, ours):
            if q.grad is None:
                q.grad = p.grad.clone()
            else:
                q.grad.copy_(p.grad)
        oopt.step()
        topt.step()
    assert max_ulp_all(ref, ours) == 0

    def roundtrip(opt):
        buf = io.BytesIO()
        torch.save({"optimizer_state": opt.state_dict(), "step": 3}, buf)
        buf.seek(0)
        return torch.load(buf, map_location=dev, weights_only=True)["optimizer_state"]

    # ours -> torch, torch -> ours; both continue two more steps in lockstep.
    p_t = clone_params(ours)
    t2 = torch.optim.AdamW(p_t, **hp)
    t2.load_state_dict(roundtrip(oopt))
    p_o = clone_params(ref)
    o2 = mi_adamw.FusedAdamW(p_o, flat_buffer=flat, **hp)
    o2.load_state_dict(roundtrip(topt))
    for step in range(4, 6):
        set_grads(p_t, step, 1e-3)
        for p, q in zip(p_t, p_o):
            if q.grad is None:
                q.grad = p.grad.clone()
            else:
                q.grad.copy_(p.grad)
        t2.step()
        o2.step()
    torch.cuda.synchronize()
    assert max_ulp_all(p_t, p_o) == 0
    for p, q in zip(p_t, p_o):
        assert max_ulp(t2.state[p]["exp_avg"], o2.state[q]["exp_avg"]) == 0
        assert max_ulp(t2.state[p]["exp_avg_sq"], o2.state[q]["exp_avg_sq"]) == 0
        assert float(t2.state[p]["step"]) == float(o2.state[q]["step"]) == 5.0


def test_clip_grad_norm_error_if_nonfinite(dev):
    import mi_adamw
    p = torch.nn.Parameter(torch.zeros(100, device=dev))
    p.grad = torch.ones(100, device=dev)
    p.grad[3] = float("inf")
    with pytest.raises(RuntimeError, match="non-finite"):
        mi_adamw.clip_grad_norm_([p], 1.0, error_if_nonfinite=True)
    with pytest.raises(NotImplementedError):
        mi_adamw.clip_grad_norm_([p], 1.0, norm_type=float("inf"))
    q = torch.nn.Parameter(torch.zeros(100, device=dev))
    q.grad = torch.full((100,), 0.5, device=dev)
    n = mi_adamw.clip_grad_norm_([q], 1.0)
    assert n.item() == 5.0                       # |0.5| * sqrt(100)
    assert torch.all(q.grad == torch.tensor(0.5 * (1.0 / (5.0 + 1e-6)), device=dev).float())


def test_moving_gradients_refresh_rows_only(dev):
    """zero_grad(set_to_none=True) frees the gradients; backward may allocate them
    elsewhere.  Gradients forced to new addresses every step: the chunk tables are built
    once, the rows are rewritten, and the results stay bit-identical to torch."""
    import mi_adamw
    from mi_adamw import optimizer as O
    shapes = [(64, 48), (48,), (4099,), (70001,), (3,)]
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    topt = torch.optim.AdamW(ref, foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW(ours, **hp)
    builds = []
    real_init = O._Launch.__init__

    def counting(self, *a, **k):
        builds.append(1)
        return real_init(self, *a, **k)

    O._Launch.__init__ = counting
    try:
        held, seen = [], set()
        for step in range(1, 6):
            set_grads(ref, step, 1e-3)
            held.append([q.grad for q in ours if q.grad is not None])  # keeps the old blocks taken
            oopt.zero_grad(set_to_none=True)
            for p, q in zip(ref, ours):
                q.grad = p.grad.clone()
            seen.add(tuple(q.grad.data_ptr() for q in ours))
            topt.step()
            oopt.step()
    finally:
        O._Launch.__init__ = real_init
    torch.cuda.synchronize()
    assert len(seen) == 5, "the gradients did not move"
    assert len(builds) == 1, f"tables built {len(builds)} times"
    assert max_ulp_all(ref, ours) == 0
    assert max_ulp_all([topt.state[p]["exp_avg"] for p in ref],
                       [oopt.state[q]["exp_avg"] for q in ours]) == 0


def test_deepcopy_mid_training_continues_identically(dev):
    """copy.deepcopy of a FusedAdamW mid-training (as torch optimizers allow) gives an
    optimizer over copied parameters that continues bit for bit like the original."""
    import copy
    import mi_adamw
    params = make_params([(64, 48), (4099,), (3,)], dev)
    opt = mi_adamw.FusedAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                              max_grad_norm=1.0, bf16_copy=True)
    for step in range(1, 4):
        set_grads(params, step, 1e-2)
        opt.step()
    clone = copy.deepcopy(opt)
    cparams = clone.param_groups[0]["params"]
    for step in range(4, 7):
        set_grads(params, step, 1e-2)
        set_grads(cparams, step, 1e-2)
        opt.step()
        clone.step()
    torch.cuda.synchronize()
    assert max_ulp_all(params, cparams) == 0
    assert torch.equal(opt.last_grad_norm, clone.last_grad_norm)
    for p, q in zip(params, cparams):
        assert float(opt.state[p]["step"]) == float(clone.state[q]["step"]) == 6.0
        assert torch.equal(opt.bf16_param(p), clone.bf16_param(q))


def _batch(dev, seed):
    return torch.randint(0, 512, (4, 32), device=dev, generator=gen(dev, seed))


def _train_step(model, opt, sch, tokens):
    """zero_grad, forward, backward, step, scheduler step (main.py:202-210)."""
    opt.zero_grad()
    logits = model(tokens)
    loss = F.cross_entropy(logits.view(-1, logits.shape[-1]), tokens.view(-1))
    loss.backward()
    opt.step()
    sch.step()
    return loss.detach()


def test_checkpoint_file_round_trip_as_the_reference_does(dev):
    """checkpoint.py:5-21: torch.save of model, optimizer and scheduler state, then
    torch.load(map_location=device, weights_only=True) and the three load_state_dict
    calls.  Training continues bit for bit, and the bf16 copies match the loaded masters."""
    import io
    import mi_adamw
    hp = dict(lr=6e-4, weight_decay=0.1, fused=False)

    def build(seed):
        torch.manual_seed(seed)
        m = TinyGPT().to(dev)
        o = mi_adamw.FusedAdamW(m.parameters(), **hp, bf16_copy=True, max_grad_norm=1.0)
        s = torch.optim.lr_scheduler.LambdaLR(o, _lr_lambda(2, 10))
        return m, o, s

    model, opt, sch = build(0)
    batches = [_batch(dev, 100 + i) for i in range(6)]
    for ids in batches[:3]:
        _train_step(model, opt, sch, ids)
    buf = io.BytesIO()
    torch.save({"model_state": model.state_dict(), "optimizer_state": opt.state_dict(),
                "scheduler_state": sch.state_dict(), "step": 3}, buf)
    buf.seek(0)
    model2, opt2, sch2 = build(1)                      # different initial weights
    state = torch.load(buf, map_location=dev, weights_only=True)
    model2.load_state_dict(state["model_state"])
    opt2.load_state_dict(state["optimizer_state"])
    sch2.load_state_dict(state["scheduler_state"])
    for p in model2.parameters():
        assert torch.equal(opt2.bf16_param(p), p.detach().bfloat16())
    for ids in batches[3:]:
        la = _train_step(model, opt, sch, ids)
        lb = _train_step(model2, opt2, sch2, ids)
        assert torch.equal(la, lb)
    torch.cuda.synchronize()
    assert max_ulp_all(list(model.parameters()), list(model2.parameters())) == 0


@pytest.mark.parametrize("flat", [False, True])
def test_empty_tensors_and_empty_groups_with_clip(dev, flat):
    """Zero-element parameters, a param group holding nothing else, and a model with
    nothing but empty tensors: the step runs, as torch's does, and the norm of no
    elements is 0."""
    import mi_adamw
    shapes_a = [(0,), (0, 5)]
    shapes_b = [(64, 48), (4099,)]
    ref_a, ref_b = make_params(shapes_a, dev), make_params(shapes_b, dev, seed=2000)
    ours_a, ours_b = clone_params(ref_a), clone_params(ref_b)
    hp = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    topt = torch.optim.AdamW([dict(params=ref_a), dict(params=ref_b)], foreach=False, **hp)
    oopt = mi_adamw.FusedAdamW([dict(params=ours_a), dict(params=ours_b)], **hp,
                               max_grad_norm=1.0, flat_buffer=flat)
    for step in range(1, 4):
        set_grads(ref_a + ref_b, step, 1e-2)
        for p, q in zip(ref_a + ref_b, ours_a + ours_b):
            if flat:
                q.grad.copy_(p.grad)
            else:
                q.grad = p.grad.clone()
        oopt.step()
        torch.nn.utils.clip_grads_with_norm_(ref_a + ref_b, 1.0, oopt.last_grad_norm.clone())
        topt.step()
    torch.cuda.synchronize()
    assert max_ulp_all(ref_b, ours_b) == 0
    # nothing but empty tensors
    empties = make_params(shapes_a, dev)
    opt = mi_adamw.FusedAdamW(empties, max_grad_norm=1.0, flat_buffer=flat)
    for p in empties:
        if not flat:
            p.grad = torch.zeros_like(p)
    opt.step()
    torch.cuda.synchronize()
    assert opt.last_grad_norm.item() == 0.0


def test_flat_buffer_under_distributed_optimizer_usage(dev):
    """The reference's DistributedOptimizer builds ``optimizer_cls([{"params": owned}],
    **kwargs)`` and its zero_grad sets every gradient to None
    (parallel/distributed_optimizer.py:26-35), so backward hands a flat-buffer optimizer
    freshly allocated gradients, and on some steps a parameter has none.  Fresh
    gradients are copied into the buffer; a group with a missing gradient is stepped
    tensor by tensor, its clip norm over the gradients present; parameters, moments,
    step counts and bf16 copies stay bit-identical to torch."""
    import mi_adamw
    shapes = [(64, 48), (48,), (128, 64), (64,), (7, 5)]
    ref = make_params(shapes, dev)
    ours = clone_params(ref)
    hp = dict(lr=6e-4, weight_decay=0.1, fused=False)
    topt = torch.optim.AdamW([{"params": ref}], **hp)
    oopt = mi_adamw.AdamW([{"params": ours}], **hp, flat_buffer=True, max_grad_norm=1.0,
                          bf16_copy=True)
    g = gen(dev, 21)
    for step in range(6):
        for p, q in zip(ref, ours):
            p.grad = None
            q.grad = None
        skip = {1, 4} if step in (2, 3) else set()
        for i, (p, q) in enumerate(zip(ref, ours)):
            if i not in skip:
                p.grad = torch.randn(p.shape, device=dev, generator=g) * 1e-2
                q.grad = p.grad.clone()          # allocated outside the flat buffer
        oopt.step()
        present = [p for p in ref if p.grad is not None]
        want = torch.nn.utils.get_total_norm([p.grad for p in present])
        assert abs(oopt.last_grad_norm.item() - want.item()) <= 1e-6 * want.item()
        torch.nn.utils.clip_grads_with_norm_(present, 1.0, oopt.last_grad_norm.clone())
        topt.step()
        torch.cuda.synchronize()
        assert max_ulp_all(ref, ours) == 0
        for i, q in enumerate(ours):
            if i not in skip:
                assert oopt._flat.is_grad_view(q, q.grad)
    for p, q in zip(ref, ours):
        ts, os_ = topt.state[p], oopt.state[q]
        assert float(ts["step"]) == float(os_["step"])
        assert max_ulp(ts["exp_avg"], os_["exp_avg"]) == 0
        assert max_ulp(ts["exp_avg_sq"], os_["exp_avg_sq"]) == 0
        assert torch.equal(oopt.bf16_param(q), q.detach().to(torch.bfloat16))
    assert float(oopt.state[ours[1]]["step"]) == 4.0
