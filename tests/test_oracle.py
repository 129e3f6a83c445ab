"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

* Golden fixtures from torch's CPU AdamW(foreach=False) and clip_grad_norm_
  (tests/golden/make_golden.py).  The oracle's CPU op model reproduces m and v
  bit for bit.  p differs only through torch's vectorised CPU sqrt, which is
  not always correctly rounded (the oracle's is): one ulp of sqrt moves an
  update by 2^-23 of itself, so p agrees to 2^-22 per step of the tensor's
  scale, |dp| <= steps 2^-22 (|p| + rms(p)).
* Closed forms: lr = 0 leaves p bitwise unchanged; the first step from zero
  state gives m = f32(0.1 g) and p1 ~ p0 (1 - lr wd) - lr sign(g); g = 0 decays
  m and v and weight decay alone moves p; wd = 0 leaves the first op out;
  constant gradients have norm |c| sqrt(N); clip coefficient 1 below max_norm.
* A float64 restatement of the same chain on small inputs bounds the fp32
  result (a dropped term, a wrong sign or a swapped operand fails it).
* bf16 rounding against torch's own Tensor.to(torch.bfloat16) over every
  rounding-boundary class.
* torch's fused=True chain (oracle.adamw_step_fused): golden fixtures written by
  torch's own GPU kernel (tests/golden/make_fused_golden.py), including inputs on
  which the candidate fused multiply-add forms round apart (each other form is
  rejected by them); closed forms (lr = 0, g = 0, the first step); a float64 bound;
  and its agreement with the default chain to a few ulp.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "adamw_golden.npz")
N_SHAPES = 4


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _run_golden(gold, name, opmodel):
    lr, b1, b2, eps, wd, steps, maximize, clip, start, amsgrad = gold[f"{name}/meta"]
    steps, start, amsgrad = int(steps), int(start), bool(amsgrad)
    out = []
    for i in range(N_SHAPES):
        p = gold[f"{name}/p0/{i}"].reshape(-1).copy()
        if start:
            m = gold[f"{name}/m0/{i}"].reshape(-1).copy()
            v = gold[f"{name}/v0/{i}"].reshape(-1).copy()
        else:
            m = np.zeros_like(p)
            v = np.zeros_like(p)
        vmax = None
        if amsgrad:
            vmax = gold[f"{name}/vmax0/{i}"].reshape(-1).copy() if start else np.zeros_like(p)
        out.append([p, m, v, vmax])
    norms = []
    for t in range(steps):
        grads = [gold[f"{name}/g/{t}/{i}"].reshape(-1) for i in range(N_SHAPES)]
        scale = None
        if clip > 0:
            # The update is pinned given torch's own norm (stored in the fixture);
            # the oracle's float64 norm is compared with it separately.
            norms.append(O.total_norm(grads))
            scale = O.clip_coef(gold[f"{name}/norms"][t], clip)
        for i in range(N_SHAPES):
            p, m, v, vmax = out[i]
            O.adamw_step(p, grads[i].copy(), m, v, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd,
                         step=float(start + t + 1), maximize=bool(maximize), grad_scale=scale,
                         vmax=vmax, opmodel=opmodel)
    return out, norms


GOLDEN_CASES = ["step1_zero", "chain10_refcfg", "midtrain_clip", "small_norm_clip", "lerp_big",
                "maximize", "wd0", "lr0", "amsgrad_decay", "amsgrad_mid_clip"]


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_oracle_matches_torch_cpu_golden(gold, name):
    out, norms = _run_golden(gold, name, O.OPMODEL_TORCH_CPU)
    steps = int(gold[f"{name}/meta"][5])
    for i, (p, m, v, vmax) in enumerate(out):
        assert O.max_ulp(m, gold[f"{name}/m/{i}"].reshape(-1))[0] == 0
        assert O.max_ulp(v, gold[f"{name}/v/{i}"].reshape(-1))[0] == 0
        if vmax is not None:
            assert O.max_ulp(vmax, gold[f"{name}/vmax/{i}"].reshape(-1))[0] == 0
        pr = gold[f"{name}/p/{i}"].reshape(-1).astype(np.float64)
        tol = steps * 2.0 ** -22 * (np.abs(pr) + np.sqrt(np.mean(pr ** 2)))
        assert np.all(np.abs(p - pr) <= tol)
    if norms:
        ref = gold[f"{name}/norms"]
        for ours, theirs in zip(norms, ref):
            assert abs(float(ours) - float(theirs)) <= 1e-6 * float(theirs)


def test_opmodels_differ_where_expected(gold):
    """The ROCm op model is a different rounding pattern, but only by ulps."""
    cpu, _ = _run_golden(gold, "chain10_refcfg", O.OPMODEL_TORCH_CPU)
    gpu, _ = _run_golden(gold, "chain10_refcfg", O.OPMODEL_TORCH_ROCM)
    differs = False
    for (pc, mc, vc, _), (pg, mg, vg, _) in zip(cpu, gpu):
        for a, b in ((pc, pg), (mc, mg), (vc, vg)):
            a64, b64 = a.astype(np.float64), b.astype(np.float64)
            tol = 10 * 2.0 ** -21 * (np.abs(b64) + np.sqrt(np.mean(b64 ** 2)))
            assert np.all(np.abs(a64 - b64) <= tol)
            differs |= O.max_ulp(a, b)[0] > 0
    assert differs


def test_golden_clip_cases(gold):
    clipped = 0
    for c in range(4):
        grads = [gold[f"clip{c}/g/{i}"].reshape(-1) for i in range(N_SHAPES)]
        norm = O.total_norm(grads)
        ref = float(gold[f"clip{c}/norm"])
        assert abs(float(norm) - ref) <= 1e-6 * ref
        coef = O.clip_coef(np.float32(ref), float(gold[f"clip{c}/max_norm"]))
        clipped += coef < 1
        for i in range(N_SHAPES):
            # torch multiplies by the clamped coefficient even when it is 1.
            assert np.array_equal((grads[i] * coef).astype(np.float32),
                                  gold[f"clip{c}/gc/{i}"].reshape(-1))
    assert clipped == 3   # the cases exercise the scale, not only the clamp


def _rand(n, seed, std):
    return (np.random.default_rng(seed).standard_normal(n) * std).astype(np.float32)


@pytest.mark.parametrize("opmodel", [O.OPMODEL_TORCH_CPU, O.OPMODEL_TORCH_ROCM])
def test_lr_zero_leaves_params_unchanged(opmodel):
    p0 = _rand(4096, 1, 0.02)
    p = p0.copy()
    g = _rand(4096, 2, 1e-3)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    O.adamw_step(p, g, m, v, lr=0.0, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, step=1,
                 opmodel=opmodel)
    assert np.array_equal(p.view(np.uint32), p0.view(np.uint32))
    assert np.array_equal(m, (np.float32(0.1) * g).astype(np.float32))


@pytest.mark.parametrize("opmodel", [O.OPMODEL_TORCH_CPU, O.OPMODEL_TORCH_ROCM])
def test_first_step_closed_form(opmodel):
    n = 8192
    p0 = _rand(n, 3, 0.02)
    g = _rand(n, 4, 1e-3)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    lr, wd = 3e-4, 0.1
    O.adamw_step(p, g, m, v, lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd, step=1,
                 opmodel=opmodel)
    # m = lerp(0, g, 0.1) = f32(0.1 g); v = f32(f32(0.05) f32(g g)).
    assert np.array_equal(m, (np.float32(1 - 0.9) * g).astype(np.float32))
    v_cf = (np.float32(1 - 0.95) * (g * g).astype(np.float32)).astype(np.float32)
    assert O.max_ulp(v, v_cf)[0] <= 2   # two roundings, fused in either order
    # Bias-corrected m / sqrt(v) = g / (|g| + eps): p1 = p0 (1 - lr wd) - lr g / (|g| + eps),
    # up to a few fp32 roundings of the scalars and of p.
    g64 = g.astype(np.float64)
    expect = p0.astype(np.float64) * (1 - lr * wd) - lr * g64 / (np.abs(g64) + 1e-8)
    assert np.all(np.abs(p - expect) <= 2.0 ** -22 * (np.abs(expect) + lr))


def test_zero_grad_decays_state():
    n = 2048
    p0 = _rand(n, 5, 0.02)
    m0 = _rand(n, 6, 1e-3)
    v0 = np.abs(_rand(n, 7, 1e-6))
    p, m, v = p0.copy(), m0.copy(), v0.copy()
    g = np.zeros(n, np.float32)
    lr, wd, b1, b2 = 3e-4, 0.1, 0.9, 0.95
    O.adamw_step(p, g, m, v, lr=lr, betas=(b1, b2), eps=1e-8, weight_decay=wd, step=1000,
                 opmodel=O.OPMODEL_TORCH_ROCM)
    assert O.max_ulp(m, (m0.astype(np.float64) * b1).astype(np.float32))[0] <= 1
    assert np.array_equal(v, (v0 * np.float32(b2)).astype(np.float32))
    d = np.sqrt(v.astype(np.float64)) / (1 - b2 ** 1000) ** 0.5 + 1e-8
    ss = lr / (1 - b1 ** 1000)
    expect = p0.astype(np.float64) * (1 - lr * wd) - ss * m / d
    # Rounding of p, plus the update's own few roundings (relative to the update,
    # which is ss m / d; the decayed parameter may cancel it).
    assert np.all(np.abs(p - expect) <= 2.0 ** -22 * np.abs(expect) + 2.0 ** -20 * ss * np.abs(m) / d)


def test_weight_decay_zero_is_identity_on_first_op():
    n = 1024
    p0 = _rand(n, 8, 0.02)
    g = _rand(n, 9, 1e-3)
    p_a, p_b = p0.copy(), p0.copy()
    for p, wd in ((p_a, 0.0), (p_b, 1e-30)):
        O.adamw_step(p, g.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32), lr=3e-4,
                     betas=(0.9, 0.95), eps=1e-8, weight_decay=wd, step=1)
    # f32(1 - 3e-4 * 1e-30) == 1.0f, so a vanishing decay equals no decay.
    assert np.array_equal(p_a, p_b)


def _float64_chain(p, g, m, v, lr, b1, b2, eps, wd, step):
    p, g, m, v = (x.astype(np.float64) for x in (p, g, m, v))
    p = p * (1 - lr * wd)
    m = m + (1 - b1) * (g - m)
    v = v * b2 + (1 - b2) * g * g
    d = np.sqrt(v) / np.sqrt(1 - b2 ** step) + eps
    p = p - lr / (1 - b1 ** step) * m / d
    return p, m, v


@pytest.mark.parametrize("opmodel", [O.OPMODEL_TORCH_CPU, O.OPMODEL_TORCH_ROCM])
@pytest.mark.parametrize("step,b1,b2", [(1, 0.9, 0.95), (7, 0.9, 0.999), (1000, 0.9, 0.95),
                                        (3, 0.3, 0.95)])
def test_float64_bound(opmodel, step, b1, b2):
    n = 1000
    p0, g = _rand(n, 10, 0.02), _rand(n, 11, 1e-3)
    m0, v0 = _rand(n, 12, 1e-3), np.abs(_rand(n, 13, 1e-6))
    p, m, v = p0.copy(), m0.copy(), v0.copy()
    lr, wd, eps = 6e-4, 0.1, 1e-8
    O.adamw_step(p, g.copy(), m, v, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, step=step,
                 opmodel=opmodel)
    p64, m64, v64 = _float64_chain(p0, g, m0, v0, lr, b1, b2, eps, wd, step)
    assert np.max(np.abs(m - m64) / (np.abs(m64) + np.abs(m0) + 1e-30)) <= 4 * 2.0 ** -24
    assert np.max(np.abs(v - v64) / v64) <= 4 * 2.0 ** -24
    # p: rounding of p itself, plus a few roundings of the update ss m / d, where
    # m carries an absolute error of order 2^-24 (|m0| + |g|) even when it
    # cancels to near zero.
    ss = lr / (1 - b1 ** step)
    d64 = np.sqrt(v64) / np.sqrt(1 - b2 ** step) + eps
    bound = (np.abs(p64) * 2.0 ** -23
             + 2.0 ** -20 * ss * (np.abs(m0) + np.abs(g) + np.abs(m64)) / d64)
    assert np.all(np.abs(p - p64) <= bound)


def test_capt_lr_zero_leaves_params_unchanged():
    """Capturable chain, lr 0: step_size is 0, both denominator terms are -inf and
    the update m / d is a signed zero."""
    p0 = _rand(4096, 21, 0.02)
    p = p0.copy()
    g = _rand(4096, 22, 1e-3)
    m, v = np.zeros_like(p), np.zeros_like(p)
    O.adamw_step_capt(p, g, m, v, lr=0.0, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1,
                      step=1)
    assert np.array_equal(p.view(np.uint32), p0.view(np.uint32))
    assert np.array_equal(m, (np.float32(0.1) * g).astype(np.float32))


@pytest.mark.parametrize("lr_is_tensor", [False, True])
def test_capt_first_step_closed_form(lr_is_tensor):
    """Capturable chain, step 1 from zero state: powf(beta, 1) is beta, and
    m / (sqrt(v) / (sqrt(bc2) * -step_size) + eps / -step_size) is
    -lr g / (|g| + eps), the same first step as the default chain."""
    n = 8192
    p0 = _rand(n, 23, 0.02)
    g = _rand(n, 24, 1e-3)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    lr, wd = 3e-4, 0.1
    O.adamw_step_capt(p, g, m, v, lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd, step=1,
                      lr_is_tensor=lr_is_tensor)
    assert np.array_equal(m, (np.float32(1 - 0.9) * g).astype(np.float32))
    g64 = g.astype(np.float64)
    expect = p0.astype(np.float64) * (1 - lr * wd) - lr * g64 / (np.abs(g64) + 1e-8)
    # about eight fp32 roundings reach the update (the two per-step values, sqrt,
    # two divisions, the add, the final add): 2^-21 of lr, plus p's own rounding
    assert np.all(np.abs(p - expect) <= 2.0 ** -21 * (np.abs(expect) + lr))
    a, e = O.capt_scalars(lr, 0.9, 0.95, 1e-8, 1.0, lr_is_tensor)
    assert abs(a - (-np.sqrt(0.05) * lr / 0.1)) <= 4 * 2.0 ** -24 * abs(a)
    assert abs(e - (-1e-8 * 0.1 / lr)) <= 4 * 2.0 ** -24 * abs(e)


@pytest.mark.parametrize("step,b1,b2,lr_is_tensor,amsgrad", [
    (1, 0.9, 0.95, False, False), (7, 0.9, 0.999, False, True), (1000, 0.9, 0.95, True, False),
    (3, 0.3, 0.95, False, False), (250, 0.8, 0.99, True, True)])
def test_capt_agrees_with_the_default_chain(step, b1, b2, lr_is_tensor, amsgrad):
    """The capturable and the default chain on the same inputs: m, v (and amsgrad's
    maximum) bit-identical, being the same ATen ops; the update u = p - p*(1-lr*wd)
    within the error analysis of the two ways of forming it.  The default chain's
    bias corrections are float64; the capturable chain's are fp32, and
    bc = 1 - beta**step cancels: one ulp of beta**step is a relative error of
    2^-23 * beta**step / bc in bc, which reaches u whole through bc1 and halved
    through sqrt(bc2).  Add 16 roundings for the ops of both chains.  The
    default chain is pinned by torch's golden vectors, so a dropped term, a sign
    or a swapped operand in the capturable one shows here."""
    n = 4096
    p0, g = _rand(n, 25, 0.02), _rand(n, 26, 1e-3)
    m0, v0 = _rand(n, 27, 1e-3), np.abs(_rand(n, 28, 1e-6))
    x0 = v0 * np.float32(1.5)
    lr, wd, eps = 6e-4, 0.1, 1e-8
    out = []
    for capt in (False, True):
        p, m, v = p0.copy(), m0.copy(), v0.copy()
        x = x0.copy() if amsgrad else None
        kw = dict(lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, step=step, vmax=x)
        if capt:
            O.adamw_step_capt(p, g.copy(), m, v, lr_is_tensor=lr_is_tensor, **kw)
        else:
            O.adamw_step(p, g.copy(), m, v, **kw)
        out.append((p, m, v, x))
    (pa, ma, va, xa), (pb, mb, vb, xb) = out
    assert np.array_equal(ma, mb) and np.array_equal(va, vb)
    if amsgrad:
        assert np.array_equal(xa, xb)
    pd = np.float32(p0 * np.float32(1 - lr * wd)).astype(np.float64)   # decayed p, both chains
    ua, ub = pa - pd, pb - pd
    bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
    rel = 2.0 ** -24 * (16 + 2 * b1 ** step / bc1 + b2 ** step / bc2)
    # each chain's final rounding of p adds up to half an ulp of p
    assert np.all(np.abs(ua - ub) <= rel * np.abs(ua) + 2.0 ** -24 * (np.abs(pa) + np.abs(pb)))


def test_clip_closed_forms():
    # Constant gradients: norm = |c| sqrt(N), exactly representable here.
    grads = [np.full(1024, 0.5, np.float32), np.full(3072, 0.5, np.float32)]
    assert O.total_norm(grads) == np.float32(32.0)
    assert O.clip_coef(np.float32(32.0), 1.0) == np.float32(np.float32(1.0) / np.float32(32.000001))
    # Below max_norm the coefficient clamps to exactly 1.
    assert O.clip_coef(np.float32(0.25), 1.0) == np.float32(1.0)
    # Small norms: the 1e-6 is 16 ulp of 0.5, so coef = 0.25 / f32(0.500001) < 0.5.
    t = np.float32(np.float32(0.5) + np.float32(1e-6))
    assert t != np.float32(0.5)
    assert O.clip_coef(np.float32(0.5), 0.25) == np.float32(np.float32(1.0) / t) * np.float32(0.25)
    # NaN propagates through the clamp, as torch.clamp does.
    assert np.isnan(O.clip_coef(np.float32(np.nan), 1.0))
    # inf norm: 1/(inf) = 0 coefficient.
    assert O.clip_coef(np.float32(np.inf), 1.0) == 0.0


def test_sumsq_float64_brute_force():
    rng = np.random.default_rng(14)
    g = (rng.standard_normal(10007) * 1e-2).astype(np.float32)
    exact = float(np.sum(g.astype(np.float64) ** 2))
    assert abs(O.sumsq([g]) - exact) <= 1e-14 * exact
    assert abs(float(O.total_norm([g])) - exact ** 0.5) <= 2.0 ** -24 * exact ** 0.5


def test_bf16_rounding_matches_torch():
    # Every upper half with the lower halves around each rounding boundary.
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7fff, 0x8000, 0x8001, 0xffff], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).reshape(-1)
    x = bits.view(np.float32)
    ours = O.to_bf16_bits(x)
    theirs = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert np.all(ours[nan] == 0x7fc0)
    assert np.all(np.isnan(O.bf16_bits_to_f32(theirs[nan])))


def test_bf16state_with_exact_states_equals_fp32_then_round():
    """With moments that are already bf16 values, the bf16-state step is the fp32 step
    followed by RNE of m and v (the fp32 math in between is identical)."""
    n = 4096
    p0, g = _rand(n, 15, 0.02), _rand(n, 16, 1e-3)
    m0 = O.bf16_bits_to_f32(O.to_bf16_bits(_rand(n, 17, 1e-3)))
    v0 = O.bf16_bits_to_f32(O.to_bf16_bits(np.abs(_rand(n, 18, 1e-6))))
    pa, ma, va = p0.copy(), m0.copy(), v0.copy()
    O.adamw_step(pa, g.copy(), ma, va, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                 step=1000)
    pb = p0.copy()
    mb, vb = O.to_bf16_bits(m0), O.to_bf16_bits(v0)
    O.adamw_step_bf16state(pb, g.copy(), mb, vb, lr=3e-4, betas=(0.9, 0.95), eps=1e-8,
                           weight_decay=0.1, step=1000)
    assert np.array_equal(pa, pb)
    assert np.array_equal(O.to_bf16_bits(ma), mb)
    assert np.array_equal(O.to_bf16_bits(va), vb)


def test_oracle_is_deterministic():
    n = 5000
    runs = []
    for _ in range(2):
        p, g = _rand(n, 19, 0.02), _rand(n, 20, 1e-3)
        m, v = _rand(n, 21, 1e-3), np.abs(_rand(n, 22, 1e-6))
        O.adamw_step(p, g, m, v, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, step=5)
        runs.append((p, m, v))
    for a, b in zip(*runs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------------------
# torch's fused=True chain (torch._fused_adamw_), pinned by its own GPU results

FUSED_GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "fused_golden.npz")
FUSED_HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
# the one-step cases of make_fused_golden.py: name -> overrides of FUSED_HP and options
FUSED_RUNS = {
    "step1": {}, "betas_0.9_0.999": dict(betas=(0.9, 0.999)), "beta1_0.3": dict(betas=(0.3, 0.95)),
    "mid": {}, "maximize": dict(maximize=True), "no_wd": dict(weight_decay=0.0),
    "amsgrad": {}, "lr_device": {}, "late": {}, "lr0": dict(lr=0.0), "tiny_moments": {},
}


@pytest.fixture(scope="module")
def fused_gold():
    with np.load(FUSED_GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(FUSED_RUNS))
def test_fused_chain_matches_torch_gpu_golden(fused_gold, name):
    gd = fused_gold
    kw = dict(FUSED_HP)
    kw.update({k: v for k, v in FUSED_RUNS[name].items() if k != "maximize"})
    if f"run_{name}_lr" in gd:
        kw["lr"] = float(gd[f"run_{name}_lr"])     # a device fp32 lr, read as float64
    p, g, m, v = (gd[f"run_{name}_{k}_in"].copy() for k in "pgmv")
    x = gd[f"run_{name}_x_in"].copy() if f"run_{name}_x_in" in gd else None
    O.adamw_step_fused(p, g, m, v, step=float(gd[f"run_{name}_step"]), vmax=x,
                       maximize=FUSED_RUNS[name].get("maximize", False), **kw)
    for k, a in (("p", p), ("m", m), ("v", v)) + ((("x", x),) if x is not None else ()):
        assert O.max_ulp(a, gd[f"run_{name}_{k}_out"])[0] == 0, k


def test_fused_chain_three_chained_steps_golden(fused_gold):
    gd = fused_gold
    p, m, v = (gd[f"chain_{k}_in"].copy() for k in "pmv")
    for k in range(3):
        O.adamw_step_fused(p, gd["chain_g"][k].copy(), m, v, step=998 + k, **FUSED_HP)
    for k, a in (("p", p), ("m", m), ("v", v)):
        assert O.max_ulp(a, gd[f"chain_{k}_out"])[0] == 0, k


def test_fused_per_step_values_golden(fused_gold):
    """At (lr, step, betas) where f32(lr / f32(bc1)) and f32(lr / bc1) differ, and where
    f32(sqrt(bc2)) and sqrtf(f32(bc2)) differ, torch's parameter after one step from 0
    (no gradient, no weight decay: p is the update) selects the oracle's forms."""
    gd = fused_gold
    for (lr, step, b1, b2), want in zip(gd["scalar_cases"], gd["scalar_p_out"]):
        p = np.zeros(8, np.float32)
        m = np.full(8, 0.01, np.float32)
        v = np.full(8, 1e-4, np.float32)
        O.adamw_step_fused(p, np.zeros(8, np.float32), m, v, lr=float(lr), betas=(b1, b2),
                           eps=1e-8, weight_decay=0.0, step=float(step))
        assert np.array_equal(p.view(np.uint32), want.view(np.uint32)), (lr, step, b1, b2)


def _fused_cases(gd, kind, model):
    x, g = gd[f"case_{kind}_in"].copy(), gd[f"case_{kind}_g"].copy()
    n = x.size
    p = np.full(n, 0.01, np.float32)
    z = np.zeros(n, np.float32)
    m, v = (x, z.copy()) if kind == "m" else (z.copy(), x)
    O.adamw_step_fused(p, g, m, v, step=1000, model=model, **FUSED_HP)
    return (m if kind == "m" else v), gd[f"case_{kind}_out"]


def test_fused_contraction_forms_are_pinned(fused_gold):
    """On the inputs where the forms round apart, torch's kernel selects the left-product
    fused multiply-add for both moments; the unfused and the right-product forms each
    disagree with it on at least one input."""
    pinned = O.FUSED_TORCH_ROCM
    for kind in ("m", "v"):
        got, want = _fused_cases(fused_gold, kind, pinned)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), kind
        for mode in (0, 2):
            other = O.FusedModel(wd_fma=1, m_mode=mode if kind == "m" else 1,
                                 v_mode=mode if kind == "v" else 1)
            got, want = _fused_cases(fused_gold, kind, other)
            assert not np.array_equal(got.view(np.uint32), want.view(np.uint32)), (kind, mode)


def test_fused_lr_zero_and_zero_grad_closed_forms():
    """lr = 0 leaves p bitwise unchanged (lr*wd = 0 and step_size = 0); g = 0 multiplies m
    and v by beta1 and beta2 in float64 with one rounding to fp32."""
    n = 4096
    p0, m0, v0 = _rand(n, 21, 0.02), _rand(n, 22, 1e-3), np.abs(_rand(n, 23, 1e-6))
    p, m, v = p0.copy(), m0.copy(), v0.copy()
    O.adamw_step_fused(p, np.zeros(n, np.float32), m, v, lr=0.0, betas=(0.9, 0.95), eps=1e-8,
                       weight_decay=0.1, step=1000)
    assert np.array_equal(p.view(np.uint32), p0.view(np.uint32))
    assert np.array_equal(m, (m0.astype(np.float64) * 0.9).astype(np.float32))
    assert np.array_equal(v, (v0.astype(np.float64) * 0.95).astype(np.float32))


def test_fused_first_step_closed_form():
    """From zero state at step 1: m = f32((1 - beta1) g) with 1 - beta1 in float64,
    v = f32((1 - beta2) g^2), and the bias-corrected update is lr * sign(g) up to eps."""
    n = 8192
    p0, g = _rand(n, 24, 0.02), _rand(n, 25, 1e-3)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    lr, wd = 3e-4, 0.1
    O.adamw_step_fused(p, g, m, v, lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd, step=1)
    g64 = g.astype(np.float64)
    assert np.array_equal(m, ((1 - 0.9) * g64).astype(np.float32))
    assert O.max_ulp(v, ((1 - 0.95) * g64 * g64).astype(np.float32))[0] <= 1
    expect = p0.astype(np.float64) * (1 - lr * wd) - lr * g64 / (np.abs(g64) + 1e-8)
    assert np.all(np.abs(p - expect) <= 2.0 ** -21 * (np.abs(expect) + lr))


@pytest.mark.parametrize("step,b1,b2", [(1, 0.9, 0.95), (7, 0.9, 0.999), (1000, 0.9, 0.95),
                                        (3, 0.3, 0.95)])
def test_fused_float64_bound(step, b1, b2):
    """The fused chain against the whole step in float64: m and v within two fp32
    roundings, p within the rounding of p plus a few roundings of the update."""
    n = 1000
    p0, g = _rand(n, 26, 0.02), _rand(n, 27, 1e-3)
    m0, v0 = _rand(n, 28, 1e-3), np.abs(_rand(n, 29, 1e-6))
    p, m, v = p0.copy(), m0.copy(), v0.copy()
    lr, wd, eps = 6e-4, 0.1, 1e-8
    O.adamw_step_fused(p, g.copy(), m, v, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd,
                       step=step)
    p64, m64, v64 = _float64_chain(p0, g, m0, v0, lr, b1, b2, eps, wd, step)
    assert np.max(np.abs(m - m64) / (np.abs(m64) + np.abs(m0) + 1e-30)) <= 2 * 2.0 ** -24
    assert np.max(np.abs(v - v64) / v64) <= 2 * 2.0 ** -24
    ss = lr / (1 - b1 ** step)
    d64 = np.sqrt(v64) / np.sqrt(1 - b2 ** step) + eps
    bound = (np.abs(p64) * 2.0 ** -23
             + 2.0 ** -20 * ss * (np.abs(m0) + np.abs(g) + np.abs(m64)) / d64)
    assert np.all(np.abs(p - p64) <= bound)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_fused_chain_agrees_with_the_default_chain(amsgrad):
    """Both chains round the same real step: m within a few roundings of its operands'
    scale (0.9 m + 0.1 g may cancel), v within 2 ulp, p within a few roundings of the
    update (the running maximum of v taken in both)."""
    n = 4096
    p0, g = _rand(n, 30, 0.02), _rand(n, 31, 1e-3)
    m0, v0 = _rand(n, 32, 1e-3), np.abs(_rand(n, 33, 1e-6))
    x0 = (v0 * np.float32(1.5)).astype(np.float32)
    x0[::2] = 0
    out = []
    for fn in (O.adamw_step_fused, O.adamw_step):
        p, m, v, x = p0.copy(), m0.copy(), v0.copy(), x0.copy()
        fn(p, g.copy(), m, v, vmax=x if amsgrad else None, step=1000, **FUSED_HP)
        out.append((p, m, v, x))
    (pf, mf, vf, xf), (pd, md, vd, xd) = out
    assert np.all(np.abs(mf.astype(np.float64) - md) <= 2.0 ** -22 * (np.abs(m0) + np.abs(g)))
    assert O.max_ulp(vf, vd)[0] <= 2
    if amsgrad:
        assert O.max_ulp(xf, xd)[0] <= 2
    ss = FUSED_HP["lr"] / (1 - 0.9 ** 1000)
    upd = ss * np.abs(md.astype(np.float64)) / (np.sqrt(np.maximum(vd, xd if amsgrad else vd))
                                                 + 1e-8)
    assert np.all(np.abs(pf.astype(np.float64) - pd) <= 2.0 ** -22 * np.abs(pd) + 2.0 ** -20 *
                  (upd + ss * (np.abs(m0) + np.abs(g)) / (np.sqrt(vd) + 1e-8)))
