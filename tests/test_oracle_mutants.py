"""The oracle's pins catch planted mistakes (CPU only).

Each case compiles a copy of oracle/adamw_oracle.c with one plausible mistake
(a dropped term, a wrong sign, a swapped operand, a wrong constant, a missing
clamp, truncation instead of rounding, an off-by-one), points the oracle's
wrappers at it, and runs the pinning checks of tests/test_oracle.py: golden
fixtures from torch, closed forms, the float64 bound, bf16 rounding against
torch, the capturable chain's closed forms and its agreement with the default
chain, and the fused=True chain's GPU fixtures, contraction forms, closed forms,
float64 bound and agreement with the default chain.  At least one check must fail for every mutant; the unmodified
source compiled the same way must pass them all.
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import test_oracle as T
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCE = os.path.join(ROOT, "oracle", "adamw_oracle.c")

MUTANTS = {
    "no_weight_decay": ("float pp = *p * wd_factor;", "float pp = *p;"),
    "lerp_weight_beta1": ("lerp_f32(*m, g, lerp_w, om->lerp_fma)",
                          "lerp_f32(*m, g, 1.0f - lerp_w, om->lerp_fma)"),
    "update_sign": ("pp = om->addcdiv_mode == 1 ? fmaf(h->neg_step_size, q, pp) : pp + h->neg_step_size * q;",
                    "pp = om->addcdiv_mode == 1 ? fmaf(-h->neg_step_size, q, pp) : pp - h->neg_step_size * q;"),
    "no_bias_correction2": ("d = om->div_recip ? d * inv_bc2 : d / bc2f;", "d = d;"),
    "no_eps": ("d = d + h->eps;", "d = d;"),
    "m_v_swapped": ("float q = mm / d;", "float q = *v / d;"),
    "g_not_squared": ("vv = addcmul_f32(vv, omb2, g, om->addcmul_mode);",
                      "vv = vv + omb2 * fabsf(g);"),
    "beta2_swapped": ("float vv = *v * beta2;", "float vv = *v * omb2;"),
    "clip_not_clamped": ("return (c > 1.0f) ? 1.0f : c;", "return c;"),
    "clip_eps_dropped": ("float t = total_norm + (float)1e-6;", "float t = total_norm;"),
    "bf16_truncates": ("u += 0x7fffu + lsb;", "u += 0u * lsb;"),
    "sumsq_off_by_one": ("for (int64_t i = b; i < e; ++i) { double x = (double)g[i]; s += x * x; }",
                         "for (int64_t i = b; i + 1 < e; ++i) { double x = (double)g[i]; s += x * x; }"),
    "amsgrad_max_unused": ("        dv = *vmax;\n", "        (void)dv;\n"),
    "amsgrad_min": ("return a < b ? b : a;", "return a < b ? a : b;"),
    "grad_scale_ignored": ("if (apply_scale) gi = gi * grad_scale;\n        gi = gi * h->grad_sign;\n        adamw_elem(",
                           "gi = gi * h->grad_sign;\n        adamw_elem("),
    "capt_multiplies_by_den_scale": ("d = d / h->den_scale;", "d = d * h->den_scale;"),
    "capt_no_den_add": ("d = d + h->den_add;", "d = d;"),
    "capt_update_sign": ("*p = *p + *m / d;", "*p = *p - *m / d;"),
    "capt_no_bias_correction1": ("float step_size = lr_is_tensor ? lr / bc1 : (1.0f / bc1) * lr;",
                                 "float step_size = lr;"),
    "capt_eps_not_scaled": ("*den_add = (1.0f / neg) * eps;", "*den_add = eps;"),
    # torch's fused=True chain
    "fused_m_in_fp32": ("case 1: mm = (float)fma(h->beta1, dm, omb1 * dg); break;",
                        "case 1: mm = fmaf((float)h->beta1, *m, (float)omb1 * g); break;"),
    "fused_v_beta1": ("case 1: vv = (float)fma(h->beta2, dvv, q * dg); break;",
                      "case 1: vv = (float)fma(h->beta1, dvv, q * dg); break;"),
    "fused_eps_in_fp32": ("const float d = (float)((double)(sqrtf(dv) / h->bc2_sqrt) + h->eps);",
                          "const float d = sqrtf(dv) / h->bc2_sqrt + (float)h->eps;"),
    "fused_no_weight_decay": ("    if (h->weight_decay != 0.0) {\n        const double t",
                              "    if (0) {\n        const double t"),
    "fused_bc1_not_rounded": ("*step_size = (float)(lr / (double)*bc1);",
                              "*step_size = (float)(lr / b1c);"),
    "fused_amsgrad_max_unused": ("const float dv = vmax ? (*vmax = fmaxf(*vmax, vv)) : vv;",
                                 "const float dv = vmax ? (*vmax = fmaxf(*vmax, vv), vv) : vv;"),
    "fused_update_sign": ("pp = pp - (h->step_size * mm) / d;", "pp = pp + (h->step_size * mm) / d;"),
    "fused_bc2_sqrt_in_fp32": ("*bc2_sqrt = (float)sqrt(b2c);", "*bc2_sqrt = sqrtf((float)b2c);"),
}


def _checks(gold, fused_gold):
    """Every pinning check of test_oracle, as (name, callable) pairs."""
    out = []
    for name in T.GOLDEN_CASES:
        out.append((f"golden:{name}", lambda n=name: T.test_oracle_matches_torch_cpu_golden(gold, n)))
    out.append(("golden:clip", lambda: T.test_golden_clip_cases(gold)))
    for om in (O.OPMODEL_TORCH_CPU, O.OPMODEL_TORCH_ROCM):
        out.append(("lr_zero", lambda om=om: T.test_lr_zero_leaves_params_unchanged(om)))
        out.append(("first_step", lambda om=om: T.test_first_step_closed_form(om)))
        for step, b1, b2 in ((1, 0.9, 0.95), (7, 0.9, 0.999), (1000, 0.9, 0.95), (3, 0.3, 0.95)):
            out.append(("float64_bound",
                        lambda om=om, s=step, a=b1, b=b2: T.test_float64_bound(om, s, a, b)))
    out.append(("zero_grad", T.test_zero_grad_decays_state))
    out.append(("capt_lr_zero", T.test_capt_lr_zero_leaves_params_unchanged))
    for lt in (False, True):
        out.append(("capt_first_step", lambda lt=lt: T.test_capt_first_step_closed_form(lt)))
    for args in ((1, 0.9, 0.95, False, False), (7, 0.9, 0.999, False, True),
                 (1000, 0.9, 0.95, True, False), (250, 0.8, 0.99, True, True)):
        out.append(("capt_vs_default", lambda a=args: T.test_capt_agrees_with_the_default_chain(*a)))
    out.append(("clip_closed_forms", T.test_clip_closed_forms))
    out.append(("sumsq_brute_force", T.test_sumsq_float64_brute_force))
    out.append(("bf16_vs_torch", T.test_bf16_rounding_matches_torch))
    out.append(("bf16_state", T.test_bf16state_with_exact_states_equals_fp32_then_round))
    for name in T.FUSED_RUNS:
        out.append((f"fused_golden:{name}",
                    lambda n=name: T.test_fused_chain_matches_torch_gpu_golden(fused_gold, n)))
    out.append(("fused_golden:chain",
                lambda: T.test_fused_chain_three_chained_steps_golden(fused_gold)))
    out.append(("fused_forms", lambda: T.test_fused_contraction_forms_are_pinned(fused_gold)))
    out.append(("fused_per_step_values",
                lambda: T.test_fused_per_step_values_golden(fused_gold)))
    out.append(("fused_closed_forms", T.test_fused_lr_zero_and_zero_grad_closed_forms))
    out.append(("fused_first_step", T.test_fused_first_step_closed_form))
    for step, b1, b2 in ((1, 0.9, 0.95), (7, 0.9, 0.999), (1000, 0.9, 0.95), (3, 0.3, 0.95)):
        out.append(("fused_float64_bound",
                    lambda s=step, a=b1, b=b2: T.test_fused_float64_bound(s, a, b)))
    for ams in (False, True):
        out.append(("fused_vs_default",
                    lambda a=ams: T.test_fused_chain_agrees_with_the_default_chain(a)))
    return out


def _build(src_text: str, out_dir: str, name: str) -> str:
    c_path = os.path.join(out_dir, f"{name}.c")
    so_path = os.path.join(out_dir, f"lib{name}.so")
    with open(c_path, "w") as f:
        f.write(src_text)
    subprocess.run(["gcc", "-O2", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-std=c11",
                    "-I", os.path.dirname(SOURCE), "-shared", "-o", so_path, c_path, "-lm"],
                   check=True)
    return so_path


def _failures(gold, fused_gold, so_path: str) -> list[str]:
    O.use_library(so_path)
    failed = []
    try:
        for name, check in _checks(gold, fused_gold):
            try:
                check()
            except AssertionError:
                failed.append(name)
    finally:
        O.use_library(None)
    return failed


@pytest.fixture(scope="module")
def gold():
    with np.load(T.GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def fused_gold():
    with np.load(T.FUSED_GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_unmodified_copy_passes_every_check(gold, fused_gold, tmp_path):
    so = _build(open(SOURCE).read(), str(tmp_path), "oracle_copy")
    assert _failures(gold, fused_gold, so) == []


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_mutant_is_caught(gold, fused_gold, tmp_path, mutant):
    old, new = MUTANTS[mutant]
    src = open(SOURCE).read()
    assert src.count(old) == 1, f"mutation site for {mutant} not found exactly once"
    so = _build(src.replace(old, new), str(tmp_path), f"oracle_{mutant}")
    failed = _failures(gold, fused_gold, so)
    print(f"{mutant}: caught by {failed}")
    assert failed, f"planted mistake {mutant} passed every pinning check"
