"""Write the golden fixtures of torch's fused=True AdamW chain (tests/golden/fused_golden.npz).

Needs a ROCm GPU: torch's fused AdamW (``torch.optim.AdamW(fused=True)`` ->
``torch._fused_adamw_``, adam.py:803-895) runs only on the device, and its CPU
implementation is different arithmetic.  The values written are torch 2.10.0+rocm7.0's
own results on an MI355X; the CPU tests pin the oracle's restatement of that chain
(oracle.adamw_step_fused) against them.

Three kinds of case:
- the discriminating inputs of tests/golden/fused_cases.txt (written by fused_cases.c):
  (m, g) and (v, g) pairs on which the candidate fused multiply-add forms of the
  float64 moment updates round apart; one fused step at lr 3e-4, betas (0.9, 0.95),
  weight decay 0.1, eps 1e-8, step 1000, storing exp_avg or exp_avg_sq;
- seeded whole chains of 1024 elements, one fused step each, over the options: first
  step from zero state, other betas, maximize, no weight decay, amsgrad, a device lr,
  a late step, lr 0, moments so small that eps dominates the denominator; and three
  chained steps with fresh gradients;
- per-step values: (lr, step, betas) where the candidate forms of the per-step values
  round apart (step_size = f32(lr / f32(bc1)) against f32(lr / bc1), bc2_sqrt =
  f32(sqrt(bc2)) against sqrtf(f32(bc2))), found on the host (scalar_cases), each
  stepped on eight elements from p = 0 with no gradient and no weight decay, so that
  p is the update itself and shows both values.

Run from the repository root on a machine with a ROCm GPU:
    python tests/golden/make_fused_golden.py [OUT]       (default: beside this file)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = os.path.join(HERE, "fused_cases.txt")
N = 1024
HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)

# name -> overrides of HP and options, for the one-step whole-chain cases
RUNS = {
    "step1": dict(step=1, zero_state=True),
    "betas_0.9_0.999": dict(step=3, betas=(0.9, 0.999)),
    "beta1_0.3": dict(step=50, betas=(0.3, 0.95)),
    "mid": dict(step=1000),
    "maximize": dict(step=1000, maximize=True),
    "no_wd": dict(step=7, weight_decay=0.0),
    "amsgrad": dict(step=1000, amsgrad=True),
    "lr_device": dict(step=2, lr_device=7e-4),
    "late": dict(step=123456),
    "lr0": dict(step=1000, lr=0.0),
    "tiny_moments": dict(step=1000, tiny=True),
}


def scalar_cases(k: int = 16) -> list[tuple[float, float, float, float]]:
    """(lr, step, beta1, beta2) where f32(lr / bc1) != f32(lr / f32(bc1)), then where
    f32(sqrt(bc2)) != sqrtf(f32(bc2)); k of each, in a fixed search order."""
    f32 = np.float32
    bc1_cases, bc2_cases = [], []
    for step in range(1, 400):
        for b1, b2 in ((0.9, 0.95), (0.9, 0.999), (0.8, 0.99)):
            b1c, b2c = 1 - b1 ** step, 1 - b2 ** step
            for lr in (3e-4, 6e-4, 1e-3, 2.5e-4, 7e-5):
                if len(bc1_cases) < k and f32(lr / b1c) != f32(lr / float(f32(b1c))):
                    bc1_cases.append((lr, float(step), b1, b2))
            if len(bc2_cases) < k and f32(b2c ** 0.5) != np.sqrt(f32(b2c)):
                bc2_cases.append((3e-4, float(step), b1, b2))
    return bc1_cases + bc2_cases


def fused_step(p, g, m, v, step, *, lr, betas, eps, weight_decay, maximize=False, vmax=None):
    st = torch.tensor(float(step), dtype=torch.float32, device=p.device)
    torch._fused_adamw_([p], [g], [m], [v], [vmax] if vmax is not None else [], [st], lr=lr,
                        beta1=betas[0], beta2=betas[1], weight_decay=weight_decay, eps=eps,
                        maximize=maximize, amsgrad=vmax is not None, grad_scale=None,
                        found_inf=None)


def main(out_path: str) -> None:
    dev = torch.device("cuda", 0)
    out: dict[str, np.ndarray] = {}
    rows = [line.split() for line in open(CASES) if line.strip()]
    for kind in ("m", "v"):
        sel = [r for r in rows if r[0][0] == kind]
        x = np.array([float.fromhex(r[1]) for r in sel], dtype=np.float32)
        g = np.array([float.fromhex(r[2]) for r in sel], dtype=np.float32)
        pair = np.array([int(r[0][1:]) for r in sel], dtype=np.int32)
        zeros = torch.zeros(len(sel), device=dev)
        p = torch.full((len(sel),), 0.01, device=dev)
        xt, gt = torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev)
        m, v = (xt.clone(), zeros.clone()) if kind == "m" else (zeros.clone(), xt.clone())
        fused_step(p, gt, m, v, 1000, **HP)
        out[f"case_{kind}_in"] = x
        out[f"case_{kind}_g"] = g
        out[f"case_{kind}_pair"] = pair
        out[f"case_{kind}_out"] = (m if kind == "m" else v).cpu().numpy()
    rng = np.random.default_rng(20261202)
    for name, r in RUNS.items():
        hp = dict(HP)
        hp.update({k: r[k] for k in ("betas", "weight_decay", "lr") if k in r})
        p = (rng.standard_normal(N) * 0.02).astype(np.float32)
        g = (rng.standard_normal(N) * 1e-3).astype(np.float32)
        if r.get("zero_state"):
            m = np.zeros(N, np.float32)
            v = np.zeros(N, np.float32)
        elif r.get("tiny"):
            g = (rng.standard_normal(N) * 1e-9).astype(np.float32)
            m = (rng.standard_normal(N) * 1e-9).astype(np.float32)
            v = np.abs(rng.standard_normal(N) * 1e-17).astype(np.float32)
        else:
            m = (rng.standard_normal(N) * 1e-3).astype(np.float32)
            v = np.abs(rng.standard_normal(N) * 1e-6).astype(np.float32)
        x = (v * np.float32(1.5)).astype(np.float32)
        x[::2] = 0
        for k, a in (("p", p), ("g", g), ("m", m), ("v", v)):
            out[f"run_{name}_{k}_in"] = a
        t = {k: torch.from_numpy(a.copy()).to(dev) for k, a in (("p", p), ("g", g), ("m", m),
                                                                 ("v", v), ("x", x))}
        vmax = None
        if r.get("amsgrad"):
            out[f"run_{name}_x_in"] = x
            vmax = t["x"]
        if "lr_device" in r:
            hp["lr"] = torch.tensor(r["lr_device"], dtype=torch.float32, device=dev)
            out[f"run_{name}_lr"] = np.float32(r["lr_device"])
        fused_step(t["p"], t["g"], t["m"], t["v"], r["step"], maximize=r.get("maximize", False),
                   vmax=vmax, **hp)
        out[f"run_{name}_step"] = np.float32(r["step"])
        for k in ("p", "m", "v") + (("x",) if vmax is not None else ()):
            out[f"run_{name}_{k}_out"] = t[k].cpu().numpy()
    # three chained steps, steps 998-1000, fresh gradients each step
    p = (rng.standard_normal(N) * 0.02).astype(np.float32)
    m = (rng.standard_normal(N) * 1e-3).astype(np.float32)
    v = np.abs(rng.standard_normal(N) * 1e-6).astype(np.float32)
    gs = (rng.standard_normal((3, N)) * 1e-2).astype(np.float32)
    out.update(chain_p_in=p, chain_m_in=m, chain_v_in=v, chain_g=gs)
    t = [torch.from_numpy(a.copy()).to(dev) for a in (p, m, v)]
    for k in range(3):
        fused_step(t[0], torch.from_numpy(gs[k]).to(dev), t[1], t[2], 998 + k, **HP)
    out.update(chain_p_out=t[0].cpu().numpy(), chain_m_out=t[1].cpu().numpy(),
               chain_v_out=t[2].cpu().numpy())
    cases = scalar_cases()
    sp = []
    for lr, step, b1, b2 in cases:
        t = [torch.full((8,), x, device=dev) for x in (0.0, 0.0, 0.01, 1e-4)]
        fused_step(t[0], t[1], t[2], t[3], step, lr=lr, betas=(b1, b2), eps=1e-8,
                   weight_decay=0.0)
        sp.append(t[0].cpu().numpy())
    out["scalar_cases"] = np.array(cases, dtype=np.float64)
    out["scalar_p_out"] = np.stack(sp)
    out["torch_version"] = np.array(torch.__version__)
    np.savez(out_path, **out)
    print(f"wrote {out_path}: {len(out)} arrays", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "fused_golden.npz"))
