#!/usr/bin/env python3
"""Benchmark of the fused clip + AdamW optimizer step on one MI355X.

A step is one ``FusedAdamW.step()`` over a GPT parameter set whose params,
grads and moments are already resident in HBM: the grad-norm pass (with
clipping) and the AdamW update, exactly what mini-megatron's training loop
runs at main.py:209.  Gradients are generated once before the timed region;
the step only reads them (the clip scale is applied in registers), so every
timed step does the full work.

Default workload (one GPU): gpt-125m, fp32 params/grads/moments, global
grad-norm clip at 1.0 fused ahead of AdamW, optimizer state mid-training
(step 1000), lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight decay 0.1.

Output: one JSON line.  ``value`` is the achieved HBM bandwidth of the whole
step in GB/s, from algorithmic bytes (every byte the step must read or write,
counted once) over the measured step time.  ``roofline`` reports the update
kernel against MI355X's 8 TB/s, timed with HIP events on the launch stream.
``cpu_baseline`` times the reference's own CPU path (torch.optim.AdamW with
foreach=False, after clip_grad_norm_) on the host's cores.

    python bench.py [--steps K] [--warmup W] [--config NAME | --config all]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mini-megatron_amd"))

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0   # MI355X published HBM3E bandwidth
METRIC = "AdamW step ms + achieved HBM GB/s (% of MI355X peak), 125M→6.7B"

# name: (shape, clip, state dtype, bf16 copy, flat buffer, stored step, grad std)
CONFIGS = {
    "125m-step1": ("gpt-125m", False, "fp32", False, False, 0, 1e-3),
    "125m-clip": ("gpt-125m", True, "fp32", False, False, 1000, 1e-2),
    "350m-master-clip-copy": ("gpt-350m", True, "fp32", True, False, 1000, 1e-3),
    "1.3b-bf16state-copy": ("gpt-1.3b", False, "bf16", True, False, 1000, 1e-3),
    "1.3b-bf16state-copy-clip": ("gpt-1.3b", True, "bf16", True, False, 1000, 1e-3),
    "6.7b-flat-clip-copy": ("gpt-6.7b", True, "fp32", True, True, 1000, 1e-3),
}
DEFAULT_CONFIG = "125m-clip"
HP = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def bytes_per_param(clip: bool, state: str, copy: bool,
                    write_grads: bool = False) -> tuple[int, int]:
    """(whole step, update kernel) algorithmic bytes per parameter.

    Update: read p, g (4 B each) and m, v (4 or 2 B each); write p, m, v and
    the bf16 copy (2 B), and with write_grads the clipped g (4 B).  The clip adds
    one more read of g in the norm pass.
    """
    s = 4 if state == "fp32" else 2
    update = 4 + 4 + 2 * s + 4 + 2 * s + (2 if copy else 0) + (4 if write_grads else 0)
    return update + (4 if clip else 0), update


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_set(name: str, device, capturable: bool = False, write_grads: bool = False):
    """Params (init as mini-megatron's model), resident grads and the optimizer."""
    import mi_adamw
    from mi_adamw.workloads import SHAPES, init_kind

    shape_name, clip, state, copy, flat, start_step, gstd = CONFIGS[name]
    shape = SHAPES[shape_name]
    params = []
    for i, (tname, shp) in enumerate(shape.tensors()):
        kind = init_kind(tname)
        if kind == "ones":
            t = torch.ones(shp, device=device)
        elif kind == "zeros":
            t = torch.zeros(shp, device=device)
        else:
            t = torch.randn(shp, device=device,
                            generator=torch.Generator(device).manual_seed(1000 + i)).mul_(0.02)
        params.append(torch.nn.Parameter(t))
    opt = mi_adamw.FusedAdamW(params, **HP, max_grad_norm=1.0 if clip else None,
                              state_dtype=torch.bfloat16 if state == "bf16" else torch.float32,
                              bf16_copy=copy, flat_buffer=flat, fused=False,
                              capturable=capturable, clip_write_grads=write_grads)
    for i, p in enumerate(params):
        g = torch.Generator(device)
        grad = torch.randn(p.shape, device=device, generator=g.manual_seed(4000 + i)).mul_(gstd)
        if p.grad is None:
            p.grad = grad
        else:
            p.grad.copy_(grad)
        del grad
        if start_step:
            m = torch.randn(p.shape, device=device, generator=g.manual_seed(2000 + i)).mul_(1e-3)
            v = torch.randn(p.shape, device=device, generator=g.manual_seed(3000 + i)).mul_(1e-6).abs_()
            opt.set_state(p, float(start_step), m, v)
            del m, v
    n = sum(p.numel() for p in params)
    return params, opt, n, len(params)


def time_fused(opt, steps: int, warmup: int):
    """Warm up, then time exactly `steps` steps; per-kernel HIP events inside."""
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for k in range(steps):
        opt.timing_events = evs[k]
        opt.step()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    opt.timing_events = None
    gpu = start.elapsed_time(end) / steps
    norm_ms = [e[0].elapsed_time(e[1]) for e in evs]
    upd_ms = [e[1].elapsed_time(e[2]) for e in evs]
    step_ms = [e[0].elapsed_time(e[2]) for e in evs]
    return gpu, wall, norm_ms, upd_ms, step_ms


def _pct(xs, q):
    """Nearest-rank percentile of a list (q in [0, 1])."""
    ys = sorted(xs)
    return ys[min(len(ys) - 1, max(0, math.ceil(q * len(ys)) - 1))]


def host_cpu() -> dict:
    """CPU model and counts of this host, for the baseline's context."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)), "torch_threads": torch.get_num_threads()}


def torch_gpu_rows(name: str, device, steps: int = 10, warmup: int = 3) -> dict:
    """torch's own GPU AdamW on the same set: per-tensor (foreach=False) and fused=True."""
    from mi_adamw.workloads import SHAPES
    shape_name, clip, state, copy, flat, start_step, gstd = CONFIGS[name]
    out = {}
    for label, kw in (("foreach_false", dict(foreach=False)), ("fused", dict(fused=True))):
        params = [torch.nn.Parameter(torch.randn(s, device=device).mul_(0.02))
                  for _, s in SHAPES[shape_name].tensors()]
        for p in params:
            p.grad = torch.randn_like(p).mul_(gstd)
        opt = torch.optim.AdamW(params, **HP, **kw)
        grads = [p.grad.clone() for p in params] if clip else None

        def one():
            if clip:
                for p, g in zip(params, grads):
                    p.grad.copy_(g)
                torch.nn.utils.clip_grad_norm_(params, 1.0)
            opt.step()
        for _ in range(warmup):
            one()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            one()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        if clip:
            # subtract the gradient refresh copies, which are not part of the step
            c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            c0.record()
            for _ in range(steps):
                for p, g in zip(params, grads):
                    p.grad.copy_(g)
            c1.record()
            torch.cuda.synchronize()
            ms -= c0.elapsed_time(c1) / steps
        out[label + "_ms"] = round(ms, 4)
        del params, opt, grads
        torch.cuda.empty_cache()
    return out


def cpu_baseline(name: str, budget_s: float = 20.0) -> dict:
    """The reference's CPU path: torch.optim.AdamW(foreach=False) (+ clip_grad_norm_),
    on CPU tensors of the same set, bounded to about `budget_s` seconds of work."""
    from mi_adamw.workloads import SHAPES
    shape_name, clip, state, copy, flat, start_step, gstd = CONFIGS[name]
    tensors = SHAPES[shape_name].tensors()
    # Bounded sample: whole tensors in model order up to ~170M parameters.
    limit = 170_000_000
    chosen, n = [], 0
    for _, s in tensors:
        k = 1
        for d in s:
            k *= d
        if n + k > limit and chosen:
            continue
        chosen.append(s)
        n += k
    threads = torch.get_num_threads()
    gen = torch.Generator().manual_seed(0)
    params = [torch.nn.Parameter(torch.randn(s, generator=gen).mul_(0.02)) for s in chosen]
    for p in params:
        p.grad = torch.randn(p.shape, generator=gen).mul_(gstd)
    opt = torch.optim.AdamW(params, **HP, foreach=False)
    if start_step:
        for p in params:
            opt.state[p]["step"] = torch.tensor(float(start_step))
            opt.state[p]["exp_avg"] = torch.randn(p.shape, generator=gen).mul_(1e-3)
            opt.state[p]["exp_avg_sq"] = torch.randn(p.shape, generator=gen).mul_(1e-6).abs_()

    def one():
        if clip:
            torch.nn.utils.clip_grad_norm_(params, 1.0)
        opt.step()
    for _ in range(2):
        one()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 200):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    total_b, _ = bytes_per_param(clip, "fp32", False)
    return {
        "value": round(total_b * n / ms / 1e6, 2), "unit": "GB/s", "cores": threads,
        "kind": "reference", "ms_per_step": round(ms, 2), "params_per_s": round(n / ms * 1e3, 1),
        "host": host_cpu(),
        "sample": f"torch.optim.AdamW(foreach=False){' after clip_grad_norm_' if clip else ''} "
                  f"on CPU, {len(params)} tensors / {n} params of {shape_name} (fp32 state), "
                  f"median of {len(times)} steps after 2 warm-up",
    }


def training_rows(device, batch: int, variants, iters: int = 20, warmup: int = 5,
                  rounds: int = 3) -> dict:
    """Training iterations of the reference GPT-125M (12 x 768, 12 heads, FFN 3072, vocab
    50304, batch x 512 tokens) as main.py:202-209 runs them with --amp: zero_grad, forward
    under bf16 autocast, backward, optimizer step.  Each variant is an optimizer choice on
    its own copy of the model (same initialisation); variants alternate round by round.
    The "_graph" variants keep their gradients in place (the flat layout, or torch's
    zero_grad(set_to_none=False)) and replay the optimizer step from a HIP graph recorded
    after the warm-up iterations."""
    import contextlib
    import warnings
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import refgpt
    from mi_adamw import FusedAdamW, bf16_weights
    warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
    ref_hp = dict(lr=6e-4, weight_decay=0.1)          # config.py:11,13; default betas and eps
    makers = {
        "torch_single_tensor": lambda ps: torch.optim.AdamW(ps, **ref_hp, fused=False),
        "torch_fused": lambda ps: torch.optim.AdamW(ps, **ref_hp, fused=True),
        "torch_fused_graph": lambda ps: torch.optim.AdamW(ps, **ref_hp, fused=True,
                                                          capturable=True),
        "mi_adamw": lambda ps: FusedAdamW(ps, **ref_hp, fused=False),
        "mi_adamw_bf16_weights": lambda ps: FusedAdamW(ps, **ref_hp, fused=False, bf16_copy=True),
        "mi_adamw_flat": lambda ps: FusedAdamW(ps, **ref_hp, fused=False, flat_buffer=True),
        "mi_adamw_flat_graph": lambda ps: FusedAdamW(ps, **ref_hp, fused=False, flat_buffer=True,
                                                     capturable=True),
    }
    ids, labels, mask = refgpt.batch(device, b=batch, s=512, vocab=50304)
    runs = {}
    for name in variants:
        torch.manual_seed(0)
        model = refgpt.GPT(vocab=50304, h=768, heads=12, ffn=3072, layers=12, seq=512).to(device)
        runs[name] = (model, makers[name](model.parameters()))
    n_linear = sum(1 for m in runs[variants[0]][0].modules() if isinstance(m, refgpt.ColumnLinear))

    graphs = {}

    def iteration(name):
        model, opt = runs[name]
        opt.zero_grad(set_to_none=not name.endswith("_graph"))
        ctx = (bf16_weights(opt, model) if name == "mi_adamw_bf16_weights"
               else contextlib.nullcontext())
        with torch.autocast("cuda", dtype=torch.bfloat16), ctx:
            _, loss = model(ids, labels, mask)
        loss.backward()
        if name in graphs:
            graphs[name].replay()
        else:
            opt.step()

    times = {name: [] for name in variants}
    for name in variants:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                iteration(name)
        torch.cuda.current_stream().wait_stream(side)
        if name.endswith("_graph"):
            torch.cuda.synchronize()
            graphs[name] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graphs[name]):
                runs[name][1].step()
    torch.cuda.synchronize()
    for _ in range(rounds):
        for name in variants:
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(iters)]
            for e0, e1 in evs:
                e0.record()
                iteration(name)
                e1.record()
            torch.cuda.synchronize()
            times[name] += [e0.elapsed_time(e1) for e0, e1 in evs]
    del runs, graphs
    torch.cuda.empty_cache()
    rows = {}
    for name in variants:
        ms = statistics.median(times[name])
        rows[name] = {"ms_per_iteration": round(ms, 4),
                      "tokens_per_s": round(batch * 512 / ms * 1e3, 1)}
    return {
        "workload": f"gpt-125m training iteration, bf16 autocast, {batch} x 512 tokens "
                    "(zero_grad, forward, backward, AdamW step)",
        "iterations_per_variant": rounds * iters,
        "weight_casts_removed_per_forward_by_bf16_weights": n_linear,
        "variants": rows,
    }


def load_traffic(name: str):
    """HBM bytes per update launch measured with rocprofv3 --pmc (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    entry = data.get(name)
    return None if entry is None else entry.get("bytes_per_launch")


def run_config(name: str, steps: int, warmup: int, device, with_context: bool,
               capturable: bool = False, write_grads: bool = False) -> dict:
    shape_name, clip, state, copy, flat, start_step, gstd = CONFIGS[name]
    log(f"[bench] {name}: building {shape_name} set" + (" (capturable)" if capturable else "")
        + (" (clipped grads written back)" if write_grads else ""))
    params, opt, n, n_tensors = build_set(name, device, capturable, write_grads)
    total_b, upd_b = bytes_per_param(clip, state, copy, write_grads)
    log(f"[bench] {name}: {n} params in {n_tensors} tensors; timing {steps} steps")
    gpu_ms, wall_ms, norm_ms, upd_ms, step_ms = time_fused(opt, steps, warmup)
    # after the timed region: the update's memory-only twin on the same tensors
    from mi_adamw.probe import time_probe
    probe_ms = time_probe(opt)
    upd_avg = statistics.mean(upd_ms)
    norm_avg = statistics.mean(norm_ms) if clip else 0.0
    step_bytes = total_b * n
    achieved_upd = upd_b * n / upd_avg / 1e6
    res = {
        "config": name, "params": n, "tensors": n_tensors, "ms_per_step": gpu_ms,
        "wall_ms_per_step": wall_ms, "bytes_per_step": step_bytes,
        "gbs": step_bytes / gpu_ms / 1e6, "params_per_s": n / gpu_ms * 1e3,
        "norm_kernel_ms": norm_avg, "update_kernel_ms": upd_avg,
        "update_kernel_ms_p90": _pct(upd_ms, 0.9),
        "step_ms_median": statistics.median(step_ms), "step_ms_p90": _pct(step_ms, 0.9),
        "update_bytes_per_launch": upd_b * n, "update_gbs": achieved_upd,
        "probe_ms": probe_ms,
        "probe_gbs": None if probe_ms is None else upd_b * n / probe_ms / 1e6,
        "dtype": "f32" if state == "fp32" else "f32 math, bf16 moments",
    }
    log(f"[bench] {name}: {gpu_ms:.4f} ms/step, {res['gbs']:.1f} GB/s "
        f"({100 * res['gbs'] / PEAK_HBM_GBS:.1f}% of peak); update {upd_avg:.4f} ms "
        f"({achieved_upd:.1f} GB/s), norm {norm_avg:.4f} ms"
        + ("" if probe_ms is None else
           f"; memory-only probe {probe_ms:.4f} ms ({res['probe_gbs']:.1f} GB/s)"))
    del params, opt
    torch.cuda.empty_cache()
    if with_context:
        res["torch_gpu"] = torch_gpu_rows(name, device)
        log(f"[bench] {name}: torch GPU context {res['torch_gpu']}")
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=DEFAULT_CONFIG,
                    help="one of %s, or 'all'" % ", ".join(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-context", action="store_true", help="skip torch's GPU rows")
    ap.add_argument("--training", action="store_true",
                    help="also time gpt-125m training iterations (bf16 autocast) with torch's "
                         "per-tensor and fused AdamW, FusedAdamW, and FusedAdamW + bf16_weights")
    ap.add_argument("--capturable", action="store_true",
                    help="step with FusedAdamW(capturable=True): torch's capturable op chain, "
                         "device step counts (the step-count increment runs before the timed "
                         "norm/update events)")
    ap.add_argument("--clip-write-grads", action="store_true",
                    help="FusedAdamW(clip_write_grads=True): the update also stores the clipped "
                         "gradients back, as torch's clip_grad_norm_ does (+4 B per parameter; "
                         "clip configurations only)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed steps, run 3 plain 1 GiB device copies (torch copy_) "
                         "so a counter run (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) sees a "
                         "kernel of known traffic next to the update kernel")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the optimizer step on one GPU; this build has no multi-GPU "
              "path (run with --gpus 1).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    import mi_adamw
    log(f"[bench] {mi_adamw.version()} on {torch.cuda.get_device_name(0)}")

    names = list(CONFIGS) if args.config == "all" else [args.config]
    if args.clip_write_grads:
        names = [nm for nm in names if CONFIGS[nm][1]]
        if not names:
            print("--clip-write-grads needs a configuration with the clip", file=sys.stderr)
            return 2
    if args.capturable:
        import warnings
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
    results = [run_config(nm, args.steps, args.warmup, device,
                          with_context=not args.no_context and nm == names[0],
                          capturable=args.capturable, write_grads=args.clip_write_grads)
               for nm in names]
    if args.calibrate_copy:
        src = torch.ones(1 << 28, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    head = results[0]
    shape_name, clip, state, copy, flat, start_step, gstd = CONFIGS[head["config"]]
    # the PMC figures in profiles/ are for the default chain's update kernel, without
    # the clipped-gradient store
    traffic = None if args.capturable or args.clip_write_grads else load_traffic(head["config"])
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0, 0.02) params (LayerNorm 1/0), resident seeded grads, "
                "mid-training moments",
        "config": {
            "workload": f"{shape_name} fused clip+AdamW step" if clip else f"{shape_name} AdamW step",
            "params": head["params"], "tensors": head["tensors"],
            "state": state, "bf16_copy": copy, "flat_buffer": flat, "clip_max_norm": 1.0 if clip else None,
            "stored_step": start_step, "lr": HP["lr"], "betas": list(HP["betas"]),
            "eps": HP["eps"], "weight_decay": HP["weight_decay"],
            "bytes_per_step": head["bytes_per_step"],
            **({"capturable": True} if args.capturable else {}),
            **({"clip_write_grads": True} if args.clip_write_grads else {}),
        },
        "pct_of_peak": round(100 * head["gbs"] / PEAK_HBM_GBS, 2),
        "params_per_s": round(head["params_per_s"], 1),
        "wall_ms_per_step": round(head["wall_ms_per_step"], 5),
        "kernels_ms": {"grad_norm": round(head["norm_kernel_ms"], 5),
                       "update": round(head["update_kernel_ms"], 5)},
        "step_ms_median": round(head["step_ms_median"], 5),
        "step_ms_p90": round(head["step_ms_p90"], 5),
        "roofline": {
            "bound": "hbm",
            "achieved": round(head["update_gbs"], 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(head["update_gbs"] / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "kernel": "mi_adamw_update_kernel",
            "bytes_per_launch": head["update_bytes_per_launch"],
            # the same launch with the arithmetic left out, on the same tensors, right
            # after the timed region: the bandwidth this read/write mix gets here
            "mix_probe": None if head["probe_ms"] is None else {
                "achieved": round(head["probe_gbs"], 2),
                "frac": round(head["probe_gbs"] / PEAK_HBM_GBS, 4),
                "update_vs_probe": round(head["update_gbs"] / head["probe_gbs"], 4),
            },
        },
    }
    if "torch_gpu" in head:
        line["torch_gpu_ms"] = head["torch_gpu"]
    if len(results) > 1:
        line["sweep"] = [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()
                          if k != "torch_gpu"} for r in results]
    if args.training:
        log("[bench] gpt-125m training iterations by optimizer")
        # the reference's micro-batch (config.py:9) with every optimizer, then a GPU-bound
        # batch for the bf16 copies against autocast's casts
        line["training"] = [
            training_rows(device, 4, ["torch_single_tensor", "torch_fused", "mi_adamw",
                                      "mi_adamw_bf16_weights", "mi_adamw_flat",
                                      "torch_fused_graph", "mi_adamw_flat_graph"]),
            training_rows(device, 16, ["mi_adamw", "mi_adamw_bf16_weights"]),
        ]
        for row in line["training"]:
            log(f"[bench] {row}")
    if not args.no_cpu:
        log("[bench] CPU baseline (torch.optim.AdamW foreach=False on host cores)")
        line["cpu_baseline"] = cpu_baseline(head["config"])
        log(f"[bench] CPU baseline {line['cpu_baseline']}")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
