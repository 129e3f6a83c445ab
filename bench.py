#!/usr/bin/env python3
"""Benchmark of the fused clip + AdamW optimizer step on one MI355X.

A step is one ``FusedAdamW.step()`` over a GPT parameter set whose params,
grads and moments are already resident in HBM: the grad-norm pass (with
clipping) and the AdamW update, exactly what mini-megatron's training loop
runs at main.py:209.  Gradients are generated once before the timed region;
the step only reads them (the clip scale is applied in registers), so every
timed step does the full work.

Default run (one GPU).  Headline: gpt-6.7b (6,863,077,376 params, 261 tensors)
in the flat-buffer layout, fp32 params/grads/moments, global grad-norm clip at
1.0 fused ahead of AdamW, bf16 model copy written by the step, optimizer state
mid-training (step 1000), lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight decay 0.1.
The other configurations of the workload list (125M, 350M, 1.3B with bf16
moments, in the layouts the optimizer offers) are timed in the same run as rows
of ``sweep``, each with its own ``roofline``.  Before its timed steps each set
takes one step and ``FusedAdamW.place_buffers(16)`` (``--placement-trials``): the
streams the update writes move to the fastest of up to 16 more allocations, by
the update's memory-only twin; each row's ``placement`` holds that report.

Output: one JSON line.  ``value`` is the achieved HBM bandwidth of the whole
step in GB/s, from algorithmic bytes (every byte the step must read or write,
counted once) over the measured step time.  ``roofline`` reports the update
kernel against MI355X's 8 TB/s, timed with HIP events on the launch stream,
with its memory-only twin on the same tensors (``mix_probe``) and the HBM bytes
per launch that rocprofv3's counters measured (``traffic``, profiles/).
``cpu_baseline`` times the reference's own CPU path (torch.optim.AdamW with
foreach=False, after clip_grad_norm_) over the same parameter set on the host's
physical cores.

    python bench.py [--steps K] [--warmup W] [--config NAME] [--sweep A,B|all|none]
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

# name: (shape, clip, state dtype, bf16 copy, flat buffer, stored step, grad std,
#        torch's fused=True chain)
CONFIGS = {
    "125m-step1": ("gpt-125m", False, "fp32", False, False, 0, 1e-3, False),
    "125m-clip": ("gpt-125m", True, "fp32", False, False, 1000, 1e-2, False),
    "350m-master-clip-copy": ("gpt-350m", True, "fp32", True, False, 1000, 1e-3, False),
    "1.3b-bf16state-copy": ("gpt-1.3b", False, "bf16", True, False, 1000, 1e-3, False),
    "1.3b-bf16state-copy-clip": ("gpt-1.3b", True, "bf16", True, False, 1000, 1e-3, False),
    "1.3b-bf16state-copy-clip-flat": ("gpt-1.3b", True, "bf16", True, True, 1000, 1e-3, False),
    "6.7b-flat-clip-copy": ("gpt-6.7b", True, "fp32", True, True, 1000, 1e-3, False),
    # the same steps in torch's fused=True chain (the reference's --fused)
    "125m-clip-fused-chain": ("gpt-125m", True, "fp32", False, False, 1000, 1e-2, True),
    "1.3b-bf16state-copy-clip-fused-chain": ("gpt-1.3b", True, "bf16", True, False, 1000, 1e-3,
                                             True),
    "6.7b-flat-clip-copy-fused-chain": ("gpt-6.7b", True, "fp32", True, True, 1000, 1e-3, True),
}
# The headline is the largest configuration that fits one GPU, the 6.7B flat clip + copy
# step; the other configurations are timed in the same run, as rows of `sweep`.
DEFAULT_CONFIG = "6.7b-flat-clip-copy"
DEFAULT_SWEEP = ("1.3b-bf16state-copy-clip", "1.3b-bf16state-copy-clip-flat",
                 "1.3b-bf16state-copy", "350m-master-clip-copy", "125m-clip", "125m-step1",
                 "1.3b-bf16state-copy-clip-fused-chain", "125m-clip-fused-chain")
# CPU baselines: the clip configurations of the workload list (125M, 350M, 1.3B, 6.7B)
DEFAULT_CPU = ("6.7b-flat-clip-copy", "1.3b-bf16state-copy-clip", "350m-master-clip-copy",
               "125m-clip")
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

    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[name]
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
                              bf16_copy=copy, flat_buffer=flat, fused=chain,
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
    """Warm up, then time exactly `steps` steps, with per-kernel HIP events inside the timed
    region on the launch stream.  Each event record is a marker packet that costs the GPU
    4-5 us, so the events are shared between steps: one step's last event is the next
    step's first.  A clipped step adds two (after the norm pass and finalize, after the
    update), a step without the clip one (its update time is then its step time)."""
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    clip = opt.max_grad_norm is not None
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    mids = [torch.cuda.Event(enable_timing=True) for _ in range(steps)] if clip else None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ends[0].record()
    for k in range(steps):
        opt.timing_events = (None, mids[k] if clip else None, ends[k + 1])
        opt.step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    opt.timing_events = None
    gpu = ends[0].elapsed_time(ends[steps]) / steps
    step_ms = [ends[k].elapsed_time(ends[k + 1]) for k in range(steps)]
    if clip:
        norm_ms = [ends[k].elapsed_time(mids[k]) for k in range(steps)]
        upd_ms = [mids[k].elapsed_time(ends[k + 1]) for k in range(steps)]
    else:
        norm_ms = [0.0] * steps
        upd_ms = list(step_ms)
    return gpu, wall, norm_ms, upd_ms, step_ms


def _pct(xs, q):
    """Nearest-rank percentile of a list (q in [0, 1])."""
    ys = sorted(xs)
    return ys[min(len(ys) - 1, max(0, math.ceil(q * len(ys)) - 1))]


def host_cpu() -> dict:
    """CPU model, logical and physical core counts of the CPUs this process may run on
    (lscpu's view, read from /proc/cpuinfo), host memory, and torch's thread count."""
    allowed = sorted(os.sched_getaffinity(0))
    model, cores = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().split("\n\n"):
                fields = dict(l.split(":", 1) for l in line.splitlines() if ":" in l)
                fields = {k.strip(): v.strip() for k, v in fields.items()}
                if "processor" not in fields or int(fields["processor"]) not in allowed:
                    continue
                model = model or fields.get("model name")
                cores.add((fields.get("physical id", "0"), fields.get("core id",
                                                                        fields["processor"])))
    except OSError:
        pass
    ram = None
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal:"):
                    ram = round(int(line.split()[1]) / 2**20, 1)
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "affinity_cpus": len(allowed),
            "physical_cores": len(cores) or None, "ram_gib": ram,
            "torch_threads": torch.get_num_threads()}


def torch_gpu_rows(name: str, device, steps: int = 10, warmup: int = 3) -> dict:
    """torch's own GPU AdamW on the same set: per-tensor (foreach=False) and fused=True."""
    from mi_adamw.workloads import SHAPES
    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[name]
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


def cpu_baseline(name: str, batch_params: int = 1 << 29, warmup: int = 2,
                 reps: int = 5) -> dict:
    """The reference's CPU path on the configuration's whole tensor set:
    ``clip_grad_norm_`` (the clip configurations) and ``torch.optim.AdamW(foreach=False)``,
    with torch's intra-op threads set to the host's physical cores.

    The set is streamed through one host pool of at most `batch_params` parameters
    (p, grad, exp_avg, exp_avg_sq in fp32: 16 B each; 8 GiB by default), so that a
    6.7B set runs on a host with far less than its 110 GB: the tensors are taken in
    model order in batches that fit the pool, every batch's tensors are views of the
    pool at their real shapes, and the step time is the sum over batches of the
    per-batch medians (`warmup` untimed, then `reps` timed repetitions).  Per batch and
    repetition the clip is timed as its two halves: ``get_total_norm`` of the batch's
    gradients (clip_grad.py:50-117) and ``clip_grads_with_norm_`` (:121-183), given a
    total norm below max_norm so the coefficient is exactly 1: the multiply costs the
    same as with a real coefficient, and the reused gradients keep their size instead
    of shrinking towards denormals (which would slow the CPU).  The CPU path keeps
    fp32 moments and writes no bf16 copy: it moves 32 B per parameter with the clip,
    28 without, and ``value`` counts those bytes."""
    from mi_adamw.workloads import SHAPES
    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[name]
    tensors = [s for _, s in SHAPES[shape_name].tensors()]
    numels = [math.prod(s) for s in tensors]
    info = host_cpu()
    threads = info["physical_cores"] or info["affinity_cpus"]
    torch.set_num_threads(threads)
    batches, cur, n_cur = [], [], 0
    for i, k in enumerate(numels):
        if cur and n_cur + k > batch_params:
            batches.append(cur)
            cur, n_cur = [], 0
        cur.append(i)
        n_cur += k
    batches.append(cur)
    pool_n = max(sum(numels[i] for i in b) for b in batches)
    gen = torch.Generator().manual_seed(0)
    pool = {"p": torch.randn(pool_n, generator=gen).mul_(0.02),
            "g": torch.randn(pool_n, generator=gen).mul_(gstd),
            "m": torch.randn(pool_n, generator=gen).mul_(1e-3),
            "v": torch.randn(pool_n, generator=gen).mul_(1e-6).abs_()}
    below = torch.tensor(0.5)            # a total norm under max_norm 1.0: coefficient 1
    total_ms, reps_done = 0.0, 0
    for b in batches:
        params, off = [], 0
        for i in b:
            k = numels[i]
            p = torch.nn.Parameter(pool["p"][off:off + k].view(tensors[i]))
            p.grad = pool["g"][off:off + k].view(tensors[i])
            params.append((p, off, k))
            off += k
        opt = torch.optim.AdamW([p for p, _, _ in params], **HP, foreach=False)
        for p, o, k in params:
            opt.state[p] = {"step": torch.tensor(float(start_step)),
                            "exp_avg": pool["m"][o:o + k].view(p.shape),
                            "exp_avg_sq": pool["v"][o:o + k].view(p.shape)}
        ps = [p for p, _, _ in params]
        times = []
        for r in range(warmup + reps):
            t0 = time.perf_counter()
            if clip:
                torch.nn.utils.get_total_norm([p.grad for p in ps])
                torch.nn.utils.clip_grads_with_norm_(ps, 1.0, below)
            opt.step()
            times.append(time.perf_counter() - t0)
        total_ms += statistics.median(times[warmup:]) * 1e3
        reps_done = reps
        del opt, params, ps
    del pool
    n = sum(numels)
    total_b, _ = bytes_per_param(clip, "fp32", False)
    info["torch_threads"] = torch.get_num_threads()
    return {
        "value": round(total_b * n / total_ms / 1e6, 2), "unit": "GB/s", "cores": threads,
        "kind": "reference", "ms_per_step": round(total_ms, 4),
        "params_per_s": round(n / total_ms * 1e3, 1), "host": info,
        "sample": f"torch.optim.AdamW(foreach=False)"
                  f"{' after clip_grad_norm_ (get_total_norm + clip_grads_with_norm_)' if clip else ''}"
                  f" on the CPU over the whole {shape_name} set ({len(tensors)} tensors, {n} "
                  f"params), fp32 moments, no bf16 copy ({total_b} B/param); "
                  f"{'streamed in ' + str(len(batches)) + ' batches of whole tensors through one ' if len(batches) > 1 else 'one '}"
                  f"{pool_n * 16 / 2**30:.1f} GiB host pool; per batch {warmup} warm-up + median of "
                  f"{reps_done} repetitions, summed over batches",
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
        # the drop-in under the reference's --fused: torch's fused=True chain
        "mi_adamw_fused_true": lambda ps: FusedAdamW(ps, **ref_hp, fused=True),
        "mi_adamw_placed": lambda ps: FusedAdamW(ps, **ref_hp, fused=False, place_trials=16),
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


def describe(name: str) -> str:
    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[name]
    parts = [f"{shape_name}", "flat buffer" if flat else "per-tensor tables",
             "bf16 moments" if state == "bf16" else "fp32 moments"]
    if copy:
        parts.append("bf16 copy")
    if chain:
        parts.append("torch's fused=True chain")
    return ", ".join(parts) + (": fused clip + AdamW step" if clip else ": AdamW step")


def range_shard_rows(opt, world: int, steps: int = 10, warmup: int = 3) -> dict:
    """The step as `world` ZeRO-1 ranks would take it, each rank's kernels on its own
    contiguous slice of the flat buffers (mi_adamw.ZeroRangeStep, gradients pre-scaled by
    f32(1/world) as allreduce_grads' div_ would leave them): per rank the sum of squares
    of its slice, the finalize from the ranks' sums (which arrive by an 8-byte all-reduce
    across GPUs) and the update of its slice.  Every rank's kernels run in turn on this
    GPU; each is timed with HIP events on the launch stream."""
    import mi_adamw
    zs = mi_adamw.ZeroRangeStep(opt, world, grad_prescale=mi_adamw.dp_prescale(world))
    clip = opt.max_grad_norm is not None
    sizes = [hi - lo for lo, hi in zs.bounds]
    per = {"sumsq": [[] for _ in range(world)], "finalize": [], "update": [[] for _ in range(world)]}
    ev = lambda: torch.cuda.Event(enable_timing=True)    # noqa: E731
    for k in range(warmup + steps):
        hypers = zs.begin()
        marks = []
        coef = None
        if clip:
            for r in range(world):
                a, b = ev(), ev()
                a.record()
                zs.grad_sumsq(r)
                b.record()
                marks.append(("sumsq", r, a, b))
            a, b = ev(), ev()
            a.record()
            _, coef = zs.finalize(zs._sumsq[:world])
            b.record()
            marks.append(("finalize", 0, a, b))
        for r in range(world):
            a, b = ev(), ev()
            a.record()
            zs.update(r, hypers, coef)
            b.record()
            marks.append(("update", r, a, b))
        torch.cuda.synchronize()
        if k >= warmup:
            for kind, r, a, b in marks:
                (per[kind] if kind == "finalize" else per[kind][r]).append(a.elapsed_time(b))
    shape_bytes = bytes_per_param(clip, "fp32" if opt.state_dtype == torch.float32 else "bf16",
                                  opt.bf16_copy)
    upd_ms = [statistics.mean(x) for x in per["update"]]
    sq_ms = [statistics.mean(x) for x in per["sumsq"]] if clip else [0.0] * world
    fin_ms = statistics.mean(per["finalize"]) if clip else 0.0
    rank_ms = [s + fin_ms + u for s, u in zip(sq_ms, upd_ms)]
    upd_gbs = [shape_bytes[1] * n / t / 1e6 for n, t in zip(sizes, upd_ms)]
    rank_gbs = [shape_bytes[0] * n / t / 1e6 for n, t in zip(sizes, rank_ms)]
    return {
        "world": world, "slice_params": sizes[0], "grad_prescale": zs.grad_prescale,
        "rank_ms_mean": statistics.mean(rank_ms), "rank_ms_max": max(rank_ms),
        "rank_gbs_mean": statistics.mean(rank_gbs),
        "rank_pct_of_peak_mean": 100 * statistics.mean(rank_gbs) / PEAK_HBM_GBS,
        "sumsq_ms_mean": statistics.mean(sq_ms), "finalize_ms": fin_ms,
        "update_ms_mean": statistics.mean(upd_ms), "update_ms_max": max(upd_ms),
        "update_gbs_mean": statistics.mean(upd_gbs),
        "update_frac_mean": statistics.mean(upd_gbs) / PEAK_HBM_GBS,
        "note": "every rank's kernels in turn on one GPU; the reduce-scatter, the 8-byte "
                "all-reduce of the sums and the all-gather need more than one GPU",
    }


def placement_ab(opt, orig: dict, streams, steps: int, warmup: int, rounds: int = 4) -> dict:
    """The step on the optimizer's original streams against the streams place_buffers
    chose, alternating in this process (same parameters and gradients): `rounds` rounds of
    `steps` timed steps on each, after `warmup` untimed ones at every switch."""
    placed = streams.current()
    res = {"original": [], "placed": []}
    for r in range(rounds):
        order = (("original", orig), ("placed", placed))
        for label, bufs in (order if r % 2 == 0 else order[::-1]):
            streams.adopt(bufs)
            opt._launch_cache = None
            opt._fast = None
            gpu_ms, _, _, _, _ = time_fused(opt, steps, warmup)
            res[label].append(round(gpu_ms, 5))
    streams.adopt(placed)
    opt._launch_cache = None
    opt._fast = None
    gain = statistics.mean(res["original"]) / statistics.mean(res["placed"]) - 1.0
    return {"rounds": rounds, "steps_per_round": steps, "original_ms": res["original"],
            "placed_ms": res["placed"], "gain": round(gain, 5)}


def run_config(name: str, steps: int, warmup: int, device, with_context: bool,
               capturable: bool = False, write_grads: bool = False,
               range_world: int = 0, trials: int = 0, ab: bool = False,
               passes: int = 1) -> dict:
    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[name]
    log(f"[bench] {name}: building {shape_name} set" + (" (capturable)" if capturable else "")
        + (" (clipped grads written back)" if write_grads else ""))
    params, opt, n, n_tensors = build_set(name, device, capturable, write_grads)
    total_b, upd_b = bytes_per_param(clip, state, copy, write_grads)
    placement = None
    if trials > 0:
        # where the streams the update writes live: the fastest of `trials` more
        # allocations by the update's memory-only twin (FusedAdamW.place_buffers)
        from mi_adamw import placement as pl
        opt.step()                      # the tables exist and every state entry is created
        torch.cuda.synchronize()
        streams = orig = None
        if ab:
            streams = pl._FlatStreams(opt, device) if flat else pl._TableStreams(opt, device)
            orig = streams.current()    # kept alive for the A/B
        placement = opt.place_buffers(trials=trials)
        log(f"[bench] {name}: place_buffers {placement}")
        if ab:
            placement["ab"] = placement_ab(opt, orig, streams, steps, warmup)
            log(f"[bench] {name}: placement A/B {placement['ab']}")
        del orig, streams
        if passes > 1:
            # more passes of the same search, each from where the last one left the streams,
            # with the step timed before and after each
            later = []
            for k in range(2, passes + 1):
                before = time_fused(opt, steps, warmup)[0]
                rep = opt.place_buffers(trials=trials)
                after = time_fused(opt, steps, warmup)[0]
                later.append({"pass": k, "chosen": rep["chosen"],
                              "per_stream_chosen": [st["chosen"] for st in rep["per_stream"]],
                              "total_twin_gain": rep["total_twin_gain"],
                              "step_ms_before": round(before, 5), "step_ms_after": round(after, 5)})
                log(f"[bench] {name}: placement pass {later[-1]}")
            placement["later_passes"] = later
    log(f"[bench] {name}: {n} params in {n_tensors} tensors; timing {steps} steps")
    gpu_ms, wall_ms, norm_ms, upd_ms, step_ms = time_fused(opt, steps, warmup)
    # after the timed region: the update's memory-only twin on the same tensors
    from mi_adamw.probe import time_probe
    probe_ms = time_probe(opt)
    upd_avg = statistics.mean(upd_ms)
    norm_avg = statistics.mean(norm_ms) if clip else 0.0
    step_bytes = total_b * n
    achieved_upd = upd_b * n / upd_avg / 1e6
    probe_gbs = None if probe_ms is None else upd_b * n / probe_ms / 1e6
    # the PMC figures in profiles/ are for the default chain's update kernel, without
    # the clipped-gradient store
    traffic = None if capturable or write_grads else load_traffic(name)
    res = {
        "config": name, "workload": describe(name), "params": n, "tensors": n_tensors,
        "state": state, "bf16_copy": copy, "flat_buffer": flat, "clip": clip,
        "dtype": "f32", "ms_per_step": gpu_ms, "wall_ms_per_step": wall_ms,
        "bytes_per_param": total_b, "bytes_per_step": step_bytes,
        "gbs": step_bytes / gpu_ms / 1e6, "pct_of_peak": 100 * step_bytes / gpu_ms / 1e6 / PEAK_HBM_GBS,
        "params_per_s": n / gpu_ms * 1e3,
        "placement": placement,
        "norm_kernel_ms": norm_avg, "update_kernel_ms": upd_avg,
        "update_kernel_ms_p90": _pct(upd_ms, 0.9),
        "step_ms_median": statistics.median(step_ms), "step_ms_p90": _pct(step_ms, 0.9),
        "roofline": {
            "bound": "hbm", "achieved": achieved_upd, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": achieved_upd / PEAK_HBM_GBS, "traffic": traffic,
            "kernel": "mi_adamw_update_kernel", "bytes_per_launch": upd_b * n,
            # the same launch with the arithmetic left out, on the same tensors, right
            # after the timed region: the bandwidth this read/write mix gets here
            "mix_probe": None if probe_ms is None else {
                "achieved": probe_gbs, "frac": probe_gbs / PEAK_HBM_GBS,
                "update_vs_probe": achieved_upd / probe_gbs,
                "step_vs_probe_ceiling": (norm_avg + probe_ms) / gpu_ms,
            },
        },
    }
    log(f"[bench] {name}: {gpu_ms:.4f} ms/step, {res['gbs']:.1f} GB/s "
        f"({res['pct_of_peak']:.1f}% of peak); update {upd_avg:.4f} ms "
        f"({achieved_upd:.1f} GB/s), norm {norm_avg:.4f} ms"
        + ("" if probe_ms is None else
           f"; memory-only probe {probe_ms:.4f} ms ({probe_gbs:.1f} GB/s)"))
    if range_world > 1 and flat and not capturable and not write_grads:
        res["range_shard"] = range_shard_rows(opt, range_world)
        rs = res["range_shard"]
        log(f"[bench] {name}: as {range_world} ZeRO-1 ranks, {rs['slice_params']} params each: "
            f"{rs['rank_ms_mean']:.4f} ms per rank ({rs['rank_pct_of_peak_mean']:.1f}% of peak), "
            f"update {rs['update_ms_mean']:.4f} ms ({rs['update_gbs_mean']:.1f} GB/s)")
    del params, opt
    torch.cuda.empty_cache()
    if with_context:
        res["torch_gpu_ms"] = torch_gpu_rows(name, device)
        log(f"[bench] {name}: torch GPU context {res['torch_gpu_ms']}")
    return res


def host_step_us(device, n_tensors: int, steps: int = 300) -> dict:
    """Host time of FusedAdamW.step() (enqueue only) with gradients that move every step,
    as after mini-megatron's zero_grad() (main.py:204): n_tensors small fp32 tensors, the
    clip on, three gradient sets in rotation.  Median and p90 in microseconds."""
    import mi_adamw
    params = [torch.nn.Parameter(torch.randn(4096, device=device)) for _ in range(n_tensors)]
    sets = [[torch.randn_like(p) for p in params] for _ in range(3)]
    opt = mi_adamw.FusedAdamW(params, **HP, max_grad_norm=1.0)
    ts = []
    for k in range(steps + 30):
        for p, g in zip(params, sets[k % 3]):
            p.grad = g
        t0 = time.perf_counter()
        opt.step()
        ts.append(time.perf_counter() - t0)
        if k % 50 == 49:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    ts = sorted(ts[30:])
    return {"tensors": n_tensors, "median_us": round(ts[len(ts) // 2] * 1e6, 1),
            "p90_us": round(_pct(ts, 0.9) * 1e6, 1)}


def _rounded(x):
    if isinstance(x, float):
        return round(x, 5)
    if isinstance(x, dict):
        return {k: _rounded(v) for k, v in x.items()}
    return x


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=DEFAULT_CONFIG,
                    help="headline configuration, one of %s" % ", ".join(CONFIGS))
    ap.add_argument("--sweep", default=",".join(DEFAULT_SWEEP),
                    help="comma-separated configurations timed in the same run as rows of "
                         "`sweep` ('all' for every other configuration, 'none' for none)")
    ap.add_argument("--cpu", default=",".join(DEFAULT_CPU),
                    help="configurations whose CPU baseline is timed (the headline's goes to "
                         "`cpu_baseline`, the others to their sweep rows)")
    ap.add_argument("--no-cpu", action="store_true", help="skip every CPU baseline")
    ap.add_argument("--no-context", action="store_true", help="skip torch's GPU rows")
    ap.add_argument("--no-host", action="store_true", help="skip the step() host-time rows")
    ap.add_argument("--range-world", type=int, default=8,
                    help="after the headline's timed steps (flat layout), time its step as this "
                         "many ZeRO-1 ranks' slices, every rank's kernels in turn (0: skip)")
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
    ap.add_argument("--placement-trials", type=int, default=16,
                    help="before each configuration's timed steps, FusedAdamW.place_buffers "
                         "with this many candidate placements of the streams the update writes "
                         "(0: keep the first allocation)")
    ap.add_argument("--placement-passes", type=int, default=1,
                    help="run place_buffers this many times before the timed steps, timing the "
                         "step before and after every pass after the first")
    ap.add_argument("--placement-ab", action="store_true",
                    help="also time each configuration's step on its original streams against "
                         "the placed ones, alternating rounds in this process")
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
    if args.config not in CONFIGS:
        print(f"unknown configuration {args.config!r}", file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    import mi_adamw
    log(f"[bench] {mi_adamw.version()} on {torch.cuda.get_device_name(0)}")

    sweep = {"all": [nm for nm in CONFIGS if nm != args.config], "none": []}.get(
        args.sweep, [nm for nm in args.sweep.split(",") if nm and nm != args.config])
    for nm in sweep:
        if nm not in CONFIGS:
            print(f"unknown configuration {nm!r}", file=sys.stderr)
            return 2
    names = [args.config] + sweep
    if args.clip_write_grads:
        names = [nm for nm in names if CONFIGS[nm][1]]
        if args.config not in names:
            print("--clip-write-grads needs a headline configuration with the clip",
                  file=sys.stderr)
            return 2
    if args.capturable:
        import warnings
        warnings.filterwarnings("ignore", message="This instance was constructed with capturable")
    results = {nm: run_config(nm, args.steps, args.warmup, device,
                              with_context=not args.no_context and nm == args.config,
                              capturable=args.capturable, write_grads=args.clip_write_grads,
                              range_world=args.range_world if nm == args.config else 0,
                              trials=args.placement_trials, ab=args.placement_ab,
                              passes=args.placement_passes)
               for nm in names}
    if args.calibrate_copy:
        src = torch.ones(1 << 28, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    head = results[args.config]
    shape_name, clip, state, copy, flat, start_step, gstd, chain = CONFIGS[args.config]
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
        "dtype": head["dtype"],
        "data": "synthetic: seeded N(0, 0.02) params (LayerNorm 1/0), resident seeded grads, "
                "mid-training moments",
        "config": {
            "workload": head["workload"],
            "params": head["params"], "tensors": head["tensors"],
            "state": state, "bf16_copy": copy, "flat_buffer": flat,
            "clip_max_norm": 1.0 if clip else None,
            "stored_step": start_step, "lr": HP["lr"], "betas": list(HP["betas"]),
            "eps": HP["eps"], "weight_decay": HP["weight_decay"],
            "bytes_per_param": head["bytes_per_param"], "bytes_per_step": head["bytes_per_step"],
            **({"capturable": True} if args.capturable else {}),
            **({"clip_write_grads": True} if args.clip_write_grads else {}),
        },
        "pct_of_peak": round(head["pct_of_peak"], 2),
        "params_per_s": round(head["params_per_s"], 1),
        "wall_ms_per_step": round(head["wall_ms_per_step"], 5),
        "kernels_ms": {"grad_norm": round(head["norm_kernel_ms"], 5),
                       "update": round(head["update_kernel_ms"], 5)},
        "step_ms_median": round(head["step_ms_median"], 5),
        "step_ms_p90": round(head["step_ms_p90"], 5),
        "roofline": _rounded(head["roofline"]),
        "placement": head["placement"],
    }
    if "torch_gpu_ms" in head:
        line["torch_gpu_ms"] = head["torch_gpu_ms"]
    if "range_shard" in head:
        line["range_shard"] = _rounded(head["range_shard"])
    if sweep:
        line["sweep"] = [_rounded(results[nm]) for nm in names if nm != args.config]
    if not args.no_host:
        line["host_step_us_moving_grads"] = [host_step_us(device, n) for n in (101, 261)]
        log(f"[bench] step() host time {line['host_step_us_moving_grads']}")
    if args.training:
        log("[bench] gpt-125m training iterations by optimizer")
        # the reference's micro-batch (config.py:9) with every optimizer, then a GPU-bound
        # batch for the bf16 copies against autocast's casts
        line["training"] = [
            training_rows(device, 4, ["torch_single_tensor", "torch_fused", "mi_adamw",
                                      "mi_adamw_fused_true", "mi_adamw_placed",
                                      "mi_adamw_bf16_weights", "mi_adamw_flat",
                                      "torch_fused_graph", "mi_adamw_flat_graph"]),
            training_rows(device, 16, ["mi_adamw", "mi_adamw_bf16_weights"]),
        ]
        for row in line["training"]:
            log(f"[bench] {row}")
    if not args.no_cpu:
        for nm in [nm for nm in args.cpu.split(",") if nm in results]:
            log(f"[bench] CPU baseline of {nm} (torch.optim.AdamW foreach=False on host cores)")
            cb = cpu_baseline(nm)
            log(f"[bench] CPU baseline of {nm}: {cb}")
            if nm == args.config:
                line["cpu_baseline"] = cb
            else:
                for row in line.get("sweep", []):
                    if row["config"] == nm:
                        row["cpu_baseline"] = cb
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
