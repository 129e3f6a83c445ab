"""Measured placement of the HBM streams the optimizer writes (FusedAdamW.place_buffers).

On the MI355X the bandwidth of the update's read/write mix depends on which physical
pages its written streams occupy.  In one process, stream sets of identical size and
virtual layout run the same update 10-13% apart, depending only on where each set was
allocated: at 1.42G parameters with bf16 moments and the bf16 copy, 4.87-4.95 ms on
some sets against 5.3-5.6 ms on others, reproducibly per set.  A set keeps its speed
for as long as it lives; the gradients' placement does not matter (only the streams
the update writes do).  The library cannot choose physical pages, but it can measure
them: ``place_buffers`` allocates up to ``trials`` more sets of the streams the
optimizer owns and writes, times the update's memory-only twin (``mi_adamw_probe``,
``mi_adamw_probe_flat``: the update's launch, loads and stores without the arithmetic)
on every set, the current one included, against the current parameters and gradients,
moves the values into the fastest set (if it beats the current one by at least
``min_gain``, 1% by default: the twin ranks the update alone, and differences below that
are within how closely it tracks the whole step) and frees the others.  Then, one stream
at a time, it tries new allocations of that stream alone with the others kept, and moves
the stream the same way: the speed is a property of how the streams' pages combine, and
replacing a single stream of a slow set can make it fast, so this stage reaches further
for the same memory (one stream per candidate rather than a set; at 6.7B only one whole
set fits beside the optimizer's own, but four or five of each stream).  A stream's best
place depends on where the others are, so the streams are swept again after a sweep that
moved one, up to ``sweeps`` sweeps.

The placed streams:
- per-tensor tables: exp_avg, exp_avg_sq and the bf16 copy, each as one block over
  every parameter with state, at 128-byte aligned offsets in param_groups order; the
  state entries and copies become views of the blocks.  Parameters and gradients stay
  the caller's.
- flat layout: the parameter, exp_avg, exp_avg_sq and copy buffers (the parameters'
  ``.data`` and the state entries are re-pointed at the new buffers); the gradient
  buffer stays.

The values are copied bit for bit, so every later step gives the results it would have
given without the move.  Transient memory: one stream set per candidate, held until the
choice is made (the candidates must coexist to land on different pages); the freed
candidates return to torch's caching allocator.  As many candidates are tried as fit
beside what is allocated, keeping ``reserve_bytes`` free.
"""
from __future__ import annotations

import ctypes
import statistics
import time

import numpy as np
import torch

from . import _lib

ALIGN_ELEMS = 32     # 128 bytes of fp32


def plan_offsets(numels) -> tuple[list[int], int]:
    """Element offset of each tensor in a block, in order, each at a 32-element (128-byte)
    boundary, and the block's length."""
    offs, off = [], 0
    for n in numels:
        offs.append(off)
        off = (off + int(n) + ALIGN_ELEMS - 1) // ALIGN_ELEMS * ALIGN_ELEMS
    return offs, off


def candidates_that_fit(set_bytes: int, trials: int, free_bytes: int, reserve_bytes: int) -> int:
    """How many more stream sets of `set_bytes` fit in `free_bytes`, keeping
    `reserve_bytes` free, at most `trials`."""
    if set_bytes <= 0 or trials <= 0:
        return 0
    return int(max(0, min(trials, (free_bytes - reserve_bytes) // set_bytes)))


def twin_row_ok(tensors, dtypes, n: int, device: torch.device) -> bool:
    """Whether the twin may read and store back `n` contiguous elements at each tensor's
    data_ptr(): every tensor present, strided, of `n` elements, of the dtype the kernel
    reads it as, on `device`, and dense (a tensor that is not, or a smaller element type,
    would put the accesses outside its memory; a host tensor is not device memory)."""
    return n > 0 and all(
        t is not None and t.layout == torch.strided and t.device == device and t.dtype == dt
        and t.numel() == n and t.is_contiguous() for t, dt in zip(tensors, dtypes, strict=True))


def _free_bytes(device: torch.device) -> tuple[int, int]:
    """(bytes an allocation can still get: the device's free memory plus what torch's
    caching allocator holds unused, the device's total)."""
    free, total = torch.cuda.mem_get_info(device)
    cached = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    return int(free + max(cached, 0)), int(total)


class _Streams:
    """One layout's placed streams: the current set, new candidate sets, the twin's launch
    over a set, and the move of the values into the chosen set."""

    names: list[str]
    set_bytes: int

    def current(self):
        raise NotImplementedError

    def allocate(self, names=None):
        raise NotImplementedError

    def stream_bytes(self, name: str) -> int:
        raise NotImplementedError

    def twin(self, cand, launches: int):
        raise NotImplementedError

    def adopt(self, cand) -> None:
        raise NotImplementedError


class _TableStreams(_Streams):
    def __init__(self, opt, device):
        from .optimizer import _ROW_DTYPE, _Launch
        self.opt, self.device = opt, device
        self._row_dtype, self._launch_cls = _ROW_DTYPE, _Launch
        self.entries = []
        for g in opt.param_groups:
            for p in g["params"]:
                st = opt.state.get(p)
                if st and "exp_avg" in st:
                    self.entries.append((p, st))
        if not self.entries:
            raise RuntimeError("place_buffers: no parameter has optimizer state yet; take a "
                               "step (or set the state) first")
        self.names = ["exp_avg", "exp_avg_sq"] + (["copy"] if opt.bf16_copy else [])
        self.dtypes = {"exp_avg": opt.state_dtype, "exp_avg_sq": opt.state_dtype,
                       "copy": torch.bfloat16}
        self.offs, self.total = plan_offsets(p.numel() for p, _ in self.entries)
        self.set_bytes = sum(self.total * torch.empty((), dtype=self.dtypes[n]).element_size()
                             for n in self.names)

    def _tensor(self, p, st, name):
        return self.opt._copies[id(p)] if name == "copy" else st[name]

    def current(self):
        return {n: [self._tensor(p, st, n) for p, st in self.entries] for n in self.names}

    def allocate(self, names=None):
        names = self.names if names is None else names
        blocks = {n: torch.empty(self.total, dtype=self.dtypes[n], device=self.device)
                  for n in names}
        return {n: [blocks[n][o:o + p.numel()].view(p.shape)
                    for o, (p, _) in zip(self.offs, self.entries)] for n in names}

    def stream_bytes(self, name):
        return self.total * torch.empty((), dtype=self.dtypes[name]).element_size()

    def _launch(self, cand):
        opt = self.opt
        rows = []
        sa = 8 if opt.state_dtype == torch.bfloat16 else 16
        dtypes = [torch.float32, torch.float32] + [self.dtypes[k] for k in self.names]
        cur = self.current()
        for i, (p, _) in enumerate(self.entries):
            g = p.grad
            n = p.numel()
            # a row the twin cannot read as it stands is left out (the step converts such
            # state before it uses it, or refuses the parameter), for every candidate
            # alike, so that all of them are timed over the same rows
            if not all(twin_row_ok([p, g] + [c[k][i] for k in self.names], dtypes, n,
                                   self.device) for c in (cand, cur)):
                continue
            pp, gp = p.data_ptr(), g.data_ptr()
            mp, vp = cand["exp_avg"][i].data_ptr(), cand["exp_avg_sq"][i].data_ptr()
            cp = cand["copy"][i].data_ptr() if "copy" in cand else 0
            vec = pp % 16 == 0 and gp % 16 == 0 and mp % sa == 0 and vp % sa == 0 and cp % 8 == 0
            rows.append((pp, gp, mp, vp, cp, 0, p.numel(), 0, _lib.T_VEC if vec else 0))
        if not rows:
            raise RuntimeError("place_buffers: no parameter with state has a gradient; the "
                               "twin reads the gradients, so call it after backward")
        arr = np.zeros(len(rows), dtype=self._row_dtype)
        for i, r in enumerate(rows):
            arr[i] = r
        return self._launch_cls(arr, self.opt.chunk_elems, self.device, tables=True)

    def twin(self, cand, launches):
        opt, lib = self.opt, _lib.load()
        launch = self._launch(cand)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        state = _lib.STATE_BF16 if opt.state_dtype == torch.bfloat16 else _lib.STATE_F32
        flags = _twin_flags(opt)

        def run():
            _lib.check(lib.mi_adamw_probe(launch.rows.data_ptr(), launch.chunks.data_ptr(),
                                          launch.n_chunks, opt.chunk_elems, state, flags,
                                          opt.max_blocks, stream), "mi_adamw_probe")
        return _timed(run, launches)

    def adopt(self, cand):
        opt = self.opt
        cur = self.current()
        with torch.no_grad():
            for n in self.names:
                for i, (p, st) in enumerate(self.entries):
                    new, old = cand[n][i], cur[n][i]
                    if new is old or old.numel() != new.numel():
                        # an entry of another size stays as it is: the step replaces a
                        # copy of the wrong size and refuses such state
                        continue
                    new.copy_(old.reshape(new.shape))
                    if n == "copy":
                        opt._copies[id(p)] = new
                    else:
                        st[n] = new


class _FlatStreams(_Streams):
    NAMES = ("param", "exp_avg", "exp_avg_sq", "copy")

    def __init__(self, opt, device):
        self.opt, self.device, self.flat = opt, device, opt._flat
        fl = self.flat
        self.names = [n for n in self.NAMES if getattr(fl, n) is not None]
        self.set_bytes = sum(getattr(fl, n).numel() * getattr(fl, n).element_size()
                             for n in self.names)

    def current(self):
        return {n: getattr(self.flat, n) for n in self.names}

    def allocate(self, names=None):
        names = self.names if names is None else names
        return {n: torch.empty_like(getattr(self.flat, n)) for n in names}

    def stream_bytes(self, name):
        t = getattr(self.flat, name)
        return t.numel() * t.element_size()

    def twin(self, cand, launches):
        opt, fl, lib = self.opt, self.flat, _lib.load()
        row = _lib.TensorRow(param=cand["param"].data_ptr(), grad=fl.grad.data_ptr(),
                             exp_avg=cand["exp_avg"].data_ptr(),
                             exp_avg_sq=cand["exp_avg_sq"].data_ptr(),
                             param_copy=cand["copy"].data_ptr() if "copy" in cand else 0,
                             max_exp_avg_sq=0, numel=fl.total, hyper=0, flags=_lib.T_VEC)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        state = _lib.STATE_BF16 if opt.state_dtype == torch.bfloat16 else _lib.STATE_F32
        flags = _twin_flags(opt)

        def run():
            _lib.check(lib.mi_adamw_probe_flat(ctypes.byref(row), opt.chunk_elems, state, flags,
                                               opt.max_blocks, stream), "mi_adamw_probe_flat")
        return _timed(run, launches)

    def adopt(self, cand):
        params = [p for g in self.opt.param_groups for p in g["params"]]
        self.flat.adopt_buffers(cand, params, self.opt.state)


def _twin_flags(opt) -> int:
    flags = 0
    if opt.bf16_copy:
        flags |= _lib.F_BF16_COPY
    if opt.max_grad_norm is not None and opt.clip_write_grads:
        flags |= _lib.F_WRITE_GRAD
    return flags


def _timed(run, launches: int) -> list[float]:
    """ms of `launches` launches of run(), each between two HIP events on the current
    stream, after one untimed launch."""
    run()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(launches)]
    for e0, e1 in evs:
        e0.record()
        run()
        e1.record()
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) for e0, e1 in evs]


def _choose(streams, cands, launches: int, rounds: int, min_gain: float):
    """Twin ms of every candidate (index 0: the current streams), timed in `rounds`
    interleaved rounds; the fastest; the one to take (the fastest if it beats the current
    one by at least `min_gain`, else 0)."""
    times = [[] for _ in cands]
    for r in range(max(1, rounds)):
        order = range(len(cands)) if r % 2 == 0 else reversed(range(len(cands)))
        for i in order:
            times[i] += streams.twin(cands[i], launches)
    twin_ms = [statistics.mean(t) for t in times]
    fastest = min(range(len(cands)), key=lambda i: twin_ms[i])
    best = fastest if twin_ms[0] / twin_ms[fastest] - 1.0 >= min_gain else 0
    return twin_ms, fastest, best


def _allocate_up_to(streams, k: int, names=None) -> list:
    out = []
    for _ in range(k):
        try:
            out.append(streams.allocate(names))
        except torch.cuda.OutOfMemoryError:
            break
    return out


@torch.no_grad()
def place_buffers(opt, trials: int = 16, launches: int = 3, rounds: int = 2,
                  reserve_bytes: int | None = None, min_gain: float = 0.01,
                  per_stream: bool = True, sweeps: int = 3) -> dict:
    """Choose where the optimizer's written streams live by timing the update's
    memory-only twin on the current set and on up to `trials` newly allocated sets
    (`rounds` interleaved rounds of `launches` timed launches each); move the values
    into the fastest set if its twin beats the current set's by at least `min_gain`
    (below that, the difference is within how closely the twin's ranking tracks the
    whole step), and free the rest.  With `per_stream`, then do the same for each
    stream alone (up to `trials` new allocations of it, the other streams kept), in
    sweeps over the streams: a stream's best place depends on where the others are, so
    a sweep that moved a stream is followed by another, up to `sweeps` sweeps.
    Returns what was tried and chosen."""
    if getattr(opt, "captured", False):
        raise RuntimeError("place_buffers: a step of this optimizer was recorded into a graph, "
                           "which keeps the addresses of the buffers it recorded; place the "
                           "buffers before capturing")
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("place_buffers cannot run under graph capture")
    if any(g["amsgrad"] for g in opt.param_groups):
        raise NotImplementedError("place_buffers: amsgrad state is not placed")
    params = [p for g in opt.param_groups for p in g["params"]]
    if not params:
        raise RuntimeError("place_buffers: the optimizer has no parameters")
    device = params[0].device
    if device.type != "cuda":
        raise RuntimeError("place_buffers needs parameters on a ROCm GPU")
    if any(p.device != device for p in params):
        raise NotImplementedError("place_buffers: all parameters must be on one device")
    if any(torch.is_complex(p) for p in params):
        raise NotImplementedError("place_buffers: complex parameters are not supported")
    t0 = time.perf_counter()
    with torch.cuda.device(device):
        # the twin stores back the values it reads, the current streams' included: work
        # still queued on any stream (a step on another stream) must finish first
        torch.cuda.synchronize(device)
        streams = (_FlatStreams(opt, device) if opt._flat is not None
                   else _TableStreams(opt, device))
        avail, total = _free_bytes(device)
        reserve = max(2 << 30, total // 50) if reserve_bytes is None else int(reserve_bytes)
        # stage 1: whole sets
        k = candidates_that_fit(streams.set_bytes, trials, avail, reserve)
        cands = [streams.current()] + _allocate_up_to(streams, k)
        twin_ms, fastest, best = _choose(streams, cands, launches, rounds, min_gain)
        if best != 0:
            streams.adopt(cands[best])
        peak = streams.set_bytes * (len(cands) - 1)
        del cands
        first_ms = twin_ms[0]
        last_ms = twin_ms[best]
        # stage 2: one stream at a time, in sweeps while a sweep moves a stream
        stages = []
        n_sweeps = 0
        while per_stream and n_sweeps < max(1, sweeps):
            n_sweeps += 1
            moved = False
            for name in streams.names:
                avail, _ = _free_bytes(device)
                k = candidates_that_fit(streams.stream_bytes(name), trials, avail, reserve)
                if k == 0:
                    continue
                cur = streams.current()
                alts = _allocate_up_to(streams, k, [name])
                cands = [cur] + [{**cur, name: a[name]} for a in alts]
                ms, f, b = _choose(streams, cands, launches, rounds, min_gain)
                if b != 0:
                    streams.adopt(cands[b])
                    moved = True
                last_ms = ms[b]
                peak = max(peak, streams.stream_bytes(name) * len(alts))
                stages.append({"sweep": n_sweeps, "stream": name, "candidates": len(ms),
                               "twin_ms": [round(x, 5) for x in ms], "fastest": f,
                               "chosen": b, "twin_gain": round(ms[0] / ms[b] - 1.0, 5)})
                del cands, alts, cur
            if not moved:
                break
        opt._launch_cache = None
        opt._fast = None
        torch.cuda.synchronize(device)
    return {
        "layout": "flat" if opt._flat is not None else "tables",
        "streams": list(streams.names), "set_bytes": int(streams.set_bytes),
        "candidates": len(twin_ms), "twin_ms": [round(x, 5) for x in twin_ms],
        "fastest": fastest, "min_gain": min_gain,
        "chosen": best, "twin_gain": round(twin_ms[0] / twin_ms[best] - 1.0, 5),
        "transient_bytes": int(streams.set_bytes) * (len(twin_ms) - 1),
        "per_stream": stages, "sweeps": n_sweeps,
        "total_twin_gain": round(first_ms / last_ms - 1.0, 5),
        "peak_transient_bytes": int(peak),
        "seconds": round(time.perf_counter() - t0, 3),
    }
