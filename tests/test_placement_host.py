"""Host-side pieces of the buffer placement, on the CPU: block offsets, how many candidate
sets fit, which rows the memory-only twin may touch, and the refusals that come before any
device work."""
from __future__ import annotations

import pytest
import torch

from mi_adamw import placement
from mi_adamw.placement import candidates_that_fit, plan_offsets, twin_row_ok

CPU = torch.device("cpu")
F32, BF16 = torch.float32, torch.bfloat16


def test_plan_offsets_aligns_every_tensor_to_128_bytes():
    offs, total = plan_offsets([1, 32, 33, 0, 70001, 5])
    assert offs == [0, 32, 64, 128, 128, 70144]     # 128 + 70001 = 70129, rounded up
    assert total == 70176
    # each tensor fits before the next one starts, and the block ends after the last
    sizes = [1, 32, 33, 0, 70001, 5]
    for (o, n), nxt in zip(zip(offs, sizes), offs[1:] + [total]):
        assert o % 32 == 0 and o + n <= nxt
    assert plan_offsets([]) == ([], 0)


def test_candidates_that_fit():
    gib = 1 << 30
    assert candidates_that_fit(10 * gib, 16, 100 * gib, 2 * gib) == 9
    assert candidates_that_fit(10 * gib, 4, 100 * gib, 2 * gib) == 4
    assert candidates_that_fit(10 * gib, 16, 11 * gib, 2 * gib) == 0
    assert candidates_that_fit(10 * gib, 16, 1 * gib, 2 * gib) == 0   # reserve above free
    assert candidates_that_fit(0, 16, 100 * gib, 0) == 0
    assert candidates_that_fit(gib, 0, 100 * gib, 0) == 0


def test_twin_row_ok_accepts_only_dense_tensors_of_the_read_type():
    n = 96
    p, g = torch.zeros(n), torch.zeros(n)
    m, v, c = torch.zeros(n), torch.zeros(n), torch.zeros(n, dtype=BF16)
    dt = [F32, F32, F32, F32, BF16]
    assert twin_row_ok([p, g, m, v, c], dt, n, CPU)
    assert twin_row_ok([p.view(8, 12), g, m, v, c], dt, n, CPU)      # any dense shape
    assert not twin_row_ok([p, g, m, v, c], dt, 0, CPU)               # nothing to read
    assert not twin_row_ok([p, None, m, v, c], dt, n, CPU)            # no gradient
    assert not twin_row_ok([p, g, torch.zeros(2 * n)[::2], v, c], dt, n, CPU)   # strided
    assert not twin_row_ok([p, g, m, torch.zeros(n + 1), c], dt, n, CPU)        # other size
    # a state entry of a smaller type than the kernel reads would be overrun
    assert not twin_row_ok([p, g, m.to(BF16), v, c], dt, n, CPU)
    assert not twin_row_ok([p.to(BF16), g, m, v, c], dt, n, CPU)
    assert not twin_row_ok([p, g, m, v, c.float()], dt, n, CPU)
    # host memory is not device memory: a tensor on another device is left out
    assert not twin_row_ok([p, g, m, torch.zeros(n, device="meta"), c], dt, n, CPU)
    assert not twin_row_ok([p, g, m, v, c], dt, n, torch.device("meta"))
    assert not twin_row_ok([p, g.to_sparse(), m, v, c], dt, n, CPU)   # not strided
    with pytest.raises(ValueError):
        twin_row_ok([p, g, m, v], dt, n, CPU)                         # one dtype per tensor


def test_place_buffers_refusals_before_any_device_work():
    import mi_adamw
    ps = [torch.nn.Parameter(torch.zeros(4)), torch.nn.Parameter(torch.zeros(3))]
    opt = mi_adamw.FusedAdamW(ps, lr=1e-3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        placement.place_buffers(opt)
    ams = mi_adamw.FusedAdamW([torch.nn.Parameter(torch.zeros(4))], lr=1e-3, amsgrad=True)
    with pytest.raises(NotImplementedError, match="amsgrad"):
        ams.place_buffers()
    opt.captured = True
    with pytest.raises(RuntimeError, match="recorded into a graph"):
        opt.place_buffers()
