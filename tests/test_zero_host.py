"""Host-side logic of ZeRO-1 range sharding and the gradient pre-scale (CPU only).

shard_bounds: the slices cover [0, total) in order without gaps or overlap, start at
128-byte (32-element) boundaries and differ in size by at most one alignment unit.
dp_prescale: the fp32 reciprocal that torch's ``tensor.div_(world)`` multiplies by.
FusedAdamW's grad_prescale argument is validated up front.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import mi_adamw
from mi_adamw.zero import ZeroRangeStep, dp_prescale, shard_bounds


@pytest.mark.parametrize("total", [0, 32, 96, 4096 * 3 + 64, 162_954_240, 6_863_077_376, 100])
@pytest.mark.parametrize("world", [1, 2, 3, 4, 7, 8, 64])
def test_shard_bounds_partition(total, world):
    b = shard_bounds(total, world)
    assert len(b) == world
    assert b[0][0] == 0 and b[-1][1] == total
    for (lo, hi), (lo2, _) in zip(b, b[1:]):
        assert lo <= hi == lo2
    for lo, _ in b:
        assert lo % 32 == 0
    sizes = [hi - lo for lo, hi in b]
    if total % 32 == 0:
        assert max(sizes) - min(sizes) <= 32


def test_shard_bounds_of_the_6p7b_flat_buffer():
    # 6.7B at 8 ranks: 857,884,672 elements each (858M per rank)
    b = shard_bounds(6_863_077_376, 8)
    assert [hi - lo for lo, hi in b] == [857_884_672] * 8


def test_shard_bounds_rejects_no_ranks():
    with pytest.raises(ValueError):
        shard_bounds(100, 0)


@pytest.mark.parametrize("world", [1, 2, 3, 4, 5, 6, 7, 8, 12, 16, 64, 1000])
def test_dp_prescale_is_torchs_cpu_scalar_reciprocal(world):
    # torch divides a float tensor by a Python number as a multiply by the reciprocal
    # rounded to fp32; on the CPU the same product is checked against torch's own div_
    x = torch.randn(4096, generator=torch.Generator().manual_seed(world)) * 10
    s = dp_prescale(world)
    assert s == float(np.float32(1.0 / world))
    if world & (world - 1) == 0:
        # a power of two: multiply and divide agree exactly
        assert torch.equal(x * s, x / world)


def test_grad_prescale_validation():
    p = [torch.nn.Parameter(torch.zeros(4))]
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            mi_adamw.FusedAdamW(p, grad_prescale=bad)
    with pytest.raises(NotImplementedError):
        mi_adamw.FusedAdamW(p, grad_prescale=0.5, capturable=True)
    opt = mi_adamw.FusedAdamW(p, grad_prescale=1.0 / 3)
    assert opt.grad_prescale == float(np.float32(1.0 / 3))


def test_range_step_needs_the_flat_layout():
    p = [torch.nn.Parameter(torch.zeros(4))]
    with pytest.raises(ValueError):
        ZeroRangeStep(mi_adamw.FusedAdamW(p), 2)


def test_range_step_takes_the_optimizers_prescale():
    """grad_prescale=None takes the optimizer's own pre-scale; an explicit value that
    differs from one the optimizer was built with is refused; over an optimizer without a
    pre-scale an explicit value applies to the ranks' kernels."""
    import types
    flat = types.SimpleNamespace(total=4096, device=torch.device("cpu"))
    third = float(np.float32(1.0 / 3))
    opt = types.SimpleNamespace(_flat=flat, capturable=False, grad_prescale=third)
    assert ZeroRangeStep(opt, 2).grad_prescale == third
    assert ZeroRangeStep(opt, 2, grad_prescale=1.0 / 3).grad_prescale == third
    with pytest.raises(ValueError, match="differs"):
        ZeroRangeStep(opt, 2, grad_prescale=0.5)
    plain = types.SimpleNamespace(_flat=flat, capturable=False, grad_prescale=1.0)
    assert ZeroRangeStep(plain, 2).grad_prescale == 1.0
    assert ZeroRangeStep(plain, 4, grad_prescale=dp_prescale(4)).grad_prescale == 0.25
