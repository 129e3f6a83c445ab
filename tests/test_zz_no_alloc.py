"""mi_adamw_grad_norm_flat_noalloc against mi_adamw_grad_norm_flat, through the C ABI.

The no-alloc entry point keeps its partial sums in the library's static device
scratch instead of a caller's workspace.  It must give the same norm and clip
coefficient bit for bit, call after call: the scratch keeps the previous call's
partials, so a second, smaller call (fewer norm workgroups) must not read stale
ones.  The sizes cross the norm pass's 512-workgroup cap (2,100,000 elements at
4096 per chunk are 513 chunks), then drop below it, then reach the scalar path
(a gradient view one element off 16-byte alignment).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _norm_pair(lib, g: torch.Tensor, max_norm: float):
    from mi_adamw import _lib
    dev = g.device
    stream = torch.cuda.current_stream(dev).cuda_stream
    partials = torch.full((_lib.MAX_NORM_BLOCKS,), float("nan"), dtype=torch.float64, device=dev)
    out = torch.full((4,), float("nan"), dtype=torch.float32, device=dev)
    n = g.numel()
    _lib.check(lib.mi_adamw_grad_norm_flat(g.data_ptr(), n, 4096, max_norm, partials.data_ptr(),
                                           out[0:1].data_ptr(), out[1:2].data_ptr(), stream),
               "mi_adamw_grad_norm_flat")
    _lib.check(lib.mi_adamw_grad_norm_flat_noalloc(g.data_ptr(), n, 4096, max_norm,
                                                   out[2:3].data_ptr(), out[3:4].data_ptr(),
                                                   stream),
               "mi_adamw_grad_norm_flat_noalloc")
    torch.cuda.synchronize(dev)
    return out.cpu()


def test_noalloc_norm_equals_workspace_norm_on_successive_calls():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    from mi_adamw import _lib
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(77)
    big = torch.randn(2_100_000, device=dev, generator=gen) * 1e-2
    small = torch.randn(1_000_003, device=dev, generator=gen) * 3.0
    ragged = torch.randn(40_001, device=dev, generator=gen)[1:]        # misaligned view
    cases = [("2.1M elements, 513 chunks", big, 1.0),
             ("1.0M elements, 245 chunks", small, 1.0),
             ("40,000 elements, misaligned", ragged, 1e9)]
    for label, g, max_norm in cases:
        print(f"[no-alloc] {label}", flush=True)
        r = _norm_pair(lib, g, max_norm)
        exact = float(g.double().pow(2).sum().sqrt())
        print(f"[no-alloc] {label}: norm {r[0].item():.9g} / {r[2].item():.9g} "
              f"(float64 {exact:.12g}), coef {r[1].item():.9g} / {r[3].item():.9g}", flush=True)
        assert torch.equal(r[0:2].view(torch.int32), r[2:4].view(torch.int32)), label
        assert abs(r[2].item() - exact) <= 1e-6 * exact
    # the coefficient path: the last case does not clip, the first two do
    assert _norm_pair(lib, ragged, 1e9)[3].item() == 1.0
    assert _norm_pair(lib, big, 1.0)[3].item() < 1.0


def test_noalloc_rejects_bad_arguments_before_any_launch():
    from mi_adamw import _lib
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    g = torch.ones(8, device=dev)
    out = torch.zeros(2, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    assert lib.mi_adamw_grad_norm_flat_noalloc(g.data_ptr(), 0, 4096, 1.0, out.data_ptr(),
                                               out.data_ptr() + 4, stream) == _lib.E_INVALID
    assert lib.mi_adamw_grad_norm_flat_noalloc(g.data_ptr(), 8, 1000, 1.0, out.data_ptr(),
                                               out.data_ptr() + 4, stream) == _lib.E_INVALID
    assert lib.mi_adamw_grad_norm_flat_noalloc(None, 8, 4096, 1.0, out.data_ptr(),
                                               out.data_ptr() + 4, stream) == _lib.E_INVALID
    assert lib.mi_adamw_grad_norm_flat_noalloc(g.data_ptr(), 8, 4096, 1.0, None,
                                               out.data_ptr() + 4, stream) == _lib.E_INVALID
    assert b"scratch" in lib.mi_adamw_strerror(_lib.E_SCRATCH)
