"""GPU: the ctypes stub of the repository's integration guide, run as written.

The stub binds libmi_adamw.so with ctypes alone (no mi_adamw package) and steps
one flat range.  Its result must equal FusedAdamW's on the same tensors, bit for
bit, so the documented binding cannot drift from the library.
"""
from __future__ import annotations

import os
import re

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_integration_ctypes_stub_matches_fusedadamw():
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    import mi_adamw
    from mi_adamw.optimizer import _hyper
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = re.search(r"### ctypes stub.*?```python\n(.*?)```", text, re.S).group(1)
    lib_path = os.path.join(ROOT, "mini-megatron_amd", "mi_adamw", "libmi_adamw.so")
    assert 'ctypes.CDLL("libmi_adamw.so")' in block
    ns: dict = {}
    exec(block.replace('ctypes.CDLL("libmi_adamw.so")', f"ctypes.CDLL({lib_path!r})"), ns)
    dev = torch.device("cuda", 0)
    n = (1 << 20) + 3
    p = torch.randn(n, device=dev) * 0.02
    g = torch.randn(n, device=dev) * 1e-3
    q = torch.nn.Parameter(p.clone())
    q.grad = g.clone()
    opt = mi_adamw.FusedAdamW([q], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    opt.step()
    m, v = torch.zeros(n, device=dev), torch.zeros(n, device=dev)
    hy = _hyper(opt.param_groups[0], 1.0)
    ns["step_flat"](p, g, m, v, ns["Hyper"](*[getattr(hy, f) for f, _ in ns["Hyper"]._fields_]))
    torch.cuda.synchronize()
    assert torch.equal(p, q.detach())
    assert torch.equal(m, opt.state[q]["exp_avg"]) and torch.equal(v, opt.state[q]["exp_avg_sq"])
