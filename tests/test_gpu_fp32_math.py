"""GPU: the update kernels' fp32 helpers against the forms they replace.

``mini-megatron_amd/mi_adamw/csrc/fp32_math.h`` holds
- ``bf16x2_bits``: gfx950's packed bf16 conversion with NaN mapped to 0x7FC0, used for
  every bf16 moment and bf16 copy the update stores;
- ``div_by_recip``: the fused=True chain's quotient sqrtf(v) / bc2_sqrt, formed from a
  per-workgroup reciprocal with one fma correction instead of a division;
- ``div_by_neg_recip``: the same for the capturable chain's negative divisor
  sqrt(bc2) * -step_size, used while it lies in [2^-62, 2^50] in magnitude.

All must equal the slower forms bit for bit.  ``tests/c/fp32_math_check`` (built from
that header by ``__graft_entry__.build()``) checks the conversion on all 2^32 fp32
patterns against round-to-nearest-even on the integers, the device's fp32 division
against the host's IEEE division, and the quotient against that division at every
exponent pairing the chain can give (sampled, with 0, -0, inf and NaN) and on every
pair of significands (2^46 pairs, which with the exact scaling of its roundings covers
every quotient the kernel forms); and the negative-divisor form over its whole range
(sampled) and on an eighth of the significand pairs (its nonzero results are exact
negations of the positive form's).
"""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "fp32_math_check")


def test_fp32_helpers_equal_the_forms_they_replace():
    if not os.path.exists(BIN):
        pytest.fail("tests/c/fp32_math_check is not built: run __graft_entry__.build()")
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "fp32_math_check: ok" in res.stdout
    assert "significand pairs (128 of 128 launches): 0 differ" in res.stdout
    assert "div_by_neg_recip, significand pairs (16 launches): 0 differ" in res.stdout
