"""The C ABI from a plain C host (tests/c/abi_check.c, built by __graft_entry__.build()).

CPU: version, error text, the chunk-table helper and the argument rejections
that return before any launch.  GPU: flat clip, tensor/chunk tables with bf16
state and copy, amsgrad, the capturable chain, the clip split over slices with
the data-parallel pre-scale (and the no-alloc norm), gradient pointers patched
into a table, and torch's fused=True chain (flat with the clip, tables, device step
counts and lr), each bit-exact against the C oracle.
"""
from __future__ import annotations

import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "abi_check")


def _run(mode: str) -> str:
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built; run __graft_entry__.build() first")
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_c_host_cpu_checks():
    assert "abi_check cpu: ok" in _run("cpu")


@pytest.mark.gpu
def test_c_host_gpu_parity_against_oracle():
    out = _run("gpu")
    assert out.count("bit-exact") == 7 and "abi_check gpu: ok" in out
