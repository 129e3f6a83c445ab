"""pytest configuration: import paths and the `gpu` marker.

Tests marked `gpu` need a ROCm GPU (an MI355X) and libmi_adamw.so built for
gfx950; everything else runs on the CPU.  The oracle under oracle/ is test
infrastructure: tests import it as the checker only.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "mini-megatron_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
