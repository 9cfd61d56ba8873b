"""pytest configuration: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X (they call the HIP library through the C
ABI); everything else runs on the CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "yasakani-for-mac_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); parity tests through the C ABI")
