"""pytest configuration: the `gpu` marker and import paths.

GPU tests (`-m gpu`) need an MI355X and the built libhipbackend.so; every
other test runs on the CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "laya-js_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) and the built HIP library")
