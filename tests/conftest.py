"""pytest configuration: the `gpu` marker and repo-root imports.

Tests marked ``gpu`` need an MI355X (gfx950) and the built HIP library; they
run with ``-m gpu`` on the GPU box and fail loudly when the library or the
device is missing.  Everything else runs on the CPU here.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP code objects")
