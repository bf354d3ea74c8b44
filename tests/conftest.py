"""Shared pytest setup: markers and import paths.

``-m "not gpu"`` runs on any CPU host; ``-m gpu`` needs an MI355X.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "single-gpu-inference-lab_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")
