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


import pytest  # noqa: E402


@pytest.fixture(autouse=True)
def _split_path_by_default(monkeypatch):
    """By the library's own rule, small shapes run as one launch (one workgroup
    per (sequence, KV head), no split workspace, no merge).  Tests of the split
    kernels, the work queue and the merge pin the split path here; the tests of
    the single launch ask for it (L20_PD_FUSED=1) or for the library's choice
    (the variable removed).  Likewise the single-launch kernel's split mode
    (512-token splits whose triples fill the CUs once) is off unless a test
    asks for it (L20_PD_FUSED_SPLIT=1) or for the library's choice."""
    monkeypatch.setenv("L20_PD_FUSED", "0")
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "0")
