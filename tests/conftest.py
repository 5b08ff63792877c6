"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle checks, host logic and C-ABI export checks on the CPU;
``-m gpu`` runs the HIP kernels against the oracle on an MI355X.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "warpstate-ai_amd", ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels)")
