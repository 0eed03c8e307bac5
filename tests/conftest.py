"""Test configuration: import paths, the ``gpu`` marker and shared fixtures.

``-m "not gpu"`` runs on any machine (oracle, golden vectors, host logic, the
C ABI's symbols).  ``-m gpu`` runs the parity tests proper on an MI355X: every
GPU test calls libglm_moe through its C ABI and compares with the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "glm-tpu_amd", ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libglm_moe.so")


def pytest_terminal_summary(terminalreporter):
    """Print every closeness check's measured flips beside its bounds (also under -q)."""
    import closeness

    lines = closeness.summary_lines()
    if lines:
        terminalreporter.section("parity against the oracle")
        for line in lines:
            terminalreporter.write_line(line)


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from glm_moe import _lib

    _lib.lib()  # fail loudly if the HIP library is missing: there is no fallback
    return torch.device("cuda:0")
