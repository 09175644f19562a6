"""Shared pytest configuration: the `gpu` marker and import paths.

The product package lives in ``qwen2-int4-systems_amd/`` (a source root, like
the reference's ``src/``); the oracle package is ``oracle/`` at the repo root.
"""

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = REPO_ROOT / "qwen2-int4-systems_amd"
for path in (REPO_ROOT, PACKAGE_ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def c_oracle():
    from oracle.oracle import COracle, build_c_oracle

    try:
        return COracle()
    except FileNotFoundError:
        build_c_oracle()
        return COracle()
