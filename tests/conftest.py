"""Test configuration: import paths, the `gpu` marker, oracle build."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
for path in (REPO_ROOT, REPO_ROOT / "prism-infer_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import build_oracle

    build_oracle()
    yield


@pytest.fixture(autouse=True)
def _restore_decode_overrides():
    """A test that forces a decode kernel family leaves the process's choice as
    it found it (the automatic choice, or what PRISM_DECODE_* selected)."""

    import ctypes

    from prism_infer import _native

    if not _native.available():
        yield
        return
    saved = (ctypes.c_int * 3)()
    _native.lib().prism_paged_decode_get_overrides(saved)
    yield
    _native.lib().prism_paged_decode_set_overrides(saved[0], saved[1], saved[2])
