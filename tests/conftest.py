"""Shared test configuration.

``-m "not gpu"`` runs on any machine: the oracle against closed forms, the host-side allocator
and cache logic, and the C-ABI library's exports (no kernel launch). ``-m gpu`` tests call the
HIP kernels through the C ABI and compare them with the oracle; they need a HIP device and the
in-tree ``libpkv.so`` and fail loudly, not silently, when the library is missing.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

os.environ.setdefault("OMP_NUM_THREADS", "1")

try:  # single-threaded BLAS, as the reference's tests pin it (tests/conftest.py:25 there)
    from threadpoolctl import threadpool_limits

    threadpool_limits(1)
except ImportError:  # pragma: no cover
    pass

from hypothesis import HealthCheck, settings  # noqa: E402

settings.register_profile("dev", max_examples=40, deadline=None)
settings.register_profile(
    "ci", max_examples=200, deadline=None, derandomize=True, suppress_health_check=[HealthCheck.too_slow]
)
settings.load_profile(os.environ.get("HYPOTHESIS_PROFILE", "dev"))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device and the in-tree libpkv.so")


@pytest.fixture(scope="session")
def device():
    """The HIP device the GPU tests run on; skips (with a reason) only when no GPU exists."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device on this machine")
    from paged_kv_serving_amd import _native

    _native.library()  # raises if libpkv.so was not built: no silent fallback
    return torch.device("cuda", 0)

