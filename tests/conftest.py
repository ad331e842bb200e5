"""Shared pytest setup: import paths, the `gpu` marker and Hypothesis profiles.

CPU tests (`-m "not gpu"`) pin the oracle against the reference's known answers and recorded
outputs, and test the host logic and the C ABI without launching anything.  GPU tests
(`-m gpu`) compare the HIP library with the oracle on the same seeded inputs.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT, ROOT / "proof-carrying-kernels_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

from hypothesis import HealthCheck, settings  # noqa: E402

settings.register_profile(
    "default", deadline=None, suppress_health_check=[HealthCheck.too_slow], max_examples=60
)
settings.register_profile(
    "ci", parent=settings.get_profile("default"), max_examples=300, derandomize=True
)
settings.load_profile(os.environ.get("HYPOTHESIS_PROFILE", "default"))


def pytest_configure(config) -> None:  # type: ignore[no-untyped-def]
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpck_hip.so)")
    config.addinivalue_line("markers", "slow: long CPU reproduction of a recorded output")
