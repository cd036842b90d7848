"""Shared test setup: import paths, the `gpu` marker, device fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "thrml-rs_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libthrml_hip.so)")


@pytest.fixture(scope="session")
def device():
    import thrml_hip

    dev = thrml_hip.Device(0)
    yield dev
    dev.close()


def log_case(msg):
    """Name the case before a GPU step (flushed, so a crash still shows it)."""
    print(f"[case] {msg}", flush=True)
