"""Shared pytest setup: repo root on sys.path, the ``gpu`` marker, oracle build."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs on the GPU box")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    so = os.path.join(ROOT, "oracle", "liboracle_kv.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; fails (never skips) when the library or the GPU is missing."""
    import atomflow_amd
    from atomflow_amd import device

    atomflow_amd.lib()
    n = device.device_count()
    assert n >= 1, "no HIP device visible: the -m gpu tests must run on the GPU box"
    info = device.device_info()
    print(f"[gpu] {info}", flush=True)
    return info
