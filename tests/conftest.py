"""Shared pytest setup: markers, import paths, a session GPU device."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
for p in (REPO, os.path.join(REPO, "draw-instant_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libdrawinstant_hip.so)")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def dev():
    import drawinstant
    d = drawinstant.Device(0)
    print(f"[dev] cus={d.num_cus} clock_khz={d.clock_khz} hbm={d.hbm_bytes >> 30} GiB", flush=True)
    yield d
    d.sync()
    d.destroy()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def max_rel(got, ref):
    """max |got-ref| / max(1, |ref|): the per-element metric of the fp32 gate."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))))
