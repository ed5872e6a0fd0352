import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "tests", "golden")):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmidge_hip.so")


@pytest.fixture(scope="session")
def mh():
    """The HIP library, initialised on device 0 (GPU tests only; no fallback)."""
    import midge_amd
    from midge_amd import _lib
    _lib.load()
    midge_amd.init(0)
    yield midge_amd
    midge_amd.sync()


@pytest.fixture
def path_switch(mh):
    """set(name, on): a library path switch (mh_set_switch) for this test;
    every switch it touched is turned off again at teardown."""
    from midge_amd import set_switch
    used = []

    def set_(name: str, on: bool = True) -> None:
        set_switch(name, on)
        used.append(name)

    yield set_
    for n in used:
        set_switch(n, False)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    d = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (d if d > 0 else 1.0))


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still shows it)."""
    print(f"[case] {msg}", flush=True)
