import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def tsn():
    return importlib.import_module("thinksound-native_amd")


@pytest.fixture(scope="session")
def orc():
    import pyoracle
    if not os.path.exists(pyoracle.LIB_PATH):
        pyoracle.build()
    return pyoracle


@pytest.fixture(scope="session")
def rt(tsn):
    r = tsn.Runtime(0)
    yield r
    r.close()


def rel_l2(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    dt = np.complex128 if np.iscomplexobj(a) or np.iscomplexobj(b) else np.float64
    a, b = a.astype(dt), b.astype(dt)
    return float(np.linalg.norm((a - b).ravel()) / max(np.linalg.norm(b.ravel()), 1e-300))


def f16r(a):
    """round to f16 and back (the MFMA operand rounding)"""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def rng(seed):
    return np.random.default_rng(seed)
