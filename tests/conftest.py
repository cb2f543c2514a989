import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    """One pbx context for the whole GPU session (one process, one GPU)."""
    from purebee_amd import Context
    c = Context(0)
    name, cus = c.device_info()
    print(f"\n[pbx] device: {name}, {cus} CUs", flush=True)
    yield c
    c.close()


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def synth_matrix(seed, N, K, std=0.02):
    from purebee_amd import synth_normal
    return synth_normal(seed, N * K, 0.0, std).reshape(N, K)
