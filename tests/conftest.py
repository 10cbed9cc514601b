import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "int8nk_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import Reference, reference_available
    if not reference_available():
        pytest.skip("oracle/_ref (compiled reference) not built here")
    return Reference()


def u8_to_s8(aq_u8: np.ndarray, K: int) -> np.ndarray:
    """Reference activation bytes (q + 128, K-tail pad 0) -> device codes (q, pad 0)."""
    s8 = aq_u8.astype(np.int16) - 128
    s8[:, K:] = 0
    return s8.astype(np.int8)
