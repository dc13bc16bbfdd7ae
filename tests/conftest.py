import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the GPU)")


@pytest.fixture
def kq_env(monkeypatch):
    """Sets KQ_* launch-shape overrides for one test: the library reads them
    once, so each change is followed by kq_tuning_reload, and the previous
    environment is restored and re-read when the test ends."""
    import stratum_amd as K

    def set_env(**kv):
        for k, v in kv.items():
            monkeypatch.setenv(k, str(v))
        K.reload_tuning()
    yield set_env
    monkeypatch.undo()
    K.reload_tuning()


@pytest.fixture(scope="session")
def port():
    from oracle import oracle as O
    return O.port()


@pytest.fixture(scope="session")
def ref():
    from oracle import oracle as O
    r = O.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    return r


def load_golden(name: str):
    """{case: {w, x, shape, deq, y}} from tests/golden/<name>.npz."""
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    cases = {}
    for key in z.files:
        case, field = key.split("_", 1)
        cases.setdefault(case, {})[field] = z[key]
    return cases


GOLDEN_FILES = {12: "q4k", 14: "q6k", 10: "q2k", 42: "q2k_nib", 13: "q5k", 11: "q3k", 8: "q8_0"}


def same_values(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-for-bit equality, except that any NaN equals any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))
