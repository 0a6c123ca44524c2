import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")
    config.addinivalue_line("markers", "slow: full-size model (minutes of CPU or large GPU memory)")


@pytest.fixture(scope="session")
def tmpdir_session(tmp_path_factory):
    return tmp_path_factory.mktemp("qpack")


@pytest.fixture(scope="session")
def synth(tmpdir_session):
    """synth(name, seed) -> path of a cached synthetic QPACK2 file"""
    import qpack_amd
    cache = {}

    def make(name, seed=1234):
        key = (name, seed)
        if key not in cache:
            p = str(tmpdir_session / f"{name}_{seed}.qpack")
            qpack_amd.write_synthetic(name, p, seed=seed)
            cache[key] = p
        return cache[key]
    return make
