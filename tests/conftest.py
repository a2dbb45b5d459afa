import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size model shapes")


@pytest.fixture(scope="session")
def oracle_threads():
    """Run the oracle's pool on up to 16 host cores (results do not depend on it)."""
    import oracle
    n = min(16, os.cpu_count() or 1)
    oracle.oracle_lib().orc_threads_init(n)
    yield n
    oracle.oracle_lib().orc_threads_shutdown()
