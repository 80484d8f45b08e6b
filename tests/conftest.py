import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("friday-inference-engine_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libfriday_attn.so")


@pytest.fixture(scope="session")
def oracle():
    from py_oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def fa():
    import friday_attn
    friday_attn.load()
    return friday_attn


@pytest.fixture(scope="session")
def gpu(fa):
    n = fa.Hip.device_count()
    if n < 1:
        raise RuntimeError("no HIP device visible: GPU tests need an MI355X")
    return fa
