import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "strim-engine_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    import torch
    from strim_amd import ops

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = ops.Context(0, max_rows=8192, max_vocab=262144)
    yield c
    c.close()
