import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "strim-engine_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(autouse=True)
def _tie_ledger(request):
    """Points the fp-tie ledger of the GPU checks at the running test."""
    import gpu_util

    gpu_util.TIE_LEDGER["current"] = request.node.nodeid
    yield


def pytest_terminal_summary(terminalreporter):
    """Rows and sequences whose token differed from the oracle's at a documented fp tie
    (oracle margin below TIE_EPS), per test: every excused row is listed here."""
    import gpu_util

    rows = gpu_util.TIE_LEDGER["rows"]
    checked = gpu_util.TIE_LEDGER["checked"]
    if not checked:
        return
    tot = sum(rows.values())
    terminalreporter.write_line(
        f"fp-tie exemptions: {tot} of {sum(checked.values())} compared rows/sequences "
        f"in {len(rows)} of {len(checked)} tests")
    for k, v in sorted(rows.items()):
        terminalreporter.write_line(f"  {v} of {checked[k]} in {k}")


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
