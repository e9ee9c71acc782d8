import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle


def pytest_terminal_summary(terminalreporter):
    """The bf16-bar comparisons of the session: outputs beyond 1e-2 against
    each comparison's cap."""
    from tests.helpers import BAR_LOG

    if not BAR_LOG:
        return
    terminalreporter.write_sep("-", "bf16 bar: outputs beyond 1e-2 / cap (of n)")
    for test, label, over, cap, n, max_abs, fail in BAR_LOG:
        terminalreporter.write_line(f"{over:>5} / {cap:<5} of {n:>9}  max_abs {max_abs:.4g}"
                                    f"{'  FAIL ' + str(fail) if fail else ''}  {test} {label}")
