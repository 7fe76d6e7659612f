import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

# Lines that tests report for the run's summary (printed even under -q).
_REPORT = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def pytest_terminal_summary(terminalreporter):
    if _REPORT:
        terminalreporter.section("whallm_amd results")
        for line in _REPORT:
            terminalreporter.write_line(line)


@pytest.fixture(scope="session")
def report():
    """report(line): add a line to the summary printed at the end of the run."""
    return _REPORT.append


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o
