import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "refinekv-release_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    return oracle


def pytest_terminal_summary(terminalreporter):
    """Near-eps exceptions of the golden mask comparisons: blocks whose
    reduced risk lies within 1e-6 relative of eps (where a reordered fp32 sum
    may decide either way) and how many of them differed."""
    near = diff = cases = 0
    for report in terminalreporter.stats.get("passed", []) + terminalreporter.stats.get(
            "failed", []):
        props = dict(getattr(report, "user_properties", []))
        if "near_eps_blocks" in props and report.when == "call":
            cases += 1
            near += props["near_eps_blocks"]
            diff += props.get("near_eps_mask_differences", 0)
    if cases:
        terminalreporter.write_line(
            f"near-eps blocks over {cases} golden mask cases: {near} within 1e-6 relative of "
            f"eps; {diff} mask entries differ from the golden masks (only near-eps entries may)")
