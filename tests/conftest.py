import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libchatnet_hip.so")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    try:
        from gpu_util import GREEDY_RECORDS
    except ImportError:
        return
    if not GREEDY_RECORDS:
        return
    terminalreporter.section("greedy identity vs the oracle")
    for case, same, steps, forced, mm in GREEDY_RECORDS:
        terminalreporter.write_line(f"{case}: {same}/{steps} identical, {forced} near-tie steps teacher-forced, "
                                    f"min oracle margin {mm:.3g}")
