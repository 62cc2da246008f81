import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "wg-kv_amd"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    import parity_log
    if parity_log.LINES:
        terminalreporter.section("parity counts")
        for line in parity_log.LINES:
            terminalreporter.write_line(line)


def pytest_collection_modifyitems(config, items):
    # GPU tests run in file order, but keep every CPU-only check before them.
    items.sort(key=lambda it: 1 if it.get_closest_marker("gpu") else 0)
