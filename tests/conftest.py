"""Test configuration: import paths, the `gpu` marker, a session-wide device."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "gpt2-opencl-1.1_amd"), ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="session")
def g2():
    """The HIP library initialised on device 0 (GPU tests only)."""
    import g2hip

    g2hip.init(0)
    name, cus = g2hip.device_name()
    print(f"\n[g2] device {name} with {cus} CUs", flush=True)
    yield g2hip
    g2hip.sync()
    import gc

    gc.collect()  # models and buffers the tests dropped are freed while the library is up
    g2hip.shutdown()


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The greedy-identity record of every full-depth run, so a quiet run
    (pytest -q) still states how many ids agreed with the oracle."""
    try:
        from parity import IDENTITY_RECORDS
    except ImportError:
        return
    if IDENTITY_RECORDS:
        terminalreporter.section("greedy identity against the oracle (full depth)")
        for line in IDENTITY_RECORDS:
            terminalreporter.write_line(line)
