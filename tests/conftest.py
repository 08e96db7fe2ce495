import glob
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def golden_names(prefix):
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, prefix + "*.npz")))


@pytest.fixture(scope="session")
def gpu_lib():
    """The built HIP library on a GPU host; a GPU test fails (not skips) without it."""
    from redpanda_amd import _lib
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    return _lib.load()


@pytest.hookimpl(trylast=True)
def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line per parity test (its worst figures), recorded by the tests
    through record_property("parity", ...), printed even under -q so that
    a run's log carries the numbers and not only the pass count."""
    lines = []
    for key in ("passed", "failed"):
        for rep in terminalreporter.stats.get(key, []):
            if getattr(rep, "when", "call") != "call":
                continue
            for name, value in getattr(rep, "user_properties", ()):
                if name == "parity":
                    lines.append(("" if key == "passed" else "FAILED ") + str(value))
    if lines:
        terminalreporter.write_sep("-", "parity figures (max|a-b|/max|b| per tensor)")
        for line in lines:
            terminalreporter.write_line(line)
