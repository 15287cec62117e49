"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"``: the oracle against the reference's fixtures and mathematics,
host-side validation (meta tensors), and that the C-ABI library loads and
exports every symbol of include/cascade_kernels.h.
``-m gpu``: parity of the HIP kernels (through the C ABI and the torch ops)
against the oracle on seeded inputs.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "vllm-hust-cascade-kernel_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_terminal_summary(terminalreporter):
    """Per-case error margins of the parity tests that record them: the measured
    max error next to the tolerance it is held to."""
    from tests._util import MARGINS
    if not MARGINS:
        return
    tr = terminalreporter
    tr.write_sep("-", "parity margins (max error / bound)")
    for case, oe, ob, le, lb in MARGINS:
        lse = "" if le is None else "  LSE rel %.2e / %.0e" % (le, lb)
        tr.write_line("%-48s O %.3e / %.0e (%5.1f%%)%s" % (case, oe, ob, 100.0 * oe / ob, lse))


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture
def no_wait_giveups():
    """GPU tests of the suffix / fused cascade kernels: none of their bounded
    waits may run out during the test (ck_wait_giveups stays 0)."""
    import torch
    from cascade_amd import abi
    torch.cuda.synchronize()
    abi.wait_giveups(reset=True)
    yield
    torch.cuda.synchronize()
    assert abi.wait_giveups() == 0, "a bounded wait in the suffix / cascade kernels ran out"
