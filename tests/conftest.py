import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU: a missing device is a failure, not a skip")
    # The library is built for gfx950 only (as the reference's device test insists on its target arch,
    # ROCmKernels.Tests/DeviceTests.cpp:14-25): any other device is a failure, not a silent mismatch.
    arch = torch.cuda.get_device_properties(0).gcnArchName
    if not arch.startswith("gfx950"):
        pytest.fail(f"GPU tests need an MI355X (gfx950); device 0 is {arch}")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Parity headroom: the checks of tests/parity.py that came closest to their tolerance in this run."""
    try:
        import parity
    except ImportError:
        return
    if not parity.RECORDS:
        return
    worst = {}
    for label, quantity, err, tol in parity.RECORDS:
        if quantity not in worst or err / tol > worst[quantity][1] / worst[quantity][2]:
            worst[quantity] = (label, err, tol)
    terminalreporter.write_sep("-", f"parity headroom over {len(parity.RECORDS)} checks (largest error per quantity)")
    for quantity in sorted(worst):
        label, err, tol = worst[quantity]
        terminalreporter.write_line(f"{quantity:>16}: {err:.3e} of {tol:.0e} ({100 * err / tol:5.1f}% of tolerance)  [{label}]")
