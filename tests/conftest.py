"""Test configuration: the `gpu` marker and shared helpers.

CPU tests (-m "not gpu") cover the oracle against the reference's
known-answer tests and the golden fixtures, the host logic, and the C ABI's
exported symbols.  GPU tests (-m gpu) run the HIP kernels through the C ABI
and compare them with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")
if GOLDEN_DIR not in sys.path:
    sys.path.insert(0, GOLDEN_DIR)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: large shapes (minutes on CPU)")


def _ensure_built():
    # load what is built; build only when nothing is
    import cima_amd.build as b
    import oracle

    b.ensure()
    oracle.build()


_ensure_built()


@pytest.fixture(scope="session")
def hip():
    """One HipCtx on device 0, launching on torch's current stream."""
    import torch
    from cima_amd.hip import HipCtx

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    ctx = HipCtx(0)
    ctx.use_torch_stream()
    yield ctx
    torch.cuda.synchronize()
    ctx.close()
