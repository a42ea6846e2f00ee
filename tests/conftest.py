"""Test configuration: import paths and the `gpu` marker.

CPU tests (`-m "not gpu"`) cover the oracle, the host-side page owner and
the C ABI's loading and argument checks.  GPU tests (`-m gpu`) run the HIP
kernels through the C ABI and the torch ops and compare them with the
oracle."""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "branchcraft-cuda_amd" / "python", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def compiled_kernels(tmp_path_factory):
    """gfx950 device assembly of decode.hip and tree_verify.hip, built with
    the library's flags: {source: {kernel symbol: lines}}."""
    import shutil

    import asm_hazards as H
    if not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()):
        pytest.skip("hipcc not available")
    tmp = tmp_path_factory.mktemp("asm")
    return {src: H.kernels(H.compile_device_asm(H.CSRC / src, tmp))
            for src in ("decode.hip", "tree_verify.hip")}


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle_c
    oracle_c.lib()
    return oracle_c
