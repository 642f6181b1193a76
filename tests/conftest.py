import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "amdgpu-arch-gemm_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path")


@pytest.fixture(scope="session")
def kernels():
    """Names of the built catalog instances; fails (never skips) if they are missing."""
    from generator import catalog
    missing = [n for n in catalog.SOLUTIONS if not os.path.exists(catalog.paths(n)[0])]
    if missing:
        pytest.fail(f"kernel code objects missing ({missing[:3]}...): run __graft_entry__.build()")
    return list(catalog.SOLUTIONS)
