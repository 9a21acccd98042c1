import sys
from pathlib import Path

import pytest
import torch  # noqa: F401  (load torch's HIP runtime before libsnhip.so)

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def gpu():
    """Skip only when there is no GPU at all; a missing library is an error."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from sunnynet_amd import _native
    _native.lib()   # raises if libsnhip.so is missing
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ref_built():
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent at build time)")
    return True
