import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libdimq_hip.so")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a HIP device (run with -m 'not gpu')")
    from dimq_amd import _C  # noqa: F401  (fails loudly if the library is missing)

    return torch.device("cuda:0")


def announce(name: str) -> None:
    """Print and flush the case name before a GPU step, so a crash names its case."""
    print(f"[case] {name}", flush=True)
