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


def out_tol(dtype) -> float:
    """Parity bar of a weight-only GEMM/conv output in `dtype`: max|err| / max|ref| <= 2e-3 (fp32
    accumulation) plus the one rounding of the result to a 16-bit output, which alone moves an element by up
    to 2^-9 (bf16) or 2^-11 (fp16) of its magnitude."""
    import torch

    return 2e-3 + {torch.bfloat16: 2.0 ** -9, torch.float16: 2.0 ** -11}.get(dtype, 0.0)
