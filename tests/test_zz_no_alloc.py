"""The no-allocation linear_lut entry point (dimq_linear_lut_noalloc) against
the workspace entry point it mirrors (dimq_linear_lut_ws), through the C ABI:
two calls in a row on the shared scratch, the second with a smaller input,
must give the workspace path's bits; sizes beyond the scratch are refused."""

import pytest
import torch

import oracle
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _case(g, M, N, K, dev):
    x = torch.randn(M, K, generator=g).to(dev)
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4)).to(dev)
    cb = torch.linspace(-0.5, 0.5, 16).half().to(dev)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    return x, packed, cb, bias


def _run(lib, C, fn, x, packed, cb, bias, M, N, K, ws=None):
    y = torch.full((M, N), float("nan"), device=x.device)
    s = torch.cuda.current_stream().cuda_stream
    args = [x.data_ptr(), C.F32, M, packed.data_ptr(), packed.numel(), cb.data_ptr(), C.F16, 16, 0.25, 8,
            bias.data_ptr(), C.F32, N, N, K, y.data_ptr()]
    if fn == "ws":
        rc = lib.dimq_linear_lut_ws(*args, ws.data_ptr(), ws.numel(), s)
    else:
        rc = lib.dimq_linear_lut_noalloc(*args, s)
    assert rc == 0, lib.dimq_last_error()
    return y


def test_linear_lut_noalloc_matches_workspace_path(gpu):
    from dimq_amd import _C
    lib = _C.lib
    g = torch.Generator().manual_seed(5)
    for M, N, K in ((1576, 384, 768), (37, 96, 256)):  # second call smaller: the scratch keeps the first's bytes
        announce(f"linear_lut_noalloc M={M} N={N} K={K}")
        x, packed, cb, bias = _case(g, M, N, K, gpu)
        ws = torch.empty(lib.dimq_linear_lut_workspace_bytes(M, K, _C.F16), dtype=torch.uint8, device=gpu)
        y_ws = _run(lib, _C, "ws", x, packed, cb, bias, M, N, K, ws)
        y_na = _run(lib, _C, "noalloc", x, packed, cb, bias, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ws), (M, N, K)


def test_linear_lut_noalloc_rejects_sizes_beyond_its_scratch(gpu):
    from dimq_amd import _C
    lib = _C.lib
    K = 1024
    M = 8 * 1024 + 1  # M * K = 8,389,632 > 8,388,608 fp16 activations
    rc = lib.dimq_linear_lut_noalloc(None, _C.F32, M, None, 64 * K, None, _C.F16, 16, 0.25, 8, None, 0, 0, 128, K,
                                     None, None)
    assert rc == 1
    assert b"exceeds the scratch limit" in lib.dimq_last_error()
