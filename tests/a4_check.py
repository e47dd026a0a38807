"""Accuracy bar of the W4A4 ops against the exact (float64) LUT sum; shared by the GPU parity tests and
the CPU test that pins the bar itself (tests/test_oracle.py)."""

import numpy as np
import torch

import oracle


def a4_exact_check(y, ref32, exact, K):
    """W4A4 accuracy bar: at the reference's test sizes (K = 11 and 27 there;
    here K <= 128) its own tolerance against the oracle's fp32 LUT loop
    (rtol = atol = 1e-5, test_cuda_ops.py:64,93); at every size, the
    deviation from the exact (float64) value of s * sum_k C[w] (a - zp) + b is
    at most twice the deviation of that fp32 LUT loop (the reference's
    arithmetic) plus 1e-6 max|exact|: over K in the hundreds and millions of
    outputs, fp32 summation order alone moves some sums by more than 1e-5, in
    the reference as here."""
    y = y.detach().cpu().double()
    ref32 = torch.as_tensor(ref32).double()
    if K <= 128:
        torch.testing.assert_close(y.float(), ref32.float(), rtol=1e-5, atol=1e-5)
    err = (y - exact).abs().max().item()
    err_ref = (ref32 - exact).abs().max().item()
    assert err <= 2 * err_ref + 1e-6 * exact.abs().max().item(), (err, err_ref)


def a4_levels(x, scale, zp):
    """s * (a - zp) in float64, a = the reference's u4 activation code (oracle)."""
    a = torch.from_numpy(oracle.quantize_act_u4(x.float(), scale, zp).astype(np.int64))
    return scale * (a - zp).double()
