"""Chained W4A4 layers with the next layer's activation quantization fused into the producing layer's epilogue.

Activations travel between layers as the fp16 integers a - zp.  A layer's codes must be the reference's u4 codes
(reference.py:11-21) of its own fp32 result -- except where that result sits on a rounding tie, which fp32
summation order may put on either side -- and the last layer's float output must meet the W4A4 accuracy bar
against the exact (float64) sum over the codes it was given."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests.a4_check import a4_exact_check, a4_levels
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _ops():
    from dimq_amd import ops
    return ops


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _layer(N, K, g):
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    cb = (torch.linspace(-0.4, 0.45, 16) * (1.0 / K ** 0.5) * 4 + 0.002 * torch.randn(16, generator=g)).half()
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    bias = torch.randn(N, generator=g) * 0.05
    return idx, cb, packed, bias


def _codes(y, s, zp):
    """fp32 tensor of the reference's q - zp for the float values y."""
    q = oracle.quantize_act_u4(torch.as_tensor(y).float(), s, zp).astype(np.float32)
    return torch.from_numpy(q - zp).reshape(torch.as_tensor(y).shape)


def _check_codes(codes, y_exact, s, zp):
    """GPU codes against the codes of the exact result: equal except within 1e-3 of a rounding tie, and never more
    than one step apart."""
    ref = _codes(y_exact.float(), s, zp)
    got = codes.detach().cpu().float()
    t = y_exact.double() / s
    near_tie = ((t - torch.floor(t)) - 0.5).abs() < 1e-3
    assert bool(((got == ref) | near_tie).all()), int((got != ref).sum())
    assert float((got - ref).abs().max()) <= 1.0
    assert float((got != ref).float().mean()) < 1e-3


def test_quantize_activation_f16_matches_reference_codes(gpu):
    ops = _ops()
    x = torch.randn(7, 1001, generator=_gen(3)) * 3
    x[0, :5] = torch.tensor([float("nan"), float("inf"), float("-inf"), 1e30, -1e30])
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        for s, zp in ((0.2, 7), (2.0 ** -3, 8), (0.05, 0)):
            q = ops.quantize_activation_f16(x.to(dt).to(gpu), s, zp)
            assert q.dtype == torch.float16 and q.shape == x.shape
            assert torch.equal(q.cpu().float(), _codes(x.to(dt).float(), s, zp))
            # a view one element into its storage: the element-wise (unaligned) loads
            xv = x.to(dt).to(gpu).flatten()[1:]
            qv = ops.quantize_activation_f16(xv, s, zp)
            assert torch.equal(qv.cpu().float(), _codes(x.to(dt).flatten()[1:].float(), s, zp))


def test_quantize_codes_at_rounding_ties(gpu):
    """The kernels form x / s as x * RN(1/s) and fall back to the IEEE quotient near ties: values within a few
    ulps of every tie k + 0.5, for scales that are and are not powers of two, give the oracle's codes."""
    ops = _ops()
    g = _gen(11)
    scales = [0.2, 0.1, 2.0 ** -3, 0.0731, 1.7, 3e-5, 1234.5] + (torch.rand(20, generator=g) * 2).tolist()
    k = torch.arange(-20, 21, dtype=torch.float32) + 0.5
    for s in scales:
        s = float(np.float32(s))
        base = (k * np.float32(s)).numpy().astype(np.float32)
        cand, up, dn = [base], base, base
        for _ in range(64):  # up to 64 ulps on either side of each tie
            up = np.nextafter(up, np.float32(np.inf), dtype=np.float32)
            dn = np.nextafter(dn, np.float32(-np.inf), dtype=np.float32)
            cand += [up, dn]
        x = torch.from_numpy(np.concatenate(cand + [np.linspace(-20 * s, 20 * s, 4001, dtype=np.float32)]))
        for zp in (0, 7, 15):
            q = ops.quantize_activation_u4(x.to(gpu), s, zp).cpu().numpy()
            assert np.array_equal(q, oracle.quantize_act_u4(x, s, zp)), (s, zp)
            qf = ops.quantize_activation_f16(x.to(gpu), s, zp).cpu().float()
            assert torch.equal(qf, _codes(x, s, zp)), (s, zp)


@pytest.mark.parametrize("M,K1,N1,N2,act", [
    (4, 4096, 256, 192, "relu"),     # decode shape: streamed GEMV, runtime epilogue
    (300, 768, 512, 256, "relu"),    # 128x128 tiles with the quantizing mode
    (2100, 768, 512, 256, "gelu"),   # 256x256 shared-decode tile with the quantizing mode
    (37, 96, 130, 40, None),         # generic tiles
])
def test_linear_lut_q_chain(gpu, M, K1, N1, N2, act):
    ops = _ops()
    announce(f"linear_lut_q chain M={M} K1={K1} N1={N1} N2={N2} {act}")
    g = _gen(M + K1 + N1)
    idx1, cb1, p1, b1 = _layer(N1, K1, g)
    idx2, cb2, p2, b2 = _layer(N2, N1, g)
    s1, zp1, s2, zp2 = 0.125, 7, 0.0625, 3
    x = torch.randn(M, K1, generator=g)
    xq = ops.quantize_activation_f16(x.to(gpu), s1, zp1)
    c2 = ops.dimq_linear_lut_q(xq, p1.to(gpu), cb1.to(gpu), s1, b1.to(gpu), N1, K1, activation=act,
                               out_act=(s2, zp2))
    assert c2.dtype == torch.float16 and c2.shape == (M, N1)
    y1 = a4_levels(x, s1, zp1) @ cb1.double()[idx1.long()].T + b1.double()
    y1 = torch.relu(y1) if act == "relu" else (F.gelu(y1) if act == "gelu" else y1)
    _check_codes(c2, y1, s2, zp2)
    # the second layer on the codes it was given, float output
    y2 = ops.dimq_linear_lut_q(c2, p2.to(gpu), cb2.to(gpu), s2, b2.to(gpu), N2, N1)
    x2 = c2.cpu().float() * s2  # exact: (q - zp) * s re-quantizes to q - zp
    ref32 = oracle.linear_lut(x2, p2, cb2, s2, zp2, b2, N2, N1)
    exact = (c2.cpu().double() * s2) @ cb2.double()[idx2.long()].T + b2.double()
    a4_exact_check(y2, ref32, exact, N1)


@pytest.mark.parametrize("B,C,H,W,OC,prepared", [
    (2, 64, 28, 28, 64, True),   # band kernel with the quantizing epilogue, fp16 codes out
    (2, 16, 13, 11, 24, False),  # generic implicit GEMM, runtime epilogue
])
def test_conv2d_lut_q_chain(gpu, B, C, H, W, OC, prepared):
    ops = _ops()
    announce(f"conv2d_lut_q chain B={B} C={C} {H}x{W} OC={OC} prepared={prepared}")
    g = _gen(B + C + OC)
    shape1, shape2 = (OC, C, 3, 3), (OC, OC, 3, 3)
    idx1, cb1, p1, b1 = _layer(OC, C * 9, g)
    idx2, cb2, p2, b2 = _layer(OC, OC * 9, g)
    s1, zp1, s2, zp2 = 0.125, 8, 0.0625, 2
    x = torch.randn(B, C, H, W, generator=g)
    pg1, pg2 = p1.to(gpu), p2.to(gpu)
    pr1 = ops.prepare_conv_weight(pg1, 4, shape1) if prepared else None
    pr2 = ops.prepare_conv_weight(pg2, 4, shape2) if prepared else None
    if prepared:
        assert pr1 is not None and pr2 is not None
    xq = ops.quantize_activation_f16(x.to(gpu), s1, zp1)
    c2 = ops.dimq_conv2d_lut_q(xq, pg1, cb1.to(gpu), s1, b1.to(gpu), shape1, 1, 1, prepared_weight=pr1,
                               activation="relu", out_act=(s2, zp2))
    assert c2.dtype == torch.float16 and c2.shape == (B, OC, H, W)
    w1 = cb1.double()[idx1.long()].reshape(shape1)
    y1 = torch.relu(F.conv2d(a4_levels(x, s1, zp1), w1, b1.double(), 1, 1))
    _check_codes(c2, y1, s2, zp2)
    y2 = ops.dimq_conv2d_lut_q(c2, pg2, cb2.to(gpu), s2, b2.to(gpu), shape2, 1, 1, prepared_weight=pr2)
    assert y2.dtype == torch.float32
    x2 = c2.cpu().float() * s2
    ref32 = oracle.conv2d_lut(x2, p2, cb2, s2, zp2, b2, shape2, (1, 1), (1, 1))
    w2 = cb2.double()[idx2.long()].reshape(shape2)
    exact = F.conv2d(c2.cpu().double() * s2, w2, b2.double(), 1, 1)
    a4_exact_check(y2, ref32, exact, OC * 9)


def test_lut_q_errors(gpu):
    ops = _ops()
    g = _gen(1)
    idx, cb, packed, bias = _layer(32, 64, g)
    xq = ops.quantize_activation_f16(torch.randn(4, 64, device=gpu), 0.1, 8)
    with pytest.raises(RuntimeError, match="quantized output"):
        ops.dimq_linear_lut_q(xq, packed.to(gpu), cb.to(gpu), 0.1, None, 32, 64, out_act=(0.1, 8),
                              out_dtype=torch.float32)
    with pytest.raises(RuntimeError, match="fp16 codebook"):
        ops.dimq_linear_lut_q(xq, packed.to(gpu), cb.float().to(gpu), 0.1, None, 32, 64)
    with pytest.raises(RuntimeError, match="out_act_zero_point"):
        ops.dimq_linear_lut_q(xq, packed.to(gpu), cb.to(gpu), 0.1, None, 32, 64, out_act=(0.1, 16))
    with pytest.raises(RuntimeError, match="fp16 activation codes"):
        ops.dimq_linear_lut_q(xq.float(), packed.to(gpu), cb.to(gpu), 0.1, None, 32, 64)
