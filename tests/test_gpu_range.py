"""fp16 range guard of the weight-only kernels: fp32 / bf16 activations beyond the fp16 range (|x| up to 1e6)
or far below it (|x| < 2^-24) must still match the dequantize-then-F.linear / F.conv2d reference.

The matrix path rounds activations to fp16; a tile holding a value that rounds to inf (an inf or NaN
accumulator) or no value of magnitude >= 2^-7 is recomputed in fp32 by the work-group.  Every kernel
family that converts activations is reached by the shape that selects it (see the ids)."""

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import announce

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _ops():
    from dimq_amd import ops
    return ops


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _codebook_case(N, K, bits, per_channel, g):
    rows = N if per_channel else 1
    cb = (torch.randn(rows, 1 << bits, generator=g) * 0.05).sort(dim=1).values
    idx = torch.randint(0, 1 << bits, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, bits))
    return (cb if per_channel else cb[0]), packed


def _scaled(x, mode, g):
    """Activations for one range mode; the scale of every row for the per-group checks."""
    M = x.shape[0]
    if mode == "huge":      # every row beyond fp16 (|x| up to ~4e5..1e6)
        s = torch.full((M,), 2.5e5)
    elif mode == "tiny":    # every value below fp16's smallest subnormal 2^-24
        s = torch.full((M,), 1e-9)
    elif mode == "mixed":   # rows alternate between beyond-fp16 and ordinary magnitudes
        s = torch.where(torch.arange(M) % 2 == 0, torch.tensor(3e4), torch.tensor(1.0))
    else:                   # ordinary rows with a single 1e6 entry
        s = torch.ones(M)
    xs = x * s.reshape(-1, *([1] * (x.dim() - 1)))
    if mode == "one":
        xs.view(-1)[int(torch.randint(0, xs.numel(), (1,), generator=g))] = 1e6
    return xs, s


LINEAR_CASES = [
    # id, M, N, K, bits; the ops entry allocates the workspace its query asks for
    ("gemv_stream", 1, 256, 4096, 3),
    ("gemv_stream_splitk_4col", 8, 128, 2048, 4),  # bf16: the direct bf16 kernel
    ("gemv_direct_k1024", 5, 64, 1024, 2),
    ("gemv_cb", 5, 77, 1000, 3),
    ("gemm_fast", 40, 256, 512, 4),
    ("gemm_cb", 40, 100, 100, 2),
    ("gemm_cb8", 40, 64, 256, 8),
    ("deep_128x128", 200, 256, 768, 4),
    ("big_128x128", 130, 200, 2048, 3),
    # M >= 2048: activations converted to fp16 in the pre-decode launch, per-row flags, one tile shape each
    ("predecoded_128x128", 2100, 300, 192, 4),
    ("predecoded_128x384", 2200, 768, 64, 3),
    ("predecoded_160x256", 4200, 768, 192, 2),
    ("predecoded_256x256", 8192, 1024, 64, 2),
    ("predecoded_128x256", 8704, 2048, 32, 4),
    # the same shape through the plain C entry (no workspace): the shared-decode 256x256 tile, 16-bit only
    ("lds_256x256_no_workspace", 2100, 300, 192, 4),
]


def _linear_no_workspace(gpu, x, packed, cb, bits, bias, N, K):
    from dimq_amd import _C
    y = torch.empty(x.shape[0], N, dtype=torch.float32, device=gpu)
    xg, pg, cg, bg = x.to(gpu), packed.to(gpu), cb.to(gpu), bias.to(gpu)
    dt = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
    with torch.cuda.device(gpu):
        rc = _C.lib.dimq_linear_codebook(xg.data_ptr(), dt[x.dtype], x.shape[0], K, pg.data_ptr(), pg.numel(), bits,
                                         cg.data_ptr(), 0, cg.shape[0] if cg.dim() == 2 else 1, cg.shape[-1],
                                         bg.data_ptr(), 0, N, y.data_ptr(), 0, 0,
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _C.lib.dimq_last_error()
    return y


@pytest.mark.parametrize("mode", ["huge", "tiny", "mixed", "one"])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", LINEAR_CASES, ids=[c[0] for c in LINEAR_CASES])
def test_linear_codebook_activation_range(gpu, case, xdt, mode):
    name, M, N, K, bits = case
    if name == "lds_256x256_no_workspace" and xdt == torch.float32:
        pytest.skip("fp32 activations do not take the 256x256 tile")
    ops = _ops()
    announce(f"range linear {name} {xdt} {mode}")
    g = _gen(M + N + K + bits)
    cb, packed = _codebook_case(N, K, bits, True, g)
    x, s = _scaled(torch.randn(M, K, generator=g), mode, g)
    x = x.to(xdt)
    bias = torch.randn(N, generator=g) * 0.1 * float(s.min())
    if name.endswith("no_workspace"):
        y = _linear_no_workspace(gpu, x, packed, cb, bits, bias, N, K)
    else:
        y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                     out_dtype=torch.float32)
    ref = oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias)
    assert bool(torch.isfinite(y).all())
    assert oracle.rel_err(y, ref) <= TOL, (name, mode, oracle.rel_err(y, ref))
    if mode == "mixed":  # each magnitude group on its own: a recomputed tile holds both
        for sel in (s > 1, s == 1):
            assert oracle.rel_err(y.cpu()[sel], ref[sel]) <= TOL, (name, mode, oracle.rel_err(y.cpu()[sel], ref[sel]))


@pytest.mark.parametrize("M", [300, 2200])  # 2200: the pre-decoded path's guard
def test_linear_codebook_range_inf_nan_inputs(gpu, M):
    """Genuine inf / NaN activations give the reference's inf / NaN pattern (the tiles holding them are
    recomputed in fp32), and the other rows stay exact to tolerance."""
    ops = _ops()
    g = _gen(5)
    N, K = 256, 768
    cb, packed = _codebook_case(N, K, 4, True, g)
    x = torch.randn(M, K, generator=g)
    x[3, 10] = float("inf")
    x[150, 0] = float("nan")
    x[M - 2, 5] = float("-inf")
    for xdt in (torch.bfloat16, torch.float32):
        announce(f"range linear inf/nan {xdt}")
        xd = x.to(xdt)
        y = ops.dimq_linear_codebook(xd.to(gpu), packed.to(gpu), cb.to(gpu), 4, None, N, K,
                                     out_dtype=torch.float32).cpu()
        ref = oracle.linear_dequant_reference(xd.float(), packed, 4, cb, N, K, None)
        assert torch.equal(torch.isnan(y), torch.isnan(ref))
        assert torch.equal(torch.isinf(y), torch.isinf(ref))
        fin = torch.isfinite(ref).all(dim=1)
        assert oracle.rel_err(y[fin], ref[fin]) <= TOL


CONV_CASES = [
    # id, B, C, H, W, OC, KH, stride, pad, bits, layout, prepared
    ("implicit_gemm_nhwc", 2, 64, 12, 12, 64, 3, 1, 1, 2, "nhwc", True),
    ("generic_nchw", 2, 16, 10, 9, 32, 3, 1, 1, 3, "nchw", False),
    ("generic_stem", 2, 3, 31, 29, 16, 7, 2, 3, 8, "nchw", False),
]


@pytest.mark.parametrize("mode", ["huge", "tiny", "one"])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv2d_codebook_activation_range(gpu, case, xdt, mode):
    name, B, C, H, W, OC, KH, st, pd, bits, layout, prepared = case
    if name == "implicit_gemm_nhwc" and xdt == torch.float32:
        pytest.skip("the implicit-GEMM tiles take 16-bit activations")
    ops = _ops()
    announce(f"range conv {name} {xdt} {mode}")
    g = _gen(B + C + OC + bits)
    shape = (OC, C, KH, KH)
    cb, packed = _codebook_case(OC, C * KH * KH, bits, True, g)
    x, s = _scaled(torch.randn(B, C, H, W, generator=g), mode, g)
    x = x.to(xdt)
    xd = x.to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    pdv = packed.to(gpu)
    prep = ops.prepare_conv_weight(pdv, bits, shape) if prepared else None
    y = ops.dimq_conv2d_codebook(xd, pdv, cb.to(gpu), bits, None, shape, (st, st), (pd, pd), (1, 1), 1,
                                 out_dtype=torch.float32, prepared_weight=prep)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, bits, cb, shape, None, st, pd, 1, 1)
    assert bool(torch.isfinite(y).all())
    assert oracle.rel_err(y.float(), ref) <= TOL, (name, mode, oracle.rel_err(y.float(), ref))


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_linear_codebook_act_centres_beyond_fp16(gpu, xdt):
    """Activation centres outside the fp16 range: the activations become centers[idx].to(x.dtype), as the
    reference's hard_quantize_weight returns them, and the weight-codebook product stays finite."""
    ops = _ops()
    announce(f"act centres beyond fp16 {xdt}")
    g = _gen(17)
    M, N, K, bits = 64, 128, 256, 4
    cb, packed = _codebook_case(N, K, bits, True, g)
    centres = torch.linspace(-2e5, 2e5, 16)
    x = (torch.randn(M, K, generator=g) * 1e5).to(xdt)
    y = ops.dimq_linear_codebook_act(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, centres.to(gpu), None, N, K,
                                     out_dtype=torch.float32)
    q = centres[((x.float()[..., None] - centres) ** 2).argmin(dim=-1)].to(xdt).float()
    ref = oracle.linear_dequant_reference(q, packed, bits, cb, N, K, None)
    assert bool(torch.isfinite(y).all())
    assert oracle.rel_err(y, ref) <= TOL, oracle.rel_err(y, ref)
