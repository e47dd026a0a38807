"""GPU parity: every HIP entry point against the CPU oracle on the same inputs.

Inputs are generated on the CPU with seeded torch.Generator and copied to the
device.  Integer work (codec, index assignment, activation codes) must be
bit-exact; W4A4 LUT ops follow the reference's tolerance (rtol = atol = 1e-5,
dimq_cuda_backend/tests/test_cuda_ops.py:64,93); weight-only GEMM/conv must
satisfy max|y - ref| / max|ref| <= 2e-3 against dequantize-then-F.linear /
F.conv2d in fp32 on the CPU.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.a4_check import a4_exact_check as _a4_exact_check, a4_levels as _a4_levels
from tests.conftest import announce, out_tol

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = 2e-3


def _ops():
    from dimq_amd import ops

    return ops


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- codec
def test_codec_golden_vectors_gpu(gpu):
    ops = _ops()
    cases = json.loads((GOLD / "codec_vectors.json").read_text())
    for c in cases:
        announce(f"codec golden bits={c['bits']} n={len(c['indices'])}")
        idx = torch.tensor(c["indices"], dtype=torch.uint8, device=gpu)
        packed = ops.pack_bits(idx, c["bits"])
        assert packed.cpu().numpy().tobytes().hex(" ") == c["packed"], (c["bits"], len(c["indices"]))
        back = ops.unpack_bits(packed, idx.numel(), c["bits"])
        assert torch.equal(back, idx)
        if c["bits"] == 4:
            assert torch.equal(ops.pack_u4(idx), packed)
            assert torch.equal(ops.unpack_u4(packed, idx.numel()), idx)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_codec_random_sizes_and_offsets(gpu, bits):
    ops = _ops()
    g = _gen(bits)
    for n in (0, 1, 31, 32, 33, 1000, 4097, 123457):
        announce(f"codec random bits={bits} n={n}")
        idx = torch.randint(0, 1 << bits, (n + 5,), generator=g, dtype=torch.uint8)
        for off in (0, 3):  # an offset view exercises the unaligned path
            sub = idx[off:off + n]
            packed = ops.pack_bits(sub.to(gpu), bits).cpu()
            assert np.array_equal(packed.numpy(), oracle.pack_bits(sub, bits))
            big = torch.zeros(packed.numel() + 7, dtype=torch.uint8)
            big[off:off + packed.numel()] = packed
            back = ops.unpack_bits(big[off:off + packed.numel()].to(gpu), n, bits).cpu()
            assert torch.equal(back, sub)


def test_codec_masks_out_of_range_values(gpu):
    ops = _ops()
    idx = torch.tensor([0x1F, 0x2E, 0xFF], dtype=torch.uint8, device=gpu)
    assert ops.pack_u4(idx).cpu().tolist() == [0xEF, 0x0F]


def test_codec_errors(gpu):
    ops = _ops()
    with pytest.raises(RuntimeError, match="packed tensor is too small"):
        ops.unpack_u4(torch.zeros(2, dtype=torch.uint8, device=gpu), 5)
    with pytest.raises(RuntimeError, match="uint8"):
        ops.pack_u4(torch.zeros(4, dtype=torch.int32, device=gpu))
    with pytest.raises(RuntimeError, match="bits must be one of"):
        ops.pack_bits(torch.zeros(4, dtype=torch.uint8, device=gpu), 5)


def test_codec_stress_2p27_3bit_round_trip(gpu):
    """cfg5: 2^27 random 3-bit indices, bit-exact pack/unpack round trip; the whole packed stream equals the
    oracle's (C packer, a few seconds on the host), and the oracle's stream unpacks to the indices."""
    ops = _ops()
    announce("codec stress 2^27 3-bit")
    n = 1 << 27
    idx = torch.randint(0, 8, (n,), generator=_gen(5), dtype=torch.uint8)
    d = idx.to(gpu)
    packed = ops.pack_bits(d, 3)
    assert packed.numel() == n * 3 // 8
    back = ops.unpack_bits(packed, n, 3)
    assert torch.equal(back, d)
    ref = oracle.pack_bits(idx, 3)
    assert np.array_equal(packed.cpu().numpy(), ref)
    assert torch.equal(ops.unpack_bits(torch.from_numpy(ref).to(gpu), n, 3), d)


# ---------------------------------------------------------------- hard quantization
def test_hard_quantize_golden_and_random(gpu):
    ops = _ops()
    for c in json.loads((GOLD / "hardquant_vectors.json").read_text()):
        announce(f"hardquant golden {c['source']}")
        idx, val = ops.hard_quantize(torch.tensor(c["w"], device=gpu), torch.tensor(c["centers"], device=gpu))
        assert idx.cpu().tolist() == c["idx"], c["source"]
    g = _gen(11)
    for K in (4, 8, 16, 256):
        for per_channel in (False, True):
            announce(f"hardquant random K={K} pc={per_channel}")
            w = torch.randn(37, 301, generator=g) * 0.02
            c = torch.randn(37 if per_channel else 1, K, generator=g) * 0.02
            cc = c if per_channel else c[0]
            idx, val = ops.hard_quantize(w.to(gpu), cc.to(gpu), per_channel)
            want_idx, want_val = oracle.hard_quantize(w, cc, per_channel=per_channel)
            assert np.array_equal(idx.cpu().numpy(), want_idx)
            assert np.array_equal(val.cpu().numpy(), want_val)


def test_hard_quantize_nan_inf(gpu):
    ops = _ops()
    w = torch.tensor([0.5, float("nan"), 2.0, float("inf")])
    for c in (torch.tensor([0.0, float("nan"), 1.0, 3.0]), torch.tensor([0.0, 1.0, 3.0])):
        idx, _ = ops.hard_quantize(w.to(gpu), c.to(gpu), False)
        assert idx.cpu().tolist() == ((w[:, None] - c[None, :]) ** 2).argmin(1).tolist()


def test_hard_quantize_half_inputs(gpu):
    ops = _ops()
    w = (torch.randn(64, 50, generator=_gen(3)) * 0.1)
    c = torch.randn(64, 16, generator=_gen(4)) * 0.1
    for dt in (torch.float16, torch.bfloat16):
        idx, val = ops.hard_quantize(w.to(dt).to(gpu), c.to(gpu), True)
        want, wv = oracle.hard_quantize(w.to(dt).float(), c, per_channel=True)
        assert np.array_equal(idx.cpu().numpy(), want)
        assert torch.equal(val.cpu(), torch.from_numpy(wv).to(dt))


def _argmin_ref(w, c):
    """The reference's assignment, (w - c)^2 in fp32 then argmin (quant/dimq.py:213-215), on the CPU."""
    return ((w.float().reshape(-1)[:, None] - c.float()[None, :]) ** 2).argmin(1)


@pytest.mark.parametrize("K", [1, 2, 3, 16, 255, 256])
def test_hard_quantize_ties_and_specials(gpu, K):
    """The sorted-search assignment against the full argmin: unsorted and duplicated centres, values exactly
    between two centres (equal distances: the first index wins), +-0, infinite centres and inputs, distances that
    overflow to inf, NaN centres, inputs beyond every centre, and a tensor large enough for several elements per
    thread."""
    ops = _ops()
    announce(f"hard_quantize ties/specials K={K}")
    g = _gen(K)
    grid = torch.randint(-12, 13, (K,), generator=g).float() * 0.25  # duplicates for K > 25
    c = grid[torch.randperm(K, generator=g)]
    mids = torch.arange(-60, 61).float() * 0.125                    # every midpoint of the 0.25 grid
    specials = torch.tensor([0.0, -0.0, 1e30, -1e30, 3.4e38, -3.4e38, 1e-40, float("inf"), float("-inf"),
                             float("nan"), 100.0, -100.0])
    w = torch.cat([mids, specials, torch.randn(2000, generator=g) * 2])
    cases = [c, torch.where(torch.arange(K) % 5 == 1, -c, c)]
    if K >= 3:
        cz = c.clone(); cz[0], cz[1] = 0.0, -0.0
        ci = c.clone(); ci[K // 2] = float("inf"); ci[K - 1] = float("-inf")
        cd = c.clone(); cd[K - 1] = 2e30; cd[0] = -2e30
        cn = c.clone(); cn[K // 2] = float("nan")
        cases += [cz, ci, cd, cn]
    for cc in cases:
        idx, val = ops.hard_quantize(w.to(gpu), cc.to(gpu), False)
        want = _argmin_ref(w, cc)
        bad = (idx.cpu().long() != want).nonzero().flatten()
        assert bad.numel() == 0, [(float(w[i]), int(idx[i]), int(want[i])) for i in bad[:5]]
        assert np.array_equal(idx.cpu().numpy(), oracle.hard_quantize(w, cc)[0])
    big = torch.randn(3, 1 << 20, generator=g)   # 4096+ segments: 16 elements per thread
    cb = torch.randn(3, K, generator=g)
    idx, val = ops.hard_quantize(big.to(gpu), cb.to(gpu), True)
    for r in range(3):
        assert torch.equal(idx[r].cpu().long(), _argmin_ref(big[r], cb[r]))
        assert torch.equal(val[r].cpu(), cb[r][idx[r].cpu().long()])


# ---------------------------------------------------------------- activation quantization / product table
def test_quantize_activation_golden_and_dtypes(gpu):
    ops = _ops()
    for c in json.loads((GOLD / "actquant_vectors.json").read_text()):
        q = ops.quantize_activation_u4(torch.tensor(c["x"], device=gpu), c["scale"], c["zp"])
        assert q.cpu().tolist() == c["q"], c["source"]
    x = torch.randn(3, 1001, generator=_gen(2)) * 2
    x[0, :7] = torch.tensor([float("nan"), float("inf"), float("-inf"), 1e30, -1e30, float("nan"), 3e9])
    for dt in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        q = ops.quantize_activation_u4(x.to(dt).to(gpu), 0.2, 7)
        assert q.shape == x.shape
        assert np.array_equal(q.cpu().numpy(), oracle.quantize_act_u4(x.to(dt).float(), 0.2, 7))
    with pytest.raises(RuntimeError, match="act_zero_point must be in"):
        ops.quantize_activation_u4(x.to(gpu), 0.2, 16)
    with pytest.raises(RuntimeError, match="act_scale must be positive"):
        ops.quantize_activation_u4(x.to(gpu), 0.0, 3)


def test_product_table(gpu):
    ops = _ops()
    c = json.loads((GOLD / "product_table_vectors.json").read_text())[0]
    cb = torch.linspace(-1.0, 1.0, 16, dtype=torch.float16)
    t = ops.build_product_table(cb.to(gpu), 0.125, 8).cpu()
    assert torch.equal(t, torch.tensor(c["table"]))
    g = torch.randn(7, 16, generator=_gen(8))
    tg = ops.build_product_table_grouped(g.to(gpu), 0.37, 5).cpu().numpy()
    assert np.array_equal(tg, oracle.product_table(g, 0.37, 5))
    with pytest.raises(RuntimeError, match="exactly 16 codebook entries"):
        ops.build_product_table(torch.zeros(8, device=gpu), 0.1, 3)


# ---------------------------------------------------------------- W4A4 LUT ops (the reference ops)
def test_linear_lut_reference_recipe(gpu):
    ops = _ops()
    r = json.loads((GOLD / "w4a4_recipes.json").read_text())["linear"]
    idx = np.array(r["indices"], np.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_linear_lut(torch.tensor(r["x"], device=gpu), packed.to(gpu), torch.tensor(r["codebook"], device=gpu),
                            r["scale"], r["zp"], torch.tensor(r["bias"], device=gpu), 6, 11)
    torch.testing.assert_close(y.cpu(), torch.tensor(r["y"]), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K", [(4, 11, 6), (1, 64, 128), (37, 130, 96), (200, 300, 768), (64, 33, 250)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.float64])
def test_linear_lut_vs_oracle(gpu, M, N, K, xdt):
    ops = _ops()
    announce(f"linear_lut M={M} N={N} K={K} {xdt}")
    g = _gen(M * 7 + N)
    x = torch.randn(M, K, generator=g)
    # non-finite activations: NaN codes as zp, +-inf clamp (both contribute like any code)
    x.view(-1)[torch.randint(0, x.numel(), (3,), generator=g)] = torch.tensor([float("nan"), float("inf"),
                                                                                 float("-inf")])
    x = x.to(xdt)
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    cb = torch.linspace(-0.5, 0.5, 16) + 0.01 * torch.randn(16, generator=g)
    bias = torch.randn(N, generator=g)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_linear_lut(x.to(gpu), packed.to(gpu), cb.to(gpu), 0.2, 7, bias.to(gpu), N, K)
    ref = oracle.linear_lut(x.float(), packed, cb, 0.2, 7, bias, N, K)
    exact = _a4_levels(x, 0.2, 7) @ cb.double()[idx.long()].T + bias.double()
    _a4_exact_check(y, ref, exact, K)


def test_linear_lut_leading_dims_and_errors(gpu):
    ops = _ops()
    x = torch.randn(2, 3, 32, generator=_gen(1))
    idx = torch.randint(0, 16, (8, 32), generator=_gen(2), dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4)).to(gpu)
    cb = torch.linspace(-1, 1, 16, device=gpu)
    y = ops.dimq_linear_lut(x.to(gpu), packed, cb, 0.25, 8, None, 8, 32)
    assert y.shape == (2, 3, 8) and y.dtype == torch.float32
    ref = oracle.linear_lut(x, packed.cpu(), cb.cpu(), 0.25, 8, None, 8, 32)
    torch.testing.assert_close(y.cpu(), torch.from_numpy(ref), rtol=1e-5, atol=1e-5)
    with pytest.raises(RuntimeError, match="codebook must have 16 entries for W4"):
        ops.dimq_linear_lut(x.to(gpu), packed, cb[:8], 0.25, 8, None, 8, 32)
    with pytest.raises(RuntimeError, match="packed_weight is too small"):
        ops.dimq_linear_lut(x.to(gpu), packed[:10], cb, 0.25, 8, None, 8, 32)
    with pytest.raises(RuntimeError, match="input last dimension must equal in_features"):
        ops.dimq_linear_lut(x.to(gpu), packed, cb, 0.25, 8, None, 16, 16)


def test_conv2d_lut_reference_recipe(gpu):
    ops = _ops()
    r = json.loads((GOLD / "w4a4_recipes.json").read_text())["conv2d"]
    idx = np.array(r["indices"], np.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_conv2d_lut(torch.tensor(r["x"], device=gpu), packed.to(gpu), torch.tensor(r["codebook"], device=gpu),
                            r["scale"], r["zp"], torch.tensor(r["bias"], device=gpu), idx.shape, r["stride"],
                            r["padding"], r["dilation"], r["groups"])
    torch.testing.assert_close(y.cpu(), torch.tensor(r["y"]), rtol=1e-5, atol=1e-5)


def test_extension_module_functions(gpu):
    """The reference extension's module-level functions (csrc/dimq_ops.cpp:55-62) called positionally, as
    dimq_backend._C.<name>(...) would be, against the registered ops and the oracle."""
    from dimq_amd import _C
    r = json.loads((GOLD / "w4a4_recipes.json").read_text())
    lin, cv = r["linear"], r["conv2d"]
    idx = torch.tensor(lin["indices"], dtype=torch.uint8, device=gpu)
    packed = _C.pack_u4(idx)
    assert bytes(packed.cpu().numpy()) == bytes(oracle.pack_bits(np.array(lin["indices"], np.uint8), 4))
    assert torch.equal(_C.unpack_u4(packed, idx.numel()), idx.view(-1))
    x = torch.tensor(lin["x"], device=gpu)
    assert torch.equal(_C.quantize_activation_u4(x, lin["scale"], lin["zp"]),
                       torch.ops.dimq.quantize_activation_u4(x, lin["scale"], lin["zp"]))
    cb = torch.tensor(lin["codebook"], device=gpu)
    assert torch.equal(_C.build_product_table(cb, 0.125, 8), torch.ops.dimq.build_product_table(cb, 0.125, 8))
    y = _C.linear_lut(x, packed, cb, lin["scale"], lin["zp"], torch.tensor(lin["bias"], device=gpu), 6, 11)
    torch.testing.assert_close(y.cpu(), torch.tensor(lin["y"]), rtol=1e-5, atol=1e-5)
    cidx = np.array(cv["indices"], np.uint8)
    oc, cin, kh, kw = cidx.shape
    yc = _C.conv2d_lut(torch.tensor(cv["x"], device=gpu), torch.from_numpy(oracle.pack_bits(cidx, 4)).to(gpu),
                       torch.tensor(cv["codebook"], device=gpu), cv["scale"], cv["zp"],
                       torch.tensor(cv["bias"], device=gpu), oc, cin, kh, kw, *cv["stride"], *cv["padding"],
                       *cv["dilation"], cv["groups"])
    torch.testing.assert_close(yc.cpu(), torch.tensor(cv["y"]), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", [
    dict(B=2, C=4, H=9, W=8, OC=6, KH=3, KW=3, s=(1, 1), p=(1, 1), d=(1, 1), g=1),
    dict(B=1, C=6, H=11, W=7, OC=4, KH=3, KW=2, s=(2, 1), p=(1, 0), d=(1, 2), g=2),
    dict(B=3, C=16, H=8, W=8, OC=32, KH=1, KW=1, s=(2, 2), p=(0, 0), d=(1, 1), g=1),
])
def test_conv2d_lut_vs_oracle(gpu, case):
    ops = _ops()
    announce(f"conv2d_lut {case}")
    g = _gen(case["C"] * 13 + case["OC"])
    x = torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g)
    shape = (case["OC"], case["C"] // case["g"], case["KH"], case["KW"])
    idx = torch.randint(0, 16, shape, generator=g, dtype=torch.uint8)
    cb = torch.linspace(-0.7, 0.6, 16)
    bias = torch.randn(case["OC"], generator=g)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_conv2d_lut(x.to(gpu), packed.to(gpu), cb.to(gpu), 0.25, 7, bias.to(gpu), shape, case["s"], case["p"],
                            case["d"], case["g"])
    ref = oracle.conv2d_lut(x, packed, cb, 0.25, 7, bias, shape, case["s"], case["p"], case["d"], case["g"])
    torch.testing.assert_close(y.cpu(), torch.from_numpy(ref), rtol=1e-5, atol=1e-5)


# W4A4 ops with an fp16 codebook (the reference exporter's default): the
# workspace path, activations as fp16 a - zp into the weight-only kernels.
# Shapes reach the GEMV kernels (M <= 16), the 128x128 tiles (cfg1), the
# shared-decode 256x256 tile (M >= 2048) and the generic tiles (odd K).
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (4, 256, 4096), (16, 300, 768), (1576, 1024, 768),
                                   (2304, 512, 768), (37, 130, 96), (5, 11, 6)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_linear_lut_fp16_codebook_fast_path(gpu, M, N, K, xdt):
    ops = _ops()
    from dimq_amd import _C
    announce(f"linear_lut fp16 codebook M={M} N={N} K={K} {xdt}")
    assert _C.lib.dimq_linear_lut_workspace_bytes(M, K, _C.F16) >= M * K * 2
    g = _gen(M * 5 + N + K)
    x = torch.randn(M, K, generator=g).to(xdt)
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    cb = (torch.linspace(-0.5, 0.5, 16) + 0.01 * torch.randn(16, generator=g)).half()
    bias = torch.randn(N, generator=g)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_linear_lut(x.to(gpu), packed.to(gpu), cb.to(gpu), 0.2, 7, bias.to(gpu), N, K)
    ref = oracle.linear_lut(x.float(), packed, cb.float(), 0.2, 7, bias, N, K)
    exact = _a4_levels(x, 0.2, 7) @ cb.double()[idx.long()].T + bias.double()
    _a4_exact_check(y, ref, exact, K)


def test_linear_lut_fp16_codebook_matches_generic_path(gpu):
    # the workspace path and the no-workspace entry point (generic A4 tiles)
    # agree on the same inputs, and a short workspace falls back
    from dimq_amd import _C
    M, N, K = 64, 96, 256
    g = _gen(77)
    x = torch.randn(M, K, generator=g).to(gpu)
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    cb = torch.linspace(-1, 1, 16).half().to(gpu)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4)).to(gpu)
    s = torch.cuda.current_stream().cuda_stream
    outs = []
    for ws_bytes in (M * K * 2, M * K * 2 - 2, 0):
        y = torch.empty(M, N, device=gpu)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=gpu)
        rc = _C.lib.dimq_linear_lut_ws(x.data_ptr(), _C.F32, M, packed.data_ptr(), packed.numel(), cb.data_ptr(),
                                       _C.F16, 16, 0.125, 8, None, 0, 0, N, K, y.data_ptr(),
                                       ws.data_ptr() if ws_bytes else None, ws_bytes, s)
        assert rc == 0, _C.lib.dimq_last_error()
        outs.append(y)
    torch.cuda.synchronize()
    torch.testing.assert_close(outs[0], outs[2], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(outs[1], outs[2], rtol=0, atol=0)  # short workspace: the generic path itself


@pytest.mark.parametrize("case", [
    dict(B=2, C=64, H=56, W=56, OC=64, KH=3, KW=3, s=(1, 1), p=(1, 1), d=(1, 1), g=1),    # cfg2 shape, halo kernel
    dict(B=2, C=128, H=28, W=28, OC=128, KH=3, KW=3, s=(1, 1), p=(1, 1), d=(1, 1), g=1),  # C 128, decode per step
    dict(B=3, C=64, H=30, W=30, OC=128, KH=1, KW=1, s=(2, 2), p=(0, 0), d=(1, 1), g=1),   # 1x1 stride 2
    dict(B=2, C=4, H=9, W=8, OC=6, KH=3, KW=3, s=(1, 1), p=(1, 1), d=(1, 1), g=1),        # generic implicit GEMM
    dict(B=1, C=6, H=11, W=7, OC=4, KH=3, KW=2, s=(2, 1), p=(1, 0), d=(1, 2), g=2),       # groups + dilation
])
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_conv2d_lut_fp16_codebook_fast_path(gpu, case, xdt):
    ops = _ops()
    announce(f"conv2d_lut fp16 codebook {case} {xdt}")
    g = _gen(case["C"] * 11 + case["OC"] + case["H"])
    x = torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g).to(xdt)
    shape = (case["OC"], case["C"] // case["g"], case["KH"], case["KW"])
    idx = torch.randint(0, 16, shape, generator=g, dtype=torch.uint8)
    cb = torch.linspace(-0.7, 0.6, 16).half()
    bias = torch.randn(case["OC"], generator=g)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    y = ops.dimq_conv2d_lut(x.to(gpu), packed.to(gpu), cb.to(gpu), 0.25, 7, bias.to(gpu), shape, case["s"], case["p"],
                            case["d"], case["g"])
    ref = oracle.conv2d_lut(x.float(), packed, cb.float(), 0.25, 7, bias, shape, case["s"], case["p"], case["d"],
                            case["g"])
    exact = torch.nn.functional.conv2d(_a4_levels(x, 0.25, 7), cb.double()[idx.long()], bias.double(), case["s"],
                                       case["p"], case["d"], case["g"])
    _a4_exact_check(y, ref, exact, shape[1] * shape[2] * shape[3])


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_conv2d_lut_fast_path_unaligned_input(gpu, xdt):
    """The W4A4 fast path's one launch that quantizes the activations and lays out the 4-bit weight: an input
    view one element into its storage (element-wise loads) gives the same output, bit for bit, as an aligned
    copy, and both match the oracle."""
    ops = _ops()
    g = _gen(77)
    B, C, H, W, OC = 2, 64, 20, 24, 64
    shape = (OC, C, 3, 3)
    flat = torch.randn(B * C * H * W + 1, generator=g).to(xdt).to(gpu)
    xv = flat[1:].view(B, C, H, W)
    idx = torch.randint(0, 16, shape, generator=g, dtype=torch.uint8)
    cb = torch.linspace(-0.7, 0.6, 16).half()
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    args = (packed.to(gpu), cb.to(gpu), 0.25, 7, None, shape, (1, 1), (1, 1), (1, 1), 1)
    y_view = ops.dimq_conv2d_lut(xv, *args)
    y_copy = ops.dimq_conv2d_lut(xv.clone(), *args)
    assert torch.equal(y_view, y_copy)
    ref = oracle.conv2d_lut(xv.cpu().float(), packed, cb.float(), 0.25, 7, None, shape, (1, 1), (1, 1), (1, 1), 1)
    exact = torch.nn.functional.conv2d(_a4_levels(xv.cpu(), 0.25, 7), cb.double()[idx.long()], None, 1, 1, 1, 1)
    _a4_exact_check(y_view, ref, exact, C * 9)


# ---------------------------------------------------------------- weight-only codebook Linear
def _codebook_case(N, K, bits, per_channel, g, cb_entries=None):
    Kc = cb_entries or (1 << bits)
    rows = N if per_channel else 1
    cb = (torch.randn(rows, Kc, generator=g) * 0.05).sort(dim=1).values
    idx = torch.randint(0, Kc, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, bits))
    return cb if per_channel else cb[0], idx, packed


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (3, 5, 13), (16, 200, 256), (33, 96, 160), (300, 260, 512)])
def test_linear_codebook_bits_shapes(gpu, bits, M, N, K):
    ops = _ops()
    for per_channel in (True, False):
        announce(f"linear_codebook bits={bits} M={M} N={N} K={K} pc={per_channel}")
        g = _gen(bits * 1000 + M + N + K)
        cb, idx, packed = _codebook_case(N, K, bits, per_channel, g)
        x = torch.randn(M, K, generator=g)
        bias = torch.randn(N, generator=g) * 0.1
        y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                     out_dtype=torch.float32)
        ref = oracle.linear_dequant_reference(x, packed, bits, cb, N, K, bias)
        assert oracle.rel_err(y, ref) <= TOL, (bits, M, N, K, per_channel, oracle.rel_err(y, ref))


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("odt", [torch.float32, torch.float16, torch.bfloat16])
def test_linear_codebook_dtypes(gpu, xdt, odt):
    ops = _ops()
    g = _gen(77)
    N, K, M = 192, 384, 130
    cb, idx, packed = _codebook_case(N, K, 4, True, g)
    x = torch.randn(M, K, generator=g).to(xdt)
    bias = (torch.randn(N, generator=g) * 0.1).to(xdt)
    for variant in ("auto", "small_m", "mfma"):
        announce(f"linear_codebook dtypes {xdt}->{odt} {variant}")
        y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu).to(xdt), 4, bias.to(gpu), N, K,
                                     out_dtype=odt, variant=variant)
        assert y.dtype == odt
        ref = oracle.linear_dequant_reference(x.float(), packed, 4, cb.to(xdt).float(), N, K, bias.float())
        tol = out_tol(odt)
        assert oracle.rel_err(y.float(), ref) <= tol, (xdt, odt, variant, oracle.rel_err(y.float(), ref))


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("M,N,K,xdt", [
    (257, 130, 128, torch.float32),    # deep-pipeline 128x128 tile (K < 2048), fp32 staging
    (520, 384, 192, torch.bfloat16),   # deep-pipeline 128x128 tile
    (65, 256, 64, torch.float16),      # deep-pipeline 128x128 tile, one k stage
    (130, 200, 2048, torch.bfloat16),  # 128x128 tile (K >= 2048)
    (2100, 300, 192, torch.bfloat16),  # 256x256 shared-decode tile (M >= 2048, 16-bit), M / N tails
    (2048, 256, 64, torch.float16),    # shared-decode tile, one k stage
])
def test_linear_codebook_large_tiles(gpu, bits, M, N, K, xdt):
    """The 32x32x16 large-tile kernels (128x128 plain and deep-pipeline, 256x256 shared decode),
    each reached by the shape that selects it, M / N tails."""
    ops = _ops()
    for per_channel in (True, False):
        announce(f"linear_codebook large bits={bits} M={M} N={N} K={K} {xdt} pc={per_channel}")
        g = _gen(bits * 7 + M + N + K)
        cb, idx, packed = _codebook_case(N, K, bits, per_channel, g)
        x = torch.randn(M, K, generator=g).to(xdt)
        bias = torch.randn(N, generator=g) * 0.1
        y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                     out_dtype=torch.float32)
        ref = oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias)
        assert oracle.rel_err(y, ref) <= TOL, (bits, M, N, K, per_channel, oracle.rel_err(y, ref))


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("M,N,K,xdt", [(1, 300, 4096, torch.bfloat16), (4, 64, 8192, torch.float16),
                                       (3, 130, 4096, torch.float32), (16, 130, 4096, torch.bfloat16),
                                       (5, 77, 4096, torch.float16), (9, 200, 8192, torch.bfloat16),
                                       (16, 48, 12288, torch.float32), (16, 256, 4096, torch.bfloat16),
                                       (8, 128, 2048, torch.float32), (12, 64, 1024, torch.float16),
                                       (16, 4096, 4096, torch.bfloat16), (8, 96, 1024, torch.bfloat16),
                                       (6, 80, 2048, torch.bfloat16)])
def test_linear_codebook_gemv_fast(gpu, bits, M, N, K, xdt):
    """Decode-shape GEMVs (streamed weight runs; 16-column work-groups with the k range split over waves, or
    64-column work-groups with k split over work-groups and the partial sums added by a second kernel; bf16
    activations with 4 < M <= 16 and K 1024 / 2048 / 4096 the direct kernel, whose lane runs are 64 / 128 /
    256 indices), N tails, per-layer and per-channel codebooks, fp32 / fp16 / bf16 activations."""
    ops = _ops()
    for per_channel in (True, False):
        announce(f"linear_codebook gemv bits={bits} M={M} N={N} K={K} {xdt} pc={per_channel}")
        g = _gen(bits * 13 + M + N)
        cb, idx, packed = _codebook_case(N, K, bits, per_channel, g)
        x = torch.randn(M, K, generator=g).to(xdt)
        bias = torch.randn(N, generator=g) * 0.1
        y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                     out_dtype=torch.float32)
        ref = oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias)
        assert oracle.rel_err(y, ref) <= TOL, (bits, M, N, K, per_channel, oracle.rel_err(y, ref))


@pytest.mark.parametrize("act", [None, "gelu"])
def test_linear_codebook_ex_ws_large_m_same_bits(gpu, act):
    """Above the decode shapes the workspace entry point needs no workspace (the query returns 0) and gives
    the plain entry point's bits, with or without a workspace passed."""
    from dimq_amd import _C
    g = _gen(91)
    M, N, K = 1576, 384, 768
    cb, idx, packed = _codebook_case(N, K, 4, True, g)
    x = torch.randn(M, K, generator=g).to(gpu)
    bias = (torch.randn(N, generator=g) * 0.1).to(gpu)
    cbg, pg = cb.to(gpu), packed.to(gpu)
    act_id = {None: 0, "gelu": 2}[act]
    s = torch.cuda.current_stream().cuda_stream
    assert _C.lib.dimq_linear_codebook_workspace_bytes(M, K, N, 4, _C.F32) == 0
    ws = torch.empty(M * K * 2, dtype=torch.uint8, device=gpu)
    y_ws = torch.empty(M, N, device=gpu)
    y_direct = torch.empty(M, N, device=gpu)
    rc = _C.lib.dimq_linear_codebook_ex_ws(x.data_ptr(), _C.F32, M, K, pg.data_ptr(), pg.numel(), 4, cbg.data_ptr(),
                                           _C.F32, N, 16, bias.data_ptr(), _C.F32, N, y_ws.data_ptr(), _C.F32,
                                           None, 0, act_id, 0, ws.data_ptr(), ws.numel(), s)
    assert rc == 0, _C.lib.dimq_last_error()
    rc = _C.lib.dimq_linear_codebook_ex(x.data_ptr(), _C.F32, M, K, pg.data_ptr(), pg.numel(), 4, cbg.data_ptr(),
                                        _C.F32, N, 16, bias.data_ptr(), _C.F32, N, y_direct.data_ptr(), _C.F32,
                                        None, 0, act_id, 0, s)
    assert rc == 0, _C.lib.dimq_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y_ws, y_direct)


def test_linear_codebook_cfg1_shape(gpu):
    """BASELINE cfg1: X fp32 [1576,768], 4-bit per-channel W [3072,768], bias, y fp32."""
    ops = _ops()
    announce("linear_codebook cfg1 shape")
    g = _gen(0)
    cb, idx, packed = _codebook_case(3072, 768, 4, True, g)
    x = torch.randn(1576, 768, generator=g)
    bias = torch.randn(3072, generator=g) * 0.02
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 4, bias.to(gpu), 3072, 768,
                                 out_dtype=torch.float32)
    ref = oracle.linear_dequant_reference(x, packed, 4, cb, 3072, 768, bias)
    assert oracle.rel_err(y, ref) <= TOL


# ---------------------------------------------------------------- weight x activation codebook Linear
@pytest.mark.parametrize("M,N,K,bits,xdt,n_act", [(1, 4096, 4096, 3, torch.bfloat16, 16),
                                                 (300, 256, 768, 4, torch.float32, 16),
                                                 (2100, 384, 256, 4, torch.bfloat16, 8),
                                                 (37, 130, 96, 2, torch.float16, 256)])
def test_linear_codebook_act_vs_reference(gpu, M, N, K, bits, xdt, n_act):
    """y = Q(x) W_hat^T + b, Q(x) = C_a[argmin (x - C_a)^2] as in the QAT wrapper's activation fake-quant
    (quant/dimq_wrapper.py:80-85 with quant/dimq.py:197-221), against torch CPU fp32."""
    ops = _ops()
    announce(f"linear_codebook_act M={M} N={N} K={K} bits={bits} {xdt} n_act={n_act}")
    g = _gen(M + N + K + n_act)
    cb, idx, packed = _codebook_case(N, K, bits, True, g)
    x = torch.randn(M, K, generator=g).to(xdt)
    x.view(-1)[7] = float("nan")  # a NaN activation takes the first centre (torch argmin of NaN distances)
    ca = torch.randn(n_act, generator=g).sort().values
    bias = torch.randn(N, generator=g) * 0.1
    y = ops.dimq_linear_codebook_act(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, ca.to(gpu), bias.to(gpu), N, K,
                                     out_dtype=torch.float32)
    xf = x.float()
    # centers[idx].to(x.dtype), as the reference's hard_quantize_weight returns them
    q = ca[((xf.reshape(-1)[:, None] - ca[None, :]) ** 2).argmin(1)].reshape(M, K).to(xdt).float()
    ref = oracle.linear_dequant_reference(q, packed, bits, cb, N, K, bias)
    assert oracle.rel_err(y, ref) <= TOL, oracle.rel_err(y, ref)


# ---------------------------------------------------------------- fused epilogue (residual + activation)
_ACTS = {None: lambda t: t, "relu": torch.relu, "gelu": torch.nn.functional.gelu}


@pytest.mark.parametrize("case", [
    dict(M=300, N=256, K=512, bits=4, xdt=torch.bfloat16, out=torch.bfloat16, rdt=torch.bfloat16, act="gelu"),  # deep
    dict(M=200, N=256, K=2048, bits=2, xdt=torch.float16, out=torch.float32, rdt=torch.float32, act="relu"),  # big
    dict(M=2100, N=320, K=256, bits=4, xdt=torch.bfloat16, out=torch.bfloat16, rdt=torch.bfloat16, act=None),  # lds
    dict(M=2050, N=264, K=2048, bits=3, xdt=torch.bfloat16, out=torch.float32, rdt=torch.float16, act="gelu"),
    dict(M=2, N=64, K=4096, bits=3, xdt=torch.bfloat16, out=torch.float32, rdt=torch.float16, act=None),  # gemv fast
    dict(M=9, N=100, K=256, bits=4, xdt=torch.float32, out=torch.float16, rdt=torch.float32, act="gelu"),  # gemv
    dict(M=70, N=50, K=96, bits=3, xdt=torch.float16, out=torch.float32, rdt=torch.bfloat16, act="relu"),  # generic
    dict(M=40, N=72, K=128, bits=8, xdt=torch.float16, out=torch.float32, rdt=torch.float32, act="gelu"),  # 8-bit
])
def test_linear_codebook_fused_epilogue(gpu, case):
    """y = act(x W_hat^T + b + residual) on every Linear kernel family, against the fp32 CPU reference."""
    ops = _ops()
    announce(f"linear fused {case}")
    M, N, K, bits = case["M"], case["N"], case["K"], case["bits"]
    g = _gen(M + N + K + bits)
    cb, idx, packed = _codebook_case(N, K, bits, True, g)
    x = torch.randn(M, K, generator=g).to(case["xdt"])
    bias = torch.randn(N, generator=g) * 0.05
    res = (torch.randn(M, N, generator=g) * 0.3).to(case["rdt"])
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                 out_dtype=case["out"], residual=res.to(gpu), activation=case["act"])
    ref = _ACTS[case["act"]](oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias) + res.float())
    tol = out_tol(case["out"])
    assert oracle.rel_err(y.float(), ref) <= tol, oracle.rel_err(y.float(), ref)


@pytest.mark.parametrize("case", [
    dict(B=2, C=64, H=20, W=18, OC=64, K=3, s=1, bits=2, prep=True, g=1),    # resident halo
    dict(B=2, C=128, H=12, W=12, OC=64, K=3, s=1, bits=3, prep=True, g=1),   # C 128 (NCHW: halo tiles)
    dict(B=2, C=256, H=9, W=9, OC=128, K=3, s=2, bits=2, prep=True, g=1),    # implicit GEMM
    dict(B=2, C=3, H=40, W=40, OC=64, K=7, s=2, bits=8, prep=False, g=1),    # stem
    dict(B=2, C=16, H=9, W=9, OC=24, K=3, s=1, bits=4, prep=False, g=2),     # generic
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
@pytest.mark.parametrize("act", ["relu", "gelu"])
def test_conv2d_codebook_fused_epilogue(gpu, case, layout, act):
    """y = act(conv + b + residual) on every Conv2d kernel family; the residual comes in the other memory order."""
    ops = _ops()
    announce(f"conv fused {case} {layout} {act}")
    g = _gen(case["C"] + case["OC"] + case["K"] + case["bits"])
    K, pad, s = case["K"], case["K"] // 2, case["s"]
    shape = (case["OC"], case["C"] // case["g"], K, K)
    x = torch.relu(torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g)).half()
    cb, idx, packed = _codebook_case(case["OC"], int(np.prod(shape[1:])), case["bits"], True, g)
    bias = torch.randn(case["OC"], generator=g) * 0.1
    ref0 = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb, shape, bias, s, pad, 1, case["g"])
    res = torch.randn(ref0.shape, generator=g) * 0.3
    xd = x.to(gpu)
    rd = res.half().to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    else:
        rd = rd.to(memory_format=torch.channels_last)
    pd = packed.to(gpu)
    prep = ops.prepare_conv_weight(pd, case["bits"], shape) if case["prep"] else None
    y = ops.dimq_conv2d_codebook(xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, (s, s), (pad, pad), (1, 1),
                                 case["g"], out_dtype=torch.float32, prepared_weight=prep, residual=rd, activation=act)
    ref = _ACTS[act](ref0 + res.half().float())
    assert oracle.rel_err(y.float(), ref) <= TOL, oracle.rel_err(y.float(), ref)


def test_fused_epilogue_errors(gpu):
    ops = _ops()
    g = _gen(9)
    cb, idx, packed = _codebook_case(16, 64, 4, True, g)
    x = torch.randn(5, 64, generator=g).to(gpu)
    with pytest.raises(RuntimeError, match="residual shape"):
        ops.dimq_linear_codebook(x, packed.to(gpu), cb.to(gpu), 4, None, 16, 64,
                                 residual=torch.zeros(5, 15, device=gpu))
    with pytest.raises(KeyError):
        ops.dimq_linear_codebook(x, packed.to(gpu), cb.to(gpu), 4, None, 16, 64, activation="tanh")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_linear_codebook_cfg5_full_shape(gpu, M):
    """BASELINE cfg5 at full size: X bf16 [M, 4096], W [4096, 4096] N(0, 0.02), 3-bit per-channel codebook
    (8 centroids), indices packed across byte boundaries; the decode GEMV kernels."""
    ops = _ops()
    announce(f"linear_codebook cfg5 M={M}")
    g = _gen(40 + M)
    cb, idx, packed = _codebook_case(4096, 4096, 3, True, g)
    x = torch.randn(M, 4096, generator=g).bfloat16()
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 3, None, 4096, 4096,
                                 out_dtype=torch.float32)
    ref = oracle.linear_dequant_reference(x.float(), packed, 3, cb, 4096, 4096)
    assert oracle.rel_err(y, ref) <= TOL, oracle.rel_err(y, ref)


def test_linear_codebook_small_codebook_and_errors(gpu):
    ops = _ops()
    g = _gen(5)
    cb, idx, packed = _codebook_case(40, 64, 3, True, g, cb_entries=5)  # fewer entries than 2^b
    x = torch.randn(7, 64, generator=g)
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 3, None, 40, 64)
    ref = oracle.linear_dequant_reference(x, packed, 3, cb, 40, 64)
    assert oracle.rel_err(y, ref) <= TOL
    with pytest.raises(RuntimeError, match="packed_weight is too small"):
        ops.dimq_linear_codebook(x.to(gpu), packed[:5].to(gpu), cb.to(gpu), 3, None, 40, 64)
    with pytest.raises(RuntimeError, match="codebook rows must hold"):
        ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), torch.zeros(40, 9, device=gpu), 3, None, 40, 64)


# ---------------------------------------------------------------- weight-only codebook Conv2d
@pytest.mark.parametrize("case", [
    dict(B=2, C=16, H=10, W=9, OC=32, KH=3, KW=3, s=(1, 1), p=(1, 1), d=(1, 1), g=1, bits=2),
    dict(B=1, C=8, H=13, W=11, OC=8, KH=3, KW=3, s=(2, 2), p=(1, 1), d=(1, 1), g=1, bits=4),
    dict(B=2, C=3, H=23, W=23, OC=16, KH=7, KW=7, s=(2, 2), p=(3, 3), d=(1, 1), g=1, bits=8),
    dict(B=2, C=12, H=9, W=9, OC=16, KH=1, KW=1, s=(2, 2), p=(0, 0), d=(1, 1), g=1, bits=4),
    dict(B=1, C=8, H=9, W=10, OC=12, KH=3, KW=3, s=(1, 2), p=(2, 1), d=(2, 1), g=4, bits=3),
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_codebook_vs_oracle(gpu, case, layout):
    ops = _ops()
    announce(f"conv2d_codebook {case} {layout}")
    g = _gen(case["C"] * 31 + case["OC"] + case["bits"])
    shape = (case["OC"], case["C"] // case["g"], case["KH"], case["KW"])
    x = torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g).half()
    cb, idx, packed = _codebook_case(case["OC"], int(np.prod(shape[1:])), case["bits"], True, g)
    bias = torch.randn(case["OC"], generator=g) * 0.1
    xd = x.to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    y = ops.dimq_conv2d_codebook(xd, packed.to(gpu), cb.to(gpu), case["bits"], bias.to(gpu), shape, case["s"],
                                 case["p"], case["d"], case["g"], out_dtype=torch.float32)
    if layout == "nhwc":
        assert y.is_contiguous(memory_format=torch.channels_last)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb, shape, bias, case["s"], case["p"],
                                          case["d"], case["g"])
    assert y.shape == ref.shape
    assert oracle.rel_err(y.float(), ref) <= TOL, oracle.rel_err(y.float(), ref)


@pytest.mark.parametrize("variant", ["auto", "mfma"])
def test_conv2d_prepared_variants_agree(gpu, variant):
    """ResNet layer1 form (C 64, 3x3/1, NHWC fp16, prepared weight): the default LDS-halo kernel and, with
    variant "mfma", the implicit-GEMM tiles both meet the bar against the CPU reference."""
    ops = _ops()
    announce(f"conv prepared variant {variant}")
    g = _gen(1234)
    shape = (64, 64, 3, 3)
    x = torch.relu(torch.randn(2, 64, 20, 18, generator=g)).half()
    cb, idx, packed = _codebook_case(64, 576, 2, True, g)
    bias = torch.randn(64, generator=g) * 0.1
    pdv = packed.to(gpu)
    prep = ops.prepare_conv_weight(pdv, 2, shape)
    y = ops.dimq_conv2d_codebook(x.to(gpu).to(memory_format=torch.channels_last), pdv, cb.to(gpu), 2, bias.to(gpu),
                                 shape, (1, 1), (1, 1), (1, 1), 1, out_dtype=torch.float32, prepared_weight=prep,
                                 variant=variant)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, 2, cb, shape, bias, 1, 1, 1, 1)
    assert oracle.rel_err(y.float(), ref) <= TOL


# ---------------------------------------------------------------- small-channel stride-2 stem conv
@pytest.mark.parametrize("case", [
    dict(B=2, C=3, H=224, W=224, OC=64, K=7, p=3, bits=8, dt=torch.float16, out=torch.float16, pc=True),  # ResNet stem
    dict(B=1, C=3, H=230, W=226, OC=64, K=7, p=3, bits=8, dt=torch.float16, out=torch.float32, pc=False),  # partial band
    dict(B=3, C=3, H=37, W=37, OC=32, K=7, p=3, bits=4, dt=torch.bfloat16, out=torch.float32, pc=True),   # W*C odd
    dict(B=2, C=4, H=40, W=34, OC=64, K=7, p=2, bits=3, dt=torch.float16, out=torch.bfloat16, pc=True),   # even pad
    dict(B=2, C=3, H=50, W=50, OC=24, K=3, p=1, bits=2, dt=torch.float16, out=torch.float16, pc=True),    # 3x3/2 stem
    dict(B=2, C=3, H=33, W=35, OC=32, K=7, p=3, bits=4, dt=torch.float16, out=torch.float16, pc=True),    # odd W
    dict(B=1, C=1, H=31, W=29, OC=16, K=3, p=0, bits=8, dt=torch.float32, out=torch.float32, pc=True),    # fp32 input
    dict(B=2, C=2, H=20, W=18, OC=40, K=7, p=3, bits=8, dt=torch.float16, out=torch.float16, pc=True, cbn=200),
    # 16-bit codebooks (staged in LDS as floats), a per-layer one, and a packed stream one byte into its
    # storage (not 16-byte aligned: the generic kernel)
    dict(B=2, C=3, H=64, W=64, OC=64, K=7, p=3, bits=8, dt=torch.float16, out=torch.float16, pc=True,
         cbdt=torch.float16),
    dict(B=1, C=3, H=40, W=44, OC=32, K=7, p=3, bits=4, dt=torch.float16, out=torch.float32, pc=False,
         cbdt=torch.bfloat16),
    dict(B=1, C=3, H=30, W=30, OC=64, K=7, p=3, bits=8, dt=torch.float16, out=torch.float16, pc=True, woff=1),
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_stem_vs_oracle(gpu, case, layout):
    """C <= 4, stride-2 convs take the stem kernel; checked against the CPU reference and the generic path."""
    ops = _ops()
    announce(f"conv stem {case} {layout}")
    g = _gen(case["C"] * 7 + case["OC"] + case["bits"] + case["H"])
    K, pad = case["K"], case["p"]
    shape = (case["OC"], case["C"], K, K)
    x = torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g).to(case["dt"])
    cb, idx, packed = _codebook_case(case["OC"], case["C"] * K * K, case["bits"], case["pc"], g,
                                     cb_entries=case.get("cbn"))
    if case.get("cbdt") is not None:
        cb = cb.to(case["cbdt"])
    bias = torch.randn(case["OC"], generator=g) * 0.1
    xd = x.to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    pd = packed.to(gpu)
    if case.get("woff"):
        pd = torch.cat([torch.zeros(case["woff"], dtype=torch.uint8), packed]).to(gpu)[case["woff"]:]
    args = (xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, (2, 2), (pad, pad), (1, 1), 1)
    y = ops.dimq_conv2d_codebook(*args, out_dtype=case["out"])
    assert y.dtype == case["out"]
    if layout == "nhwc" and case["C"] > 1:  # a 1-channel input is NCHW- and NHWC-contiguous at once
        assert y.is_contiguous(memory_format=torch.channels_last)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb.float(), shape, bias, 2, pad, 1, 1)
    assert y.shape == ref.shape
    tol = out_tol(case["out"])
    assert oracle.rel_err(y.float(), ref) <= tol, oracle.rel_err(y.float(), ref)
    y2 = ops.dimq_conv2d_codebook(*args, out_dtype=torch.float32, variant="small_m")  # generic implicit GEMM
    assert oracle.rel_err(y.float(), y2) <= max(tol, 2e-3)


# ---------------------------------------------------------------- HIP graph replay
def test_graph_replay_matches_eager(gpu):
    """Kernels captured in a HIP graph give the eager result on every replay (bench.py times graphs)."""
    ops = _ops()
    g = _gen(123)
    cb, idx, packed = _codebook_case(128, 256, 4, True, g)
    x = torch.randn(64, 256, generator=g).to(gpu)
    cbc = (torch.randn(16, 4, generator=g) * 0.1).sort(dim=1).values.to(gpu)
    pc = torch.from_numpy(oracle.pack_bits(torch.randint(0, 4, (16, 144), generator=g, dtype=torch.uint8), 2)).to(gpu)
    xc = torch.randn(2, 16, 10, 10, generator=g).half().to(gpu)
    packed, cb = packed.to(gpu), cb.to(gpu)

    def run():
        y1 = ops.dimq_linear_codebook(x, packed, cb, 4, None, 128, 256)
        y2 = ops.dimq_conv2d_codebook(xc, pc, cbc, 2, None, (16, 16, 3, 3), (1, 1), (1, 1), (1, 1), 1,
                                      out_dtype=torch.float32)
        return y1, y2

    e1, e2 = run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o1, o2 = run()
    for r in range(3):
        o1.zero_()
        o2.zero_()
        _ = (x * 2).sum()  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1, e1) and torch.equal(o2, e2), f"replay {r}"


# ---------------------------------------------------------------- LDS-halo conv (prepared weights)
@pytest.mark.parametrize("case", [
    dict(B=2, C=64, H=56, W=56, OC=64, K=3, s=1, bits=2, dt=torch.float16),    # cfg2 geometry (smaller batch)
    dict(B=1, C=64, H=17, W=13, OC=128, K=3, s=1, bits=4, dt=torch.bfloat16),
    dict(B=2, C=128, H=28, W=28, OC=64, K=3, s=1, bits=3, dt=torch.float16),
    dict(B=2, C=64, H=56, W=56, OC=128, K=3, s=2, bits=2, dt=torch.float16),
    dict(B=3, C=128, H=14, W=14, OC=64, K=1, s=2, bits=4, dt=torch.float16),
    dict(B=1, C=64, H=9, W=300, OC=64, K=3, s=1, bits=2, dt=torch.float16),    # wide rows: implicit-GEMM fallback
    dict(B=2, C=128, H=56, W=56, OC=64, K=3, s=2, bits=2, dt=torch.float16),   # window staged without prefetch
    dict(B=32, C=64, H=56, W=56, OC=64, K=3, s=1, bits=2, dt=torch.float16),   # cfg2 shape: 8 bands per image
    dict(B=3, C=64, H=20, W=12, OC=192, K=3, s=1, bits=4, dt=torch.float16),   # 3 channel blocks, odd bands
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_halo_prepared_vs_oracle(gpu, case, layout):
    """Prepared weights: NCHW fp32-output 3x3 C 64 stride-1 calls take the band kernel, other NCHW calls the
    LDS-halo tiles, NHWC calls the halo tiles (C 64 stride 1) or the implicit GEMM."""
    ops = _ops()
    announce(f"conv halo {case} {layout}")
    g = _gen(case["C"] + case["OC"] * 3 + case["bits"] + case["s"])
    K = case["K"]
    pad = K // 2
    shape = (case["OC"], case["C"], K, K)
    x = torch.relu(torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g)).to(case["dt"])
    cb, idx, packed = _codebook_case(case["OC"], case["C"] * K * K, case["bits"], True, g)
    bias = torch.randn(case["OC"], generator=g) * 0.1
    xd = x.to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    pd = packed.to(gpu)
    prep = ops.prepare_conv_weight(pd, case["bits"], shape)
    assert prep is not None
    y = ops.dimq_conv2d_codebook(xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, (case["s"],) * 2,
                                 (pad, pad), (1, 1), 1, out_dtype=torch.float32, prepared_weight=prep)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb, shape, bias, case["s"], pad, 1, 1)
    assert y.shape == ref.shape
    assert oracle.rel_err(y.float(), ref) <= TOL, oracle.rel_err(y.float(), ref)
    y2 = ops.dimq_conv2d_codebook(xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, (case["s"],) * 2,
                                  (pad, pad), (1, 1), 1, out_dtype=torch.float32)
    assert oracle.rel_err(y, y2) <= 1e-5  # prepared (halo) and generic implicit-GEMM paths agree


@pytest.mark.parametrize("case", [
    dict(B=1, H=56, W=56, OC=64, bits=2, act=None, bias=False, pc=True, out=torch.float32),   # one block per part
    dict(B=3, H=20, W=24, OC=96, bits=3, act=None, bias=True, pc=True, out=torch.float32),    # OC tail
    dict(B=2, H=7, W=8, OC=64, bits=4, act="relu", bias=True, pc=False, out=torch.float32),   # partial last block
    dict(B=40, H=56, W=56, OC=64, bits=2, act="relu", bias=True, pc=True, out=torch.float32),  # 8 parts per image
    dict(B=16, H=28, W=32, OC=128, bits=4, act=None, bias=False, pc=True, out=torch.float32),  # 2 channel blocks
    dict(B=8, H=56, W=56, OC=64, bits=2, act="relu", bias=True, pc=True, out=torch.float16),   # fp16 output
    dict(B=3, H=7, W=8, OC=96, bits=3, act=None, bias=True, pc=False, out=torch.float16),      # fp16, partial block
    # NHWC only (ResNet-18 layer1's second conv): a 16-bit residual, then ReLU
    dict(B=4, H=56, W=56, OC=64, bits=2, act="relu", bias=True, pc=True, out=torch.float16, res=True),
    dict(B=3, H=7, W=8, OC=96, bits=3, act=None, bias=True, pc=False, out=torch.float16, res=True),
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_conv2d_band_kernel(gpu, case, layout):
    """fp16 3x3 stride-1 C 64 convs with fp32 or fp16 output in the input's layout (the band kernel: runs of
    32-pixel blocks per work-group, two-stage halo, stores through a wave-private LDS area; NCHW input
    transposed into the pixel-major halo, NHWC input copied as it is) against the oracle, with bias / ReLU,
    NHWC residuals, partial blocks, channel tails, 2/3/4-bit, per-layer and per-channel codebooks."""
    ops = _ops()
    if case.get("res") and layout == "nchw":
        pytest.skip("the residual cases are NHWC (ResNet's layout); NCHW residuals take the halo tiles")
    announce(f"conv band {case} {layout}")
    g = _gen(case["H"] * 7 + case["W"] + case["OC"] + case["bits"])
    shape = (case["OC"], 64, 3, 3)
    x = torch.relu(torch.randn(case["B"], 64, case["H"], case["W"], generator=g)).half()
    cb, idx, packed = _codebook_case(case["OC"], 576, case["bits"], case["pc"], g)
    bias = torch.randn(case["OC"], generator=g) * 0.1 if case["bias"] else None
    res = (torch.randn(case["B"], case["OC"], case["H"], case["W"], generator=g) * 0.5).half() if case.get("res") \
        else None
    fmt = torch.channels_last if layout == "nhwc" else torch.contiguous_format
    pd = packed.to(gpu)
    prep = ops.prepare_conv_weight(pd, case["bits"], shape)
    y = ops.dimq_conv2d_codebook(x.to(gpu).to(memory_format=fmt), pd, cb.to(gpu), case["bits"],
                                 None if bias is None else bias.to(gpu), shape, (1, 1), (1, 1), (1, 1), 1,
                                 out_dtype=case["out"], prepared_weight=prep, activation=case["act"],
                                 residual=None if res is None else res.to(gpu).to(memory_format=fmt))
    ref = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb, shape, bias, 1, 1, 1, 1)
    if res is not None:
        ref = ref + res.float()
    if case["act"] == "relu":
        ref = torch.relu(ref)
    assert y.shape == ref.shape and y.dtype == case["out"]
    assert y.is_contiguous(memory_format=fmt)
    tol = out_tol(case["out"])
    assert oracle.rel_err(y.float(), ref) <= tol, oracle.rel_err(y.float(), ref)


# ---------------------------------------------------------------- implicit-GEMM conv on large tiles (C % 64 == 0)
@pytest.mark.parametrize("case", [
    dict(B=2, C=256, H=14, W=14, OC=256, K=3, s=1, p=1, d=1, bits=2, dt=torch.float16, out=torch.float32),  # layer3
    dict(B=3, C=256, H=14, W=14, OC=512, K=3, s=2, p=1, d=1, bits=2, dt=torch.bfloat16, out=torch.float32),
    dict(B=2, C=512, H=7, W=7, OC=512, K=3, s=1, p=1, d=1, bits=2, dt=torch.float16, out=torch.float16),  # layer4
    dict(B=4, C=256, H=14, W=14, OC=512, K=1, s=2, p=0, d=1, bits=4, dt=torch.float16, out=torch.float16),
    dict(B=1, C=192, H=11, W=9, OC=96, K=5, s=1, p=3, d=2, bits=3, dt=torch.float16, out=torch.float32, pc=False),
    dict(B=1, C=64, H=9, W=9, OC=200, K=5, s=1, p=2, d=1, bits=4, dt=torch.bfloat16, out=torch.bfloat16, cbn=11),
])
@pytest.mark.parametrize("layout", ["nhwc", "nchw"])
def test_conv2d_gemm_prepared_vs_oracle(gpu, case, layout):
    """Tap-major prepared weights: NHWC takes the large-tile implicit GEMM, NCHW the generic kernel."""
    ops = _ops()
    announce(f"conv gemm {case} {layout}")
    g = _gen(case["C"] + case["OC"] + case["bits"] * 5 + case["K"])
    K = case["K"]
    shape = (case["OC"], case["C"], K, K)
    x = torch.relu(torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g)).to(case["dt"])
    cb, idx, packed = _codebook_case(case["OC"], case["C"] * K * K, case["bits"], case.get("pc", True), g,
                                     cb_entries=case.get("cbn"))
    bias = torch.randn(case["OC"], generator=g) * 0.1
    xd = x.to(gpu)
    if layout == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    pd = packed.to(gpu)
    prep = ops.prepare_conv_weight(pd, case["bits"], shape)
    assert prep is not None and prep.numel() == case["OC"] * case["C"] * K * K * case["bits"] // 32
    conv = (case["s"],) * 2, (case["p"],) * 2, (case["d"],) * 2, 1
    y = ops.dimq_conv2d_codebook(xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, *conv,
                                 out_dtype=case["out"], prepared_weight=prep)
    ref = oracle.conv2d_dequant_reference(x.float(), packed, case["bits"], cb, shape, bias, case["s"], case["p"],
                                          case["d"], 1)
    assert y.shape == ref.shape and y.dtype == case["out"]
    tol = out_tol(case["out"])
    assert oracle.rel_err(y.float(), ref) <= tol, oracle.rel_err(y.float(), ref)
    y2 = ops.dimq_conv2d_codebook(xd, pd, cb.to(gpu), case["bits"], bias.to(gpu), shape, *conv,
                                  out_dtype=torch.float32, variant="small_m")
    assert oracle.rel_err(y.float(), y2) <= tol


def test_conv2d_prepare_tapmajor_layout(gpu):
    """The tap-major stream holds index (oc, kh, kw, c) at k = (kh*KW + kw)*C + c, LSB-first, same bits."""
    ops = _ops()
    g = _gen(77)
    for bits in (2, 3, 4):
        OC, C, KH, KW = 5, 128, 3, 2
        idx = torch.randint(0, 1 << bits, (OC, C, KH, KW), generator=g, dtype=torch.uint8)
        packed = torch.from_numpy(oracle.pack_bits(idx.reshape(-1), bits)).to(gpu)
        prep = ops.prepare_conv_weight(packed, bits, (OC, C, KH, KW))
        want = oracle.pack_bits(idx.permute(0, 2, 3, 1).reshape(-1), bits)
        assert np.array_equal(prep.cpu().view(torch.uint8).numpy()[:want.size], want), bits


def test_conv2d_prepare_unsupported_returns_none(gpu):
    ops = _ops()
    assert ops.prepare_conv_weight(torch.zeros(100, dtype=torch.uint8, device=gpu), 2, (16, 48, 3, 3)) is None
    assert ops.prepare_conv_weight(torch.zeros(100, dtype=torch.uint8, device=gpu), 8, (16, 64, 3, 3)) is None


# ---------------------------------------------------------------- LayerNorm (ViT workload support op)
@pytest.mark.parametrize("rows,D,dt", [(12608, 768, torch.bfloat16), (300, 768, torch.float16), (5, 8, torch.bfloat16),
                                       (33, 1024, torch.bfloat16), (7, 2048, torch.float16), (130, 520, torch.bfloat16)])
def test_layer_norm_vs_torch_fp32(gpu, rows, D, dt):
    """HIP LayerNorm against torch's fp32 CPU layer_norm of the same 16-bit inputs: the only
    difference allowed is the one rounding of the output to fp16/bf16 (plus fp32 noise)."""
    ops = _ops()
    announce(f"layer_norm rows={rows} D={D} {dt}")
    g = _gen(rows + D)
    x = (torch.randn(rows, D, generator=g) * 3 + 0.5).to(dt)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dt)
    b = (0.1 * torch.randn(D, generator=g)).to(dt)
    y = ops.layer_norm(x.to(gpu), w.to(gpu), b.to(gpu), 1e-6).cpu()
    ref = torch.nn.functional.layer_norm(x.float(), (D,), w.float(), b.float(), 1e-6)
    ulp = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11  # half an output ulp is the rounding bound
    assert y.dtype == dt and y.shape == x.shape
    assert ((y.float() - ref).abs() <= ulp * ref.abs() + 1e-4).all()
    # the other 16-bit output format: the same fp32 result, rounded once to it
    odt = torch.float16 if dt == torch.bfloat16 else torch.bfloat16
    y2 = ops.layer_norm(x.to(gpu), w.to(gpu), b.to(gpu), 1e-6, out_dtype=odt).cpu()
    ulp2 = 2.0 ** -8 if odt == torch.bfloat16 else 2.0 ** -11
    assert y2.dtype == odt and y2.shape == x.shape
    assert ((y2.float() - ref).abs() <= ulp2 * ref.abs() + 1e-4).all()


def test_layer_norm_strided_rows_and_module(gpu):
    # x[:, 0] of a [B, N, D] activation (the ViT head's LayerNorm) is a strided row view
    from dimq_amd.modules import DIMQLayerNorm
    g = _gen(9)
    x = torch.randn(6, 197, 768, generator=g).bfloat16()
    ln = torch.nn.LayerNorm(768, eps=1e-6)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(768, generator=g))
        ln.bias.copy_(0.1 * torch.randn(768, generator=g))
    mod = DIMQLayerNorm.from_layer_norm(ln).to(gpu).bfloat16()
    xd = x.to(gpu)
    y = mod(xd[:, 0]).cpu()
    ref = torch.nn.functional.layer_norm(x[:, 0].float(), (768,), ln.weight.bfloat16().float(),
                                         ln.bias.bfloat16().float(), 1e-6)
    assert ((y.float() - ref).abs() <= 2.0 ** -8 * ref.abs() + 1e-4).all()
    torch.testing.assert_close(mod(xd).cpu()[:, 0], y, rtol=0, atol=0)
    with pytest.raises(RuntimeError, match="CUDA"):
        mod(x)


# ---------------------------------------------------------------- max pooling (ResNet workload support op)
@pytest.mark.parametrize("shape,k,s,p,dt", [((2, 64, 112, 112), 3, 2, 1, torch.float16),
                                            ((3, 16, 9, 10), 3, 2, 1, torch.bfloat16),
                                            ((2, 8, 7, 7), 2, 2, 0, torch.float16),
                                            ((1, 24, 5, 6), 3, 1, 1, torch.bfloat16)])
def test_max_pool2d_nhwc_vs_torch(gpu, shape, k, s, p, dt):
    """Channels-last HIP max pool against torch's CPU max_pool2d of the same values: exact, NaN included."""
    ops = _ops()
    announce(f"max_pool2d {shape} k={k} s={s} p={p} {dt}")
    x = torch.randn(shape, generator=_gen(sum(shape) + k)).to(dt)
    x[0, 1, 2, 3] = float("nan")
    x = x.contiguous(memory_format=torch.channels_last)
    y = ops.max_pool2d_nhwc(x.to(gpu), k, s, p)
    ref = torch.nn.functional.max_pool2d(x.float(), k, s, p)
    assert y.shape == ref.shape and y.dtype == dt and y.is_contiguous(memory_format=torch.channels_last)
    torch.testing.assert_close(y.cpu().float(), ref, rtol=0, atol=0, equal_nan=True)
    with pytest.raises(RuntimeError, match="channels-last"):
        ops.max_pool2d_nhwc(x.contiguous().to(gpu), k, s, p)


def test_benchmark_cuda_times_an_op(gpu):
    """benchmark_cuda (dimq_backend/benchmark.py:10-26): mean milliseconds per call between two HIP events,
    after the warm-up calls; every call runs (warmup + repeat of them)."""
    from dimq_amd import ops
    from dimq_amd.benchmark import benchmark_cuda
    idx = torch.randint(0, 8, (1 << 20,), dtype=torch.uint8, device=gpu)
    calls = []

    def fn():
        calls.append(1)
        return ops.pack_bits(idx, 3)

    ms = benchmark_cuda(fn, warmup=3, repeat=7)
    assert len(calls) == 10
    assert 0.0 < ms < 100.0
