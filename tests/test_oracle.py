"""CPU checks that pin the oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against the committed golden vectors
(tests/golden/, built by an independent bit-list / torch-library formulation),
against torch CPU library routines on random inputs, and against closed forms.
A few tests plant a plausible mistake in a copy of the oracle's formula and
show that the goldens reject it.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    return json.loads((GOLD / name).read_text())


# ---------------------------------------------------------------- codec
def test_codec_golden_vectors():
    cases = _load("codec_vectors.json")
    assert len(cases) > 80
    for c in cases:
        bits = c["bits"]
        idx = np.array(c["indices"], dtype=np.uint8)
        want = bytes.fromhex(c["packed"].replace(" ", "")) if c["packed"] else b""
        got = oracle.pack_bits(idx, bits).tobytes()
        assert got == want, (bits, len(idx), c["source"])
        back = oracle.unpack_bits(np.frombuffer(want, dtype=np.uint8), len(idx), bits)
        assert np.array_equal(back, idx)


def test_codec_sizes_and_masking():
    for bits in (2, 3, 4, 8):
        for n in (0, 1, 7, 8, 9, 100):
            assert oracle.packed_nbytes(n, bits) == (n * bits + 7) // 8
    # values are masked to the field width (csrc/dimq_pack.cu:19-22)
    assert oracle.pack_bits([0x1F, 0x2E], 4).tobytes() == bytes([0xEF])
    with pytest.raises(ValueError):
        oracle.unpack_bits(np.zeros(1, np.uint8), 3, 4)


def test_codec_planted_msb_first_is_rejected():
    """An MSB-first packer (a plausible mistake) disagrees with the goldens."""
    def msb_pack(idx, bits):
        out = bytearray((len(idx) * bits + 7) // 8)
        pos = 0
        for v in idx:
            for j in reversed(range(bits)):
                if (v >> j) & 1:
                    out[pos >> 3] |= 0x80 >> (pos & 7)
                pos += 1
        return bytes(out)

    cases = [c for c in _load("codec_vectors.json") if len(c["indices"]) >= 2]
    assert any(msb_pack(c["indices"], c["bits"]).hex(" ") != c["packed"] for c in cases if c["bits"] != 8)


def test_u4_reference_recipe():
    # dimq_cuda_backend/tests/test_reference_and_export.py:19-27
    idx = np.arange(17, dtype=np.uint8) % 16
    packed = oracle.pack_bits(idx, 4)
    assert packed.size == 9
    assert np.array_equal(oracle.unpack_bits(packed, 17, 4), idx)


# ---------------------------------------------------------------- hard quantization
def test_hardquant_golden_vectors():
    for c in _load("hardquant_vectors.json"):
        idx, val = oracle.hard_quantize(np.array(c["w"], np.float32), np.array(c["centers"], np.float32))
        assert idx.tolist() == c["idx"], c["source"]
        assert np.array_equal(val, np.array(c["centers"], np.float32)[np.array(c["idx"])])


def test_hardquant_matches_torch_argmin_random_and_per_channel():
    g = torch.Generator().manual_seed(0)
    for K in (2, 3, 4, 8, 16, 100, 256):
        w = torch.randn(7, 333, generator=g) * 0.03
        c = torch.randn(7, K, generator=g) * 0.03
        want = ((w[:, :, None] - c[:, None, :]) ** 2).argmin(-1)
        idx, _ = oracle.hard_quantize(w, c, per_channel=True)
        assert np.array_equal(idx, want.numpy().astype(np.uint8)), K
        want1 = ((w.reshape(-1)[:, None] - c[0][None, :]) ** 2).argmin(-1).reshape(w.shape)
        idx1, _ = oracle.hard_quantize(w, c[0], per_channel=False)
        assert np.array_equal(idx1, want1.numpy().astype(np.uint8))


def test_hardquant_nan_semantics_match_torch():
    w = torch.tensor([0.5, float("nan"), 2.0, float("inf")])
    c = torch.tensor([0.0, float("nan"), 1.0, 3.0])
    want = ((w[:, None] - c[None, :]) ** 2).argmin(1)
    idx, _ = oracle.hard_quantize(w, c)
    assert idx.tolist() == want.tolist()
    c2 = torch.tensor([0.0, 1.0, 3.0])
    want2 = ((w[:, None] - c2[None, :]) ** 2).argmin(1)
    assert oracle.hard_quantize(w, c2)[0].tolist() == want2.tolist()


# ---------------------------------------------------------------- activation quantization
def test_actquant_golden_vectors():
    for c in _load("actquant_vectors.json"):
        q = oracle.quantize_act_u4(np.array(c["x"], np.float32), c["scale"], c["zp"])
        assert q.tolist() == c["q"], c["source"]


def test_actquant_matches_torch_round_half_even():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(100000, generator=g) * 3
    for s, zp in ((0.2, 7), (0.1, 8), (0.3, 3), (2.0 ** -3, 8), (0.0731, 0)):
        want = torch.clamp(torch.round(x / float(s)) + zp, 0, 15).to(torch.uint8)
        assert np.array_equal(oracle.quantize_act_u4(x, s, zp), want.numpy())


def test_actquant_nan_inf_semantics():
    """+-inf and out-of-range quotients clamp like the torch reference (reference.py:11-21); a NaN gives zp,
    as the reference CUDA kernel's __float2int_rn(NaN) = 0 plus zp (csrc/dimq_common.cuh:17-21) -- torch leaves
    NaN's uint8 cast unspecified, so the CUDA kernel is the anchor there."""
    x = torch.tensor([float("inf"), float("-inf"), 1e30, -1e30, 3.0e9, -3.0e9])
    for s, zp in ((0.2, 7), (2.0 ** -3, 8), (1.0, 0), (0.5, 15)):
        want = torch.clamp(torch.round(x / float(s)) + zp, 0, 15).to(torch.uint8)
        assert np.array_equal(oracle.quantize_act_u4(x, s, zp), want.numpy())
        q = oracle.quantize_act_u4(np.array([float("nan"), 1.0, float("nan")], np.float32), s, zp)
        assert q[0] == zp and q[2] == zp


# ---------------------------------------------------------------- product table
def test_product_table_golden():
    c = _load("product_table_vectors.json")[0]
    t = oracle.product_table(np.array(c["codebook"], np.float32), c["scale"], c["zp"])
    assert np.array_equal(t, np.array(c["table"], np.float32))
    assert t[0, 0] == 1.0 and t[15, 15] == 0.875 and t[7, 3] == np.float32(0.04180908203125)


def test_product_table_grouped_closed_form():
    g = torch.Generator().manual_seed(2)
    cb = torch.randn(5, 16, generator=g)
    t = oracle.product_table(cb, 0.37, 5)
    a = (np.float32(0.37) * (np.arange(16, dtype=np.float32) - 5)).astype(np.float32)
    assert np.array_equal(t, (cb.numpy()[:, :, None] * a[None, None, :]).astype(np.float32))


# ---------------------------------------------------------------- LUT linear / conv (W4A4)
def test_linear_lut_recipe_golden_and_equivalence():
    r = _load("w4a4_recipes.json")["linear"]
    x = torch.tensor(r["x"])
    idx = np.array(r["indices"], np.uint8)
    packed = oracle.pack_bits(idx, 4)
    y = oracle.linear_lut(x, packed, torch.tensor(r["codebook"]), r["scale"], r["zp"], torch.tensor(r["bias"]), 6, 11)
    np.testing.assert_allclose(y, np.array(r["y"], np.float32), rtol=0, atol=1e-6)
    y2 = oracle.linear_a4_dequant_reference(x, packed, torch.tensor(r["codebook"]), r["scale"], r["zp"], 6, 11,
                                            torch.tensor(r["bias"]))
    np.testing.assert_allclose(y, y2.numpy(), rtol=0, atol=1e-6)


def test_conv_lut_recipe_golden_and_equivalence():
    r = _load("w4a4_recipes.json")["conv2d"]
    x = torch.tensor(r["x"])
    idx = np.array(r["indices"], np.uint8)
    packed = oracle.pack_bits(idx, 4)
    kw = dict(stride=tuple(r["stride"]), padding=tuple(r["padding"]), dilation=tuple(r["dilation"]),
              groups=r["groups"])
    y = oracle.conv2d_lut(x, packed, torch.tensor(r["codebook"]), r["scale"], r["zp"], torch.tensor(r["bias"]),
                          idx.shape, **kw)
    np.testing.assert_allclose(y, np.array(r["y"], np.float32), rtol=0, atol=1e-5)
    y2 = oracle.conv2d_a4_dequant_reference(x, packed, torch.tensor(r["codebook"]), r["scale"], r["zp"], idx.shape,
                                            torch.tensor(r["bias"]), **kw)
    np.testing.assert_allclose(y, y2.numpy(), rtol=0, atol=1e-5)


def test_conv_lut_groups_dilation_equivalence():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 4, 7, 6, generator=g)
    idx = torch.randint(0, 16, (6, 2, 3, 2), generator=g, dtype=torch.uint8)
    cb = torch.linspace(-0.6, 0.7, 16)
    bias = torch.randn(6, generator=g)
    packed = oracle.pack_bits(idx, 4)
    kw = dict(stride=(1, 2), padding=(2, 1), dilation=(2, 1), groups=2)
    y = oracle.conv2d_lut(x, packed, cb, 0.3, 6, bias, idx.shape, **kw)
    y2 = oracle.conv2d_a4_dequant_reference(x, packed, cb, 0.3, 6, idx.shape, bias, **kw)
    np.testing.assert_allclose(y, y2.numpy(), rtol=0, atol=1e-5)


# ---------------------------------------------------------------- weight-only dequant references
def test_weight_only_recipes_golden():
    for key, r in _load("weight_only_recipes.json").items():
        bits = r["bits"]
        idx = np.array(r["indices"], np.uint8)
        packed = oracle.pack_bits(idx, bits)
        y = oracle.linear_dequant_reference(torch.tensor(r["x"]), packed, bits, torch.tensor(r["codebook"]),
                                            idx.shape[0], idx.shape[1], torch.tensor(r["bias"]))
        np.testing.assert_allclose(y.numpy(), np.array(r["y"], np.float32), rtol=1e-6, atol=1e-6, err_msg=key)


def test_dequantize_planted_row_swap_is_rejected():
    """Swapping the per-channel codebook rows (a plausible indexing mistake) changes the result."""
    r = _load("weight_only_recipes.json")["linear_b3"]
    idx = np.array(r["indices"], np.uint8)
    packed = oracle.pack_bits(idx, 3)
    cb = np.array(r["codebook"], np.float32)
    good = oracle.dequantize(packed, 3, cb, idx.shape[0], idx.shape[1])
    bad = oracle.dequantize(packed, 3, cb[::-1].copy(), idx.shape[0], idx.shape[1])
    want = np.take_along_axis(cb, idx.astype(np.int64), axis=1)
    assert np.array_equal(good, want) and not np.array_equal(bad, want)


def test_conv_dequant_reference_matches_direct_sum():
    """Brute-force direct convolution on a tiny case pins the torch F.conv2d usage."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 2, 5, 4, generator=g)
    cb = torch.randn(3, 4, generator=g)
    idx = torch.randint(0, 4, (3, 2, 3, 3), generator=g, dtype=torch.uint8)
    packed = oracle.pack_bits(idx, 2)
    y = oracle.conv2d_dequant_reference(x, packed, 2, cb, idx.shape, None, 1, 1, 1, 1).numpy()
    w = torch.gather(cb, 1, idx.reshape(3, -1).long()).reshape(3, 2, 3, 3).numpy()
    xp = np.pad(x.numpy(), ((0, 0), (0, 0), (1, 1), (1, 1)))
    ref = np.zeros((1, 3, 5, 4), np.float64)
    for co in range(3):
        for oh in range(5):
            for ow in range(4):
                ref[0, co, oh, ow] = (xp[0, :, oh:oh + 3, ow:ow + 3] * w[co]).sum()
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_a4_exact_bar_accepts_summation_order_and_rejects_planted_zero_point():
    """The W4A4 fast-path bar (float64-exact deviation at most twice the fp32 LUT loop's): an fp32 sum in
    another order passes at K = 4096; the oracle's own LUT with a wrong zero point fails."""
    import torch
    from tests.a4_check import a4_exact_check, a4_levels

    g = torch.Generator().manual_seed(4096)
    M, N, K = 2, 512, 4096
    x = torch.randn(M, K, generator=g)
    idx = torch.randint(0, 16, (N, K), generator=g, dtype=torch.uint8)
    cb = (torch.linspace(-0.5, 0.5, 16) + 0.01 * torch.randn(16, generator=g)).half()
    bias = torch.randn(N, generator=g)
    packed = torch.from_numpy(oracle.pack_bits(idx, 4))
    ref = oracle.linear_lut(x, packed, cb.float(), 0.2, 7, bias, N, K)
    lv = a4_levels(x, 0.2, 7)
    exact = lv @ cb.double()[idx.long()].T + bias.double()
    other_order = (lv.float() / 0.2) @ cb.float()[idx.long()].T * 0.2 + bias  # blocked fp32, scale last
    a4_exact_check(other_order, ref, exact, K)
    planted = torch.from_numpy(oracle.linear_lut(x, packed, cb.float(), 0.2, 6, bias, N, K))
    with pytest.raises(AssertionError):
        a4_exact_check(planted, ref, exact, K)


# ---------------------------------------------------------------- QAT oracle (oracle/qat.py)
def test_qat_oracle_closed_forms():
    """The float64 restatements of quant/dimq.py:224-296 against closed forms that do not retype them."""
    import math
    import torch
    from oracle import qat

    g = torch.Generator().manual_seed(4)
    w = torch.randn(500, generator=g, dtype=torch.float64) * 0.1
    # one centre: the softmin term is the plain squared distance, for any tau
    c1 = torch.tensor([0.03], dtype=torch.float64)
    for tau in (1e-6, 0.01, 10.0):
        assert torch.allclose(qat.softmin_loss(w, c1, tau), ((w - 0.03) ** 2).sum(), rtol=1e-12, atol=1e-15)
    # two centres: min(d) - tau (log1p(exp(-|d1 - d2| / tau)) - log 2) per element
    c2 = torch.tensor([-0.05, 0.07], dtype=torch.float64)
    d1, d2 = (w + 0.05) ** 2, (w - 0.07) ** 2
    for tau in (1e-4, 0.003, 0.5):
        want = (torch.minimum(d1, d2) - tau * (torch.log1p(torch.exp(-(d1 - d2).abs() / tau)) - math.log(2))).sum()
        assert torch.allclose(qat.softmin_loss(w, c2, tau), want, rtol=1e-10)
        assert torch.allclose(qat.softmin_loss(w, c2, tau, "mean_per_layer"), want / w.numel(), rtol=1e-10)
        # soft dequantization with two centres: a logistic blend
        p1 = 1.0 / (1.0 + torch.exp(-(d2 - d1) / tau))
        assert torch.allclose(qat.soft_dequantize(w, c2, tau), p1 * -0.05 + (1 - p1) * 0.07, rtol=1e-10, atol=1e-15)
    # tau -> 0: the hard nearest-centre distortion; tau -> inf: the mean over the centres
    c = torch.randn(8, generator=g, dtype=torch.float64) * 0.1
    d = (w[:, None] - c[None, :]) ** 2
    assert torch.allclose(qat.softmin_loss(w, c, 1e-12), d.min(dim=1).values.sum(), rtol=1e-9)
    assert torch.allclose(qat.softmin_loss(w, c, 1e6), d.mean(dim=1).sum(), rtol=1e-6)
    assert torch.allclose(qat.soft_dequantize(w, c, 1e9), torch.full_like(w, float(c.mean())), rtol=1e-6)
    nearest = c[d.argmin(dim=1)]
    assert torch.allclose(qat.soft_dequantize(w, c, 1e-12), nearest)
    # separation: two centres closer than the margin, and far apart
    sigma = float(w.std(unbiased=False))
    for gap in (0.1 * sigma, 10 * sigma):
        cc = torch.tensor([0.0, gap], dtype=torch.float64)
        want = max(0.0, 1.5 * 6 * sigma / 2 - math.sqrt(gap * gap + 1e-12)) ** 2
        assert math.isclose(float(qat.separation_loss(w, cc, 1.5)), want, rel_tol=1e-12, abs_tol=1e-18)
    assert float(qat.separation_loss(w, c1)) == 0.0


def test_qat_oracle_finite_differences():
    """Autograd of the restatements against finite differences (float64): the gradients the reference gets
    from torch's autograd."""
    import torch
    from oracle import qat

    g = torch.Generator().manual_seed(5)
    w = (torch.randn(40, generator=g, dtype=torch.float64) * 0.1).requires_grad_()
    c = (torch.randn(6, generator=g, dtype=torch.float64) * 0.1).requires_grad_()
    for tau in (1e-3, 0.05):
        assert torch.autograd.gradcheck(lambda a, b: qat.softmin_loss(a, b, tau), (w, c))
        assert torch.autograd.gradcheck(lambda a, b: qat.soft_dequantize(a, b, tau), (w, c))
    cs = torch.tensor([0.0, 0.01, 0.015, 0.3], dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda b: qat.separation_loss(w.detach(), b, 2.0), (cs,))


# ---------------------------------------------------------------- end-to-end model reference
def _bit_list_pack(idx, bits):
    """LSB-first bitstream written bit by bit (the packed format of dimq_backend/export.py:38-55, generalised)."""
    flat = [int(v) for v in np.asarray(idx).reshape(-1)]
    out = bytearray((len(flat) * bits + 7) // 8)
    for i, v in enumerate(flat):
        for b in range(bits):
            if (v >> b) & 1:
                out[(i * bits + b) // 8] |= 1 << ((i * bits + b) % 8)
    return torch.tensor(list(out), dtype=torch.uint8)


@torch.no_grad()
def test_dequantized_model_matches_gathered_float_layers():
    """oracle.dequantized_model (the CPU reference of the end-to-end forwards) against a model written out by
    hand: W_hat gathered with torch indexing from the indices (C[n, idx[n, k]], reference.py:47-56), then
    F.conv2d / F.linear in fp32 (quant/dimq_wrapper.py:189-197,237-240), torch's LayerNorm and max pool for the
    HIP support layers.  Covers a strided, padded, dilated, grouped conv with a per-channel codebook, a Linear
    with a per-layer codebook and no bias, 2/3/8-bit indices, and the layers' order and hyper-parameters."""
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear, DIMQLayerNorm, DIMQMaxPool2d

    g = torch.Generator().manual_seed(11)
    shape = (8, 3, 3, 2)                        # OC 8, groups 2 -> 3 input channels per group, 3x2 kernel
    cidx = torch.randint(0, 4, shape, generator=g, dtype=torch.uint8)
    ccb = torch.randn(8, 4, generator=g).sort(dim=1).values
    cbias = torch.randn(8, generator=g)
    conv = DIMQCodebookConv2d(_bit_list_pack(cidx, 2), ccb, 2, shape, cbias, stride=(2, 1), padding=(1, 2),
                              dilation=(1, 2), groups=2)
    x = torch.randn(2, 6, 9, 8, generator=g)
    conv_out = F.conv2d(x, ccb[torch.arange(8)[:, None], cidx.reshape(8, -1).long()].reshape(shape), cbias, (2, 1),
                        (1, 2), (1, 2), 2)
    pooled = F.max_pool2d(conv_out, 2, 2, 0)
    D = pooled[0].numel()
    lidx = torch.randint(0, 8, (5, D), generator=g, dtype=torch.uint8)
    lcb = torch.randn(1, 8, generator=g).sort(dim=1).values
    lin = DIMQCodebookLinear(_bit_list_pack(lidx, 3), lcb, 3, 5, D, None)
    ln = DIMQLayerNorm(5)
    ln.weight.data = torch.randn(5, generator=g)
    ln.bias.data = torch.randn(5, generator=g)
    hidx = torch.randint(0, 256, (4, 5), generator=g, dtype=torch.uint8)
    hcb = torch.randn(4, 256, generator=g)
    hbias = torch.randn(4, generator=g)
    head = DIMQCodebookLinear(_bit_list_pack(hidx, 8), hcb, 8, 4, 5, hbias)
    model = torch.nn.Sequential(conv, DIMQMaxPool2d(2, 2, 0), torch.nn.Flatten(), lin, ln, head)

    got = oracle.dequantized_model(model)(x)
    h = pooled.flatten(1) @ lcb[0][lidx.long()].T
    h = F.layer_norm(h, (5,), ln.weight, ln.bias, ln.eps)
    want = F.linear(h, hcb[torch.arange(4)[:, None], hidx.long()], hbias)
    torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)
    # a planted mistake: the conv's codebook rows taken in reverse order
    bad = oracle.dequantized_model(torch.nn.Sequential(
        DIMQCodebookConv2d(_bit_list_pack(cidx, 2), ccb.flip(0), 2, shape, cbias, stride=(2, 1), padding=(1, 2),
                           dilation=(1, 2), groups=2)))(x)
    assert not torch.allclose(bad, conv_out, rtol=1e-3, atol=1e-3)
