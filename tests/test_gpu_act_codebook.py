"""Weight x activation codebooks: the codebook product table, the index x index LUT-gather Linear (decode shapes),
the dequantize-then-MFMA form at larger M, the Conv2d form, and the layers / packed checkpoint that carry the QAT
wrapper's activation_centers (quant/dimq_wrapper.py:80-85, quant/export_dimq.py:81-86).

Reference semantics: q = C_a[argmin_c (x - C_a[c])^2].to(x.dtype) (hard_quantize_weight, quant/dimq.py:197-221),
then F.linear / F.conv2d over W_hat = C_w[idx] in fp32 on the CPU."""

import pytest
import torch
import torch.nn.functional as F

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


def _weights(N, K, bits, per_channel, g):
    rows = N if per_channel else 1
    cb = (torch.randn(rows, 1 << bits, generator=g) * 0.05).sort(dim=1).values
    idx = torch.randint(0, 1 << bits, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, bits))
    return (cb if per_channel else cb[0]), idx, packed


def _quantize(x, ca):
    xf = x.float().reshape(-1)
    a = ((xf[:, None] - ca[None, :]) ** 2).argmin(1)
    return a.reshape(x.shape), ca[a].reshape(x.shape).to(x.dtype).float()


def test_codebook_product_table(gpu):
    ops = _ops()
    g = _gen(1)
    for rows, kw, ka, dt in ((1, 16, 16, torch.float16), (300, 8, 16, torch.float32), (64, 4, 256, torch.bfloat16)):
        cw = (torch.randn(rows, kw, generator=g) * 0.1).to(dt)
        ca = torch.randn(ka, generator=g)
        t = ops.build_codebook_product_table(cw.to(gpu), ca.to(gpu))
        assert t.shape == (rows, kw, ka) and t.dtype == torch.float32
        assert torch.equal(t.cpu(), cw.float()[:, :, None] * ca[None, None, :])


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("bits,per_channel,n_act", [(2, True, 16), (3, True, 16), (4, True, 16), (4, False, 256),
                                                    (3, False, 64), (4, True, 8)])
def test_linear_lut_act_gather_vs_reference(gpu, M, bits, per_channel, n_act):
    ops = _ops()
    announce(f"linear_lut_act M={M} bits={bits} pc={per_channel} n_act={n_act}")
    N, K = 200, 1024
    g = _gen(M * 31 + bits + n_act)
    cb, idx, packed = _weights(N, K, bits, per_channel, g)
    ca = torch.randn(n_act, generator=g).sort().values
    bias = torch.randn(N, generator=g) * 0.1
    for xdt in (torch.float32, torch.bfloat16):
        x = torch.randn(M, K, generator=g).to(xdt)
        a, q = _quantize(x, ca)
        y = ops.dimq_linear_lut_act(a.to(torch.uint8).to(gpu), packed.to(gpu), cb.to(gpu), bits, ca.to(gpu), xdt,
                                    bias.to(gpu), N, K)
        ref = oracle.linear_dequant_reference(q, packed, bits, cb, N, K, bias)
        # fp32 products and fp32 sums, only the order differs
        assert oracle.rel_err(y, ref) <= 2e-5, (xdt, oracle.rel_err(y, ref))


@pytest.mark.parametrize("M,N,K,bits,xdt", [(1, 4096, 4096, 3, torch.bfloat16), (4, 300, 768, 4, torch.float32),
                                            (3, 130, 96, 2, torch.float16), (16, 512, 2048, 4, torch.bfloat16)])
def test_linear_codebook_act_variants_agree(gpu, M, N, K, bits, xdt):
    """The LUT-gather variant (small_m) and the dequantize-then-MFMA variant (mfma) against the reference."""
    ops = _ops()
    announce(f"linear_codebook_act variants M={M} N={N} K={K} bits={bits} {xdt}")
    g = _gen(M + N + K)
    cb, idx, packed = _weights(N, K, bits, True, g)
    ca = torch.randn(16, generator=g).sort().values
    bias = torch.randn(N, generator=g) * 0.1
    x = torch.randn(M, K, generator=g).to(xdt)
    _, q = _quantize(x, ca)
    ref = oracle.linear_dequant_reference(q, packed, bits, cb, N, K, bias)
    for variant in ("auto", "small_m", "mfma"):
        y = ops.dimq_linear_codebook_act(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, ca.to(gpu), bias.to(gpu), N,
                                         K, out_dtype=torch.float32, variant=variant)
        assert oracle.rel_err(y, ref) <= TOL, (variant, oracle.rel_err(y, ref))


@pytest.mark.parametrize("case", [
    dict(B=2, C=64, H=14, W=14, OC=64, K=3, s=1, p=1, bits=2, dt=torch.bfloat16, layout="nhwc", prep=True),
    dict(B=2, C=16, H=11, W=9, OC=24, K=3, s=2, p=1, bits=4, dt=torch.float32, layout="nchw", prep=False),
    dict(B=1, C=64, H=9, W=9, OC=32, K=1, s=1, p=0, bits=3, dt=torch.float16, layout="nchw", prep=True),
])
def test_conv2d_codebook_act_vs_reference(gpu, case):
    ops = _ops()
    announce(f"conv2d_codebook_act {case}")
    g = _gen(case["C"] + case["OC"] + case["bits"])
    shape = (case["OC"], case["C"], case["K"], case["K"])
    cb, idx, packed = _weights(case["OC"], case["C"] * case["K"] ** 2, case["bits"], True, g)
    ca = (torch.rand(16, generator=g) * 3).sort().values
    bias = torch.randn(case["OC"], generator=g) * 0.1
    x = torch.relu(torch.randn(case["B"], case["C"], case["H"], case["W"], generator=g)).to(case["dt"])
    _, q = _quantize(x, ca)
    xd = x.to(gpu)
    if case["layout"] == "nhwc":
        xd = xd.to(memory_format=torch.channels_last)
    pg = packed.to(gpu)
    prep = ops.prepare_conv_weight(pg, case["bits"], shape) if case["prep"] else None
    y = ops.dimq_conv2d_codebook_act(xd, pg, cb.to(gpu), case["bits"], ca.to(gpu), bias.to(gpu), shape, case["s"],
                                     case["p"], out_dtype=torch.float32, prepared_weight=prep)
    ref = oracle.conv2d_dequant_reference(q, packed, case["bits"], cb, shape, bias, case["s"], case["p"])
    assert y.shape == ref.shape
    assert oracle.rel_err(y.float(), ref) <= TOL, oracle.rel_err(y.float(), ref)


def test_layers_and_checkpoint_with_activation_centers(gpu, tmp_path):
    """A compact checkpoint whose layers carry the QAT wrapper's activation codebook exports (weight-only layout)
    with activation_centers, reloads with weights_only=True, and its layers quantize activations before the
    weight-codebook product."""
    from dimq_amd.export import export_packed_dimq_checkpoint
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear, make_packed_layer

    g = _gen(5)
    lin_idx = torch.randint(0, 8, (96, 128), generator=g)
    conv_idx = torch.randint(0, 4, (32, 16, 3, 3), generator=g)
    ca_lin = torch.randn(16, generator=g).sort().values
    ca_conv = (torch.rand(8, generator=g) * 2).sort().values
    compact = {
        "format": "dimq_compact",
        "layers": {
            "fc": {"shape": [96, 128], "bits": 3, "centers": (torch.randn(96, 8, generator=g) * 0.05).sort(1).values,
                   "indices": lin_idx, "activation_bits": 4, "activation_centers": ca_lin},
            "conv": {"shape": [32, 16, 3, 3], "bits": 2,
                     "centers": (torch.randn(32, 4, generator=g) * 0.1).sort(1).values, "indices": conv_idx,
                     "activation_bits": 3, "activation_centers": ca_conv},
        },
        "non_quantized_state_dict": {"fc.bias": torch.randn(96, generator=g) * 0.1},
    }
    path = tmp_path / "packed.pt"
    export_packed_dimq_checkpoint(compact, path, layer_hparams={"conv": {"type": "conv2d", "padding": (1, 1)}})
    state = torch.load(path, map_location="cpu", weights_only=True)
    assert state["activation_quantization"] == "codebook"
    lf, lc = state["layers"]["fc"], state["layers"]["conv"]
    assert lf["activation_quantization"] == "codebook" and lf["bit_a"] == 4
    assert torch.equal(lf["activation_centers"], ca_lin) and torch.equal(lc["activation_centers"], ca_conv)
    fc = make_packed_layer(lf).to(gpu)
    conv = make_packed_layer(lc).to(gpu)
    assert isinstance(fc, DIMQCodebookLinear) and isinstance(conv, DIMQCodebookConv2d)
    for M in (1, 37):
        x = torch.randn(M, 128, generator=g)
        _, q = _quantize(x, ca_lin)
        w_hat = torch.gather(lf["codebook"].float(), 1, lin_idx.long())
        ref = F.linear(q, w_hat, lf["bias"].float())
        assert oracle.rel_err(fc(x.to(gpu)).float(), ref) <= TOL
    x = torch.relu(torch.randn(2, 16, 10, 10, generator=g)).half()
    _, q = _quantize(x, ca_conv)
    w_hat = torch.gather(lc["codebook"].float(), 1, conv_idx.reshape(32, -1).long()).reshape(32, 16, 3, 3)
    ref = F.conv2d(q, w_hat, None, 1, 1)
    assert oracle.rel_err(conv(x.to(gpu)).float(), ref) <= TOL
