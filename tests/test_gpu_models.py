"""End-to-end forwards of the two BASELINE models through the codebook layers,
against the dequantize-then-float CPU model (oracle.dequantized_model).

Activations run in bf16 (ViT) / fp16 (ResNet) on the GPU and in fp32 on the
CPU, and every layer's output is rounded to 16 bits before the next layer
reads it, so the bound is looser than the single-layer one: max|err|/max|ref|
of the logits <= 1.5e-2 (LOGITS_TOL)."""

from __future__ import annotations

import pytest
import torch

import oracle
from tests.conftest import announce, out_tol

pytestmark = pytest.mark.gpu

LOGITS_TOL = 1.5e-2


def _cast_float_params(model, dtype):
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear
    for mod in model.modules():
        if isinstance(mod, (DIMQCodebookConv2d, DIMQCodebookLinear)):
            continue
        for name, prm in list(mod._parameters.items()):
            if prm is not None:
                mod._parameters[name] = torch.nn.Parameter(prm.detach().to(dtype), requires_grad=False)
    return model


@torch.no_grad()
def test_vit_small_forward_vs_dequant_reference(gpu):
    from dimq_amd.bench_models import ViT, quantize_vit
    from dimq_amd.modules import DIMQCodebookLinear
    announce("vit small forward")
    torch.manual_seed(0)
    m = ViT(image=32, patch=8, dim=128, depth=2, heads=4, mlp=256, classes=10)
    for mod in m.modules():
        if isinstance(mod, torch.nn.Linear):
            torch.nn.init.normal_(mod.weight, std=0.02)
    m = _cast_float_params(quantize_vit(m.cuda(), 4, out_dtype=torch.bfloat16), torch.bfloat16).eval()
    n_q = sum(isinstance(x, DIMQCodebookLinear) for x in m.modules())
    assert n_q == 2 * 4            # qkv, proj, fc1, fc2 per block
    x = torch.randn(3, 3, 32, 32)
    y = m(x.cuda().bfloat16()).float().cpu()
    ref = oracle.dequantized_model(m)(x)
    assert oracle.rel_err(y, ref) <= LOGITS_TOL, oracle.rel_err(y, ref)


@torch.no_grad()
def test_resnet18_forward_vs_dequant_reference(gpu):
    from dimq_amd.bench_models import quantize_resnet18, resnet18
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear
    announce("resnet18 forward 2x3x64x64")
    m = resnet18().cuda().to(memory_format=torch.channels_last)
    m = _cast_float_params(quantize_resnet18(m, out_dtype=torch.float16), torch.float16).eval()
    convs = [x for x in m.modules() if isinstance(x, DIMQCodebookConv2d)]
    assert len(convs) == 20 and sum(isinstance(x, DIMQCodebookLinear) for x in m.modules()) == 1
    assert sorted({c.bits for c in convs}) == [2, 4, 8]
    x = torch.randn(2, 3, 64, 64)
    y = m(x.cuda().half().contiguous(memory_format=torch.channels_last)).float().cpu()
    ref = oracle.dequantized_model(m)(x)
    assert oracle.rel_err(y, ref) <= LOGITS_TOL, oracle.rel_err(y, ref)


@torch.no_grad()
def test_resnet18_bs128_forward_vs_dequant_reference(gpu):
    """BASELINE cfg3 at its workload: ResNet-18, batch 128, 224x224, BN folded, 8-bit stem and fc, 2-bit 3x3,
    4-bit 1x1 downsample, fp16 channels-last activations (the kernels, grid sizes and tile choices of the timed
    forward: parts per image, tile rounds, the 8-bit fc's tile pick at M 128), against the dequantized fp32
    model on the CPU (quant/dimq_wrapper.py:189-197,237-240).  Checked over the whole batch, and the first
    images also per image, so that a wrong image offset cannot hide under the batch maximum."""
    from dimq_amd.bench_models import quantize_resnet18, resnet18
    announce("resnet18 forward 128x3x224x224")
    m = resnet18().cuda().to(memory_format=torch.channels_last)
    m = _cast_float_params(quantize_resnet18(m, out_dtype=torch.float16), torch.float16).eval()
    x = torch.randn(128, 3, 224, 224, generator=torch.Generator().manual_seed(2))
    y = m(x.cuda().half().contiguous(memory_format=torch.channels_last)).float().cpu()
    assert y.shape == (128, 1000)
    ref = oracle.dequantized_model(m)(x)
    err = oracle.rel_err(y, ref)
    print(f"resnet18 bs128 logits rel err {err:.3e}", flush=True)
    assert err <= LOGITS_TOL, err
    for i in (0, 63, 127):
        assert oracle.rel_err(y[i], ref[i]) <= 2 * LOGITS_TOL, (i, oracle.rel_err(y[i], ref[i]))


# ---------------------------------------------------------------- BASELINE cfg4 at its real shapes
@pytest.mark.parametrize("name,N,K,epi", [("qkv", 2304, 768, None), ("proj", 768, 768, "residual"),
                                          ("fc1", 3072, 768, "gelu"), ("fc2", 768, 3072, "residual")])
@pytest.mark.parametrize("out,xdt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float16), (torch.float16, torch.float16)])
@torch.no_grad()
def test_vit_linear_shapes_full_size(gpu, name, N, K, epi, out, xdt):
    """The four ViT-B/16 Linears at M = 64 x 197 = 12,608 tokens, bf16 or fp16 activations (the model's fp16
    links: LayerNorm -> qkv / fc1, fc1 -> fc2), 4-bit per-channel
    codebooks of N(0, 0.02) weights with the model's fused epilogue (GELU after fc1, the residual stream
    added after proj / fc2), against dequantize-then-F.linear in fp32 on the CPU (quant/dimq_wrapper.py:237-240,
    reference.py:91-110)."""
    from dimq_amd import ops
    from dimq_amd.codebook import init_centers_per_channel
    from dimq_amd.export import pack_indices
    announce(f"vit {name} M=12608 N={N} K={K} epi={epi} out={out} x={xdt}")
    g = torch.Generator().manual_seed(N + K)
    M = 64 * 197
    w = torch.randn(N, K, generator=g) * 0.02
    cb = init_centers_per_channel(w, 16)
    idx = ((w[:, :, None] - cb[:, None, :]) ** 2).argmin(dim=2).to(torch.uint8)
    packed = pack_indices(idx, 4)
    bias = torch.randn(N, generator=g) * 0.02
    x = torch.randn(M, K, generator=g).to(xdt)
    res = (torch.randn(M, N, generator=g) * 0.5).bfloat16() if epi == "residual" else None
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 4, bias.to(gpu), N, K, out_dtype=out,
                                 residual=None if res is None else res.to(gpu),
                                 activation="gelu" if epi == "gelu" else None)
    ref = oracle.linear_dequant_reference(x.float(), packed, 4, cb, N, K, bias)
    if epi == "residual":
        ref = ref + res.float()
    elif epi == "gelu":
        ref = torch.nn.functional.gelu(ref)
    tol = out_tol(out)
    err = oracle.rel_err(y.float().cpu(), ref)
    assert err <= tol, err


@torch.no_grad()
def test_vit_b16_bs64_forward_vs_dequant_reference(gpu):
    """BASELINE cfg4 end to end: ViT-B/16, batch 64, 224x224, all 48 qkv/proj/fc1/fc2 Linears 4-bit
    per-channel, bf16 on the GPU, against the dequantized fp32 model on the CPU."""
    from dimq_amd.bench_models import quantize_vit, vit_b16
    from dimq_amd.modules import DIMQCodebookLinear
    announce("vit_b16 bs64 forward")
    m = _cast_float_params(quantize_vit(vit_b16().to(gpu), 4, out_dtype=torch.bfloat16), torch.bfloat16).eval()
    assert sum(isinstance(x, DIMQCodebookLinear) for x in m.modules()) == 48
    x = torch.randn(64, 3, 224, 224, generator=torch.Generator().manual_seed(3))
    y = m(x.to(gpu).bfloat16()).float().cpu()
    ref = oracle.dequantized_model(m)(x)
    assert oracle.rel_err(y, ref) <= LOGITS_TOL, oracle.rel_err(y, ref)
