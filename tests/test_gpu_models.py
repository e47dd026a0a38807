"""End-to-end forwards of the two BASELINE models through the codebook layers,
against the dequantize-then-float CPU model (oracle.dequantized_model).

Activations run in bf16 (ViT) / fp16 (ResNet) on the GPU and in fp32 on the
CPU, so the bound is looser than the single-layer 2e-3: max|err|/max|ref| of
the logits <= 3e-2."""

from __future__ import annotations

import pytest
import torch

import oracle
from tests.conftest import announce

pytestmark = pytest.mark.gpu


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
    assert oracle.rel_err(y, ref) <= 3e-2


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
    assert oracle.rel_err(y, ref) <= 3e-2
