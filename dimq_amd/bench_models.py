"""Plain-torch models of the two end-to-end BASELINE workloads.

* ``vit_b16``: ViT-B/16 as torchvision's ``vit_b_16`` (the architecture of the
  reference's ``train_dimq_vit.py``): 16x16 patch embedding, class token,
  learned position embedding, 12 pre-norm encoder blocks (LayerNorm eps 1e-6,
  fused qkv projection, 12 heads, MLP 3072 with exact GELU), final LayerNorm,
  1000-class head.  ``quantize_vit`` replaces every qkv / proj / fc1 / fc2
  Linear with a weight-only codebook layer (BASELINE cfg4: 4-bit,
  per-output-channel); patch embedding, LayerNorm, softmax, attention and head
  stay unquantized.
* ``resnet18``: torchvision's ``resnet18`` layout (the reference's
  ``export_resnet18_dimq.py`` model) with BatchNorm folded into the
  convolutions.  ``quantize_resnet18`` replaces every conv and the fc layer
  (BASELINE cfg3: 8-bit stem and fc, 2-bit 3x3 convs, 4-bit 1x1 downsample).

torchvision is not installed here, so the layers are written out.  Weights are
random (seeded), as in the BASELINE configurations.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .modules import (DIMQCodebookConv2d, DIMQCodebookLinear, DIMQLayerNorm, DIMQMaxPool2d, decoded_weights,
                      quantize_model_weight_only)


def _fused(mod: nn.Module, x: torch.Tensor, residual: torch.Tensor | None = None,
           act: str | None = None) -> torch.Tensor:
    """act(mod(x) + residual): fused into the kernel's store for codebook layers, torch ops otherwise."""
    if isinstance(mod, (DIMQCodebookConv2d, DIMQCodebookLinear)):
        return mod(x, residual=residual, activation=act)
    y = mod(x)
    if residual is not None:
        y = y + residual
    if act == "relu":
        y = F.relu(y)
    elif act == "gelu":
        y = F.gelu(y)
    return y


# ---------------------------------------------------------------------------
# ViT-B/16
# ---------------------------------------------------------------------------

class _Attention(nn.Module):
    def __init__(self, dim: int, heads: int) -> None:
        super().__init__()
        self.heads = heads
        self.qkv = nn.Linear(dim, 3 * dim)
        self.proj = nn.Linear(dim, dim)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        b, n, d = x.shape
        h = self.heads
        # q, k, v stay strided views of the qkv output (head dim contiguous): the
        # attention kernel takes them as they are and returns o in (b, n, h, d)
        # memory order, so neither side needs a copy
        qkv = self.qkv(x).view(b, n, 3, h, d // h)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        o = F.scaled_dot_product_attention(q, k, v)
        return _fused(self.proj, o.transpose(1, 2).reshape(b, n, d), residual=residual)


class _Block(nn.Module):
    def __init__(self, dim: int, heads: int, mlp: int) -> None:
        super().__init__()
        self.ln_1 = nn.LayerNorm(dim, eps=1e-6)
        self.attn = _Attention(dim, heads)
        self.ln_2 = nn.LayerNorm(dim, eps=1e-6)
        self.fc1 = nn.Linear(dim, mlp)
        self.fc2 = nn.Linear(mlp, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # x + attn(ln_1(x)), then x + fc2(gelu(fc1(ln_2(x)))); the residual adds and
        # the GELU run in the projections' epilogues
        x = self.attn(self.ln_1(x), residual=x)
        return _fused(self.fc2, _fused(self.fc1, self.ln_2(x), act="gelu"), residual=x)


class ViT(nn.Module):
    def __init__(self, image: int = 224, patch: int = 16, dim: int = 768, depth: int = 12, heads: int = 12,
                 mlp: int = 3072, classes: int = 1000) -> None:
        super().__init__()
        self.patch = patch
        self.conv_proj = nn.Conv2d(3, dim, patch, stride=patch)
        self.class_token = nn.Parameter(torch.zeros(1, 1, dim))
        n = (image // patch) ** 2 + 1
        self.pos_embedding = nn.Parameter(torch.empty(1, n, dim).normal_(std=0.02))
        self.blocks = nn.ModuleList(_Block(dim, heads, mlp) for _ in range(depth))
        self.ln = nn.LayerNorm(dim, eps=1e-6)
        self.head = nn.Linear(dim, classes)

    def embed(self, x: torch.Tensor) -> torch.Tensor:
        """Patch embedding: a stride-16 16x16 conv is a GEMM over the unfolded patches."""
        b, c, h, w = x.shape
        p = self.patch
        patches = x.reshape(b, c, h // p, p, w // p, p).permute(0, 2, 4, 1, 3, 5).reshape(b, (h // p) * (w // p), -1)
        return F.linear(patches, self.conv_proj.weight.reshape(self.conv_proj.out_channels, -1), self.conv_proj.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.embed(x)
        x = torch.cat([self.class_token.expand(x.shape[0], -1, -1), x], dim=1) + self.pos_embedding
        # each block's codebook Linears decode their weights in one launch at the block's start (one
        # batch for the whole forward left the decoded weights cold by the time the later blocks read them)
        for blk in self.blocks:
            with decoded_weights(blk, x.shape[0] * x.shape[1]):
                x = blk(x)
        return self.head(self.ln(x[:, 0]))


def vit_b16(seed: int = 3) -> ViT:
    """ViT-B/16 with BASELINE cfg4's initialisation: Linear weights N(0, 0.02), zero biases."""
    g = torch.Generator().manual_seed(seed)
    m = ViT()
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, nn.Linear):
                mod.weight.copy_(torch.randn(mod.weight.shape, generator=g) * 0.02)
                mod.bias.zero_()
            elif isinstance(mod, nn.Conv2d):
                fan_in = mod.weight[0].numel()
                mod.weight.copy_(torch.randn(mod.weight.shape, generator=g) * math.sqrt(1.0 / fan_in))
                mod.bias.zero_()
        m.pos_embedding.copy_(torch.randn(m.pos_embedding.shape, generator=g) * 0.02)
    return m


def quantize_vit(model: ViT, bits: int = 4, out_dtype: torch.dtype = torch.bfloat16, fp16_links: bool = True) -> ViT:
    """cfg4: qkv / proj / fc1 / fc2 -> weight-only codebook layers (per-output-channel codebooks);
    the LayerNorms -> DIMQLayerNorm (the HIP LayerNorm kernel, same parameters).

    fp16_links: the tensors that only feed a codebook GEMM -- ln_1 -> qkv, ln_2 -> fc1 and fc1 (GELU) -> fc2 --
    and the qkv output, so attention runs in fp16 and hands proj fp16, are written in fp16 instead of bf16 (one
    rounding of the same fp32 result, with three more mantissa bits), so those GEMMs stage their activations
    without a bf16 -> fp16 conversion; the residual stream and the head stay bf16.  The qkv / attention link
    measured 4.26-4.34 -> 4.10-4.14 ms per bs64 forward, logits' max|err|/max|ref| against the fp32 model
    1.00e-2 -> 0.92e-2."""
    def pick(name, module):
        leaf = name.rsplit(".", 1)[-1]
        return bits if leaf in ("qkv", "proj", "fc1", "fc2") else None
    model = quantize_model_weight_only(model, pick, out_dtype=out_dtype)
    for name, mod in list(model.named_modules()):
        if type(mod) is nn.LayerNorm:
            parent = model
            parts = name.split(".")
            for part in parts[:-1]:
                parent = parent._modules[part]
            link = fp16_links and parts[-1] in ("ln_1", "ln_2")
            parent._modules[parts[-1]] = DIMQLayerNorm.from_layer_norm(mod, torch.float16 if link else None)
    if fp16_links:
        for blk in model.blocks:
            blk.fc1.out_dtype = torch.float16
            blk.attn.qkv.out_dtype = torch.float16
    return model


def vit_flops(batch: int, model: ViT | None = None) -> float:
    """Multiply-adds x 2 of one forward (patch embedding, Linears, attention)."""
    d, n, mlp, depth, p = 768, 197, 3072, 12, 16
    per_layer = 2 * n * (d * 3 * d + d * d + 2 * d * mlp) + 2 * 2 * n * n * d
    embed = 2 * 196 * d * 3 * p * p
    return float(batch * (depth * per_layer + embed + 2 * d * 1000))


# ---------------------------------------------------------------------------
# ResNet-18 (BatchNorm folded)
# ---------------------------------------------------------------------------

class _BasicBlock(nn.Module):
    def __init__(self, cin: int, cout: int, stride: int) -> None:
        super().__init__()
        self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1)
        self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1)
        self.downsample = nn.Conv2d(cin, cout, 1, stride) if (stride != 1 or cin != cout) else None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # relu(conv2(relu(conv1(x))) + identity), ReLUs and the residual add in the conv epilogues
        out = _fused(self.conv1, x, act="relu")
        idn = x if self.downsample is None else self.downsample(x)
        return _fused(self.conv2, out, residual=idn, act="relu")


class ResNet18(nn.Module):
    def __init__(self, classes: int = 1000) -> None:
        super().__init__()
        self.conv1 = nn.Conv2d(3, 64, 7, 2, 3)
        self.maxpool = nn.MaxPool2d(3, 2, 1)
        layers = []
        cin = 64
        for i, cout in enumerate((64, 128, 256, 512)):
            stride = 1 if i == 0 else 2
            layers.append(nn.Sequential(_BasicBlock(cin, cout, stride), _BasicBlock(cout, cout, 1)))
            cin = cout
        self.layer1, self.layer2, self.layer3, self.layer4 = layers
        self.fc = nn.Linear(512, classes)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = _fused(self.conv1, x, act="relu")
        x = self.maxpool(x)
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        x = torch.flatten(F.adaptive_avg_pool2d(x, 1), 1)
        return self.fc(x)


def resnet18(seed: int = 2) -> ResNet18:
    """ResNet-18 with Kaiming-normal convs and seeded non-trivial BatchNorm statistics folded in."""
    g = torch.Generator().manual_seed(seed)
    m = ResNet18()
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, nn.Conv2d):
                fan_out = mod.out_channels * mod.kernel_size[0] * mod.kernel_size[1]
                w = torch.randn(mod.weight.shape, generator=g) * math.sqrt(2.0 / fan_out)
                c = mod.out_channels
                gamma = 1.0 + 0.1 * torch.randn(c, generator=g)
                beta = 0.1 * torch.randn(c, generator=g)
                mean = 0.1 * torch.randn(c, generator=g)
                var = 1.0 + 0.1 * torch.rand(c, generator=g)
                s = gamma / torch.sqrt(var + 1e-5)
                mod.weight.copy_(w * s[:, None, None, None])
                mod.bias.copy_(beta - mean * s)
            elif isinstance(mod, nn.Linear):
                bound = 1.0 / math.sqrt(mod.in_features)
                mod.weight.copy_((torch.rand(mod.weight.shape, generator=g) * 2 - 1) * bound)
                mod.bias.copy_((torch.rand(mod.bias.shape, generator=g) * 2 - 1) * bound)
    return m


def quantize_resnet18(model: ResNet18, out_dtype: torch.dtype = torch.float16) -> ResNet18:
    """cfg3: 8-bit stem and fc, 2-bit 3x3 convs, 4-bit 1x1 downsample convs; the stem pool -> DIMQMaxPool2d."""
    def pick(name, module):
        if isinstance(module, nn.Linear) or name == "conv1":
            return 8
        return 2 if module.kernel_size == (3, 3) else 4
    model = quantize_model_weight_only(model, pick, out_dtype=out_dtype)
    model.maxpool = DIMQMaxPool2d.from_max_pool(model.maxpool)  # the HIP max-pool kernel
    return model


def resnet18_flops(batch: int) -> float:
    """Multiply-adds x 2 of one forward of the convolutions and the fc layer (224x224 input)."""
    m = ResNet18()
    macs = []

    def hook(mod, inp, out):
        if isinstance(mod, nn.Conv2d):
            macs.append(out.numel() * mod.in_channels // mod.groups * mod.kernel_size[0] * mod.kernel_size[1])
        else:
            macs.append(out.numel() * mod.in_features)
    hooks = [mod.register_forward_hook(hook) for mod in m.modules() if isinstance(mod, (nn.Conv2d, nn.Linear))]
    with torch.no_grad():
        m(torch.zeros(1, 3, 224, 224))
    for hk in hooks:
        hk.remove()
    return float(2 * batch * sum(macs))
