"""Runtime layers backed by packed codebook indices (HIP backend).

``DIMQLinear`` / ``DIMQConv2d`` keep the constructor, buffers and
``from_export_layer`` of the reference (``dimq_backend/modules.py:14-150``) and
run the W4A4 LUT ops.  ``DIMQCodebookLinear`` / ``DIMQCodebookConv2d`` are the
weight-only layers of the BASELINE configurations: b-bit indices, per-layer or
per-output-channel codebooks, y = F.linear / F.conv2d(x, W_hat, bias)
(``quant/dimq_wrapper.py:189-197,237-240``).

Difference from the reference: there is no CPU fallback.  The reference's
``forward`` runs its Python reference when the input is on the CPU
(``modules.py:40,51``); here ``forward`` requires GPU tensors and a loadable
HIP library and raises otherwise, so a missing or broken backend never goes
unnoticed.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Iterator, Mapping

import torch
import torch.nn as nn

from . import ops
from .codebook import assign_indices, init_centers_1d, init_centers_per_channel
from .export import bits_for_codebook, pack_indices


def _require_gpu(x: torch.Tensor, buf: torch.Tensor, use_kernel: bool, name: str) -> None:
    if not use_kernel:
        raise RuntimeError(f"{name}: use_cuda_kernel=False is not supported; this backend has no CPU path")
    if not (x.is_cuda and buf.is_cuda):
        raise RuntimeError(f"{name} runs on the GPU: move the module and its input to a HIP device")
    ops.require_extension()


class DIMQLinear(nn.Module):
    """Linear layer backed by packed u4 weight indices, a 16-entry codebook and A4 activations."""

    def __init__(self, packed_weight, codebook, act_scale, act_zero_point, out_features, in_features, bias=None, *,
                 use_cuda_kernel: bool = True) -> None:
        super().__init__()
        self.register_buffer("packed_weight", packed_weight.contiguous().to(torch.uint8))
        self.register_buffer("codebook", codebook.contiguous())
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        self.act_scale = float(act_scale)
        self.act_zero_point = int(act_zero_point)
        self.out_features = int(out_features)
        self.in_features = int(in_features)
        self.use_cuda_kernel = bool(use_cuda_kernel)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require_gpu(x, self.packed_weight, self.use_cuda_kernel, "DIMQLinear")
        return ops.dimq_linear_lut(x, self.packed_weight, self.codebook, self.act_scale, self.act_zero_point,
                                   self.bias, self.out_features, self.in_features)

    @classmethod
    def from_export_layer(cls, layer: Mapping[str, Any], *, use_cuda_kernel: bool = True) -> "DIMQLinear":
        return cls(layer["packed_weight"], layer["codebook"], layer["act_scale"], layer["act_zero_point"],
                   layer["out_features"], layer["in_features"], layer.get("bias"), use_cuda_kernel=use_cuda_kernel)


class DIMQConv2d(nn.Module):
    """Conv2d layer backed by packed u4 weight indices, a 16-entry codebook and A4 activations."""

    def __init__(self, packed_weight, codebook, act_scale, act_zero_point, weight_shape, bias=None, *, stride=1,
                 padding=0, dilation=1, groups=1, use_cuda_kernel: bool = True) -> None:
        super().__init__()
        self.register_buffer("packed_weight", packed_weight.contiguous().to(torch.uint8))
        self.register_buffer("codebook", codebook.contiguous())
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        self.act_scale = float(act_scale)
        self.act_zero_point = int(act_zero_point)
        self.weight_shape = tuple(int(v) for v in weight_shape)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = int(groups)
        self.use_cuda_kernel = bool(use_cuda_kernel)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _require_gpu(x, self.packed_weight, self.use_cuda_kernel, "DIMQConv2d")
        return ops.dimq_conv2d_lut(x, self.packed_weight, self.codebook, self.act_scale, self.act_zero_point,
                                   self.bias, self.weight_shape, self.stride, self.padding, self.dilation, self.groups)

    @classmethod
    def from_export_layer(cls, layer: Mapping[str, Any], *, use_cuda_kernel: bool = True) -> "DIMQConv2d":
        return cls(layer["packed_weight"], layer["codebook"], layer["act_scale"], layer["act_zero_point"],
                   layer["weight_shape"], layer.get("bias"), stride=layer.get("stride", (1, 1)),
                   padding=layer.get("padding", (0, 0)), dilation=layer.get("dilation", (1, 1)),
                   groups=layer.get("groups", 1), use_cuda_kernel=use_cuda_kernel)


class DIMQCodebookLinear(nn.Module):
    """Weight-only Linear: y = x @ W_hat^T + b, W_hat[n, k] = codebook[n or 0, idx[n, k]] (b-bit idx)."""

    def __init__(self, packed_weight, codebook, bits, out_features, in_features, bias=None, *,
                 out_dtype: torch.dtype | None = None, variant: str = "auto",
                 activation_centers: torch.Tensor | None = None) -> None:
        super().__init__()
        self.register_buffer("packed_weight", packed_weight.contiguous().to(torch.uint8))
        self.register_buffer("codebook", codebook.contiguous())
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        # the QAT wrapper's activation codebook (quant/dimq_wrapper.py:80-85): when set, activations are
        # quantized to their nearest centre before the weight-codebook product
        self.register_buffer("activation_centers",
                             None if activation_centers is None else activation_centers.detach().float().reshape(-1))
        self.bits = int(bits)
        self.out_features = int(out_features)
        self.in_features = int(in_features)
        self.out_dtype = out_dtype
        self.variant = variant
        self._decoded: torch.Tensor | None = None  # set by decoded_weights() for the span of one forward

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None,
                activation: str | None = None) -> torch.Tensor:
        """act(linear(x) + residual); residual and activation ("relu", "gelu") are fused into the kernel."""
        _require_gpu(x, self.packed_weight, True, "DIMQCodebookLinear")
        if self.activation_centers is not None:
            if residual is not None or activation is not None:
                raise RuntimeError("activation-codebook layers take no fused residual / activation")
            return ops.dimq_linear_codebook_act(x, self.packed_weight, self.codebook, self.bits,
                                                self.activation_centers, self.bias, self.out_features,
                                                self.in_features, out_dtype=self.out_dtype, variant=self.variant)
        return ops.dimq_linear_codebook(x, self.packed_weight, self.codebook, self.bits, self.bias,
                                        self.out_features, self.in_features, out_dtype=self.out_dtype,
                                        variant=self.variant, residual=residual, activation=activation,
                                        decoded=self._decoded)

    @classmethod
    @torch.no_grad()
    def from_linear(cls, linear: nn.Linear, bits: int, *, per_channel: bool = True, codebook_dtype=torch.float32,
                    out_dtype: torch.dtype | None = None) -> "DIMQCodebookLinear":
        """Quantile-initialised codebook, nearest-centre indices (GPU), packed (GPU)."""
        w = linear.weight.detach().float()
        K = 1 << int(bits)
        centers = init_centers_per_channel(w, K) if per_channel else init_centers_1d(w, K)
        idx = assign_indices(w, centers)
        packed = pack_indices(idx, bits)
        dev = linear.weight.device
        bias = None if linear.bias is None else linear.bias.detach()
        return cls(packed.to(dev), centers.to(device=dev, dtype=codebook_dtype), bits, linear.out_features,
                   linear.in_features, bias, out_dtype=out_dtype)

    @classmethod
    def from_export_layer(cls, layer: Mapping[str, Any]) -> "DIMQCodebookLinear":
        return cls(layer["packed_weight"], layer["codebook"], layer["bit_w"], layer["out_features"],
                   layer["in_features"], layer.get("bias"), activation_centers=layer.get("activation_centers"))


class DIMQCodebookConv2d(nn.Module):
    """Weight-only Conv2d with b-bit codebook indices (conv_kcrs layout)."""

    def __init__(self, packed_weight, codebook, bits, weight_shape, bias=None, *, stride=1, padding=0, dilation=1,
                 groups=1, out_dtype: torch.dtype | None = None, variant: str = "auto",
                 activation_centers: torch.Tensor | None = None) -> None:
        super().__init__()
        self.register_buffer("packed_weight", packed_weight.contiguous().to(torch.uint8))
        self.register_buffer("codebook", codebook.contiguous())
        self.register_buffer("bias", None if bias is None else bias.contiguous())
        self.register_buffer("activation_centers",
                             None if activation_centers is None else activation_centers.detach().float().reshape(-1))
        self.bits = int(bits)
        self.weight_shape = tuple(int(v) for v in weight_shape)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = int(groups)
        self.out_dtype = out_dtype
        self.variant = variant
        self._prepared = None      # kernel-layout weight, built once on the GPU
        self._prepared_key = None

    def prepared_weight(self) -> torch.Tensor | None:
        """Kernel-layout copies of packed_weight (LDS-halo and tap-major layouts), built on first use and
        rebuilt whenever packed_weight is replaced, moved or written in place (its version counter)."""
        if self.groups != 1:
            return None
        w = self.packed_weight
        key = (w.data_ptr(), w.device, w._version)
        if self._prepared_key != key:
            self._prepared = ops.prepare_conv_weight(w, self.bits, self.weight_shape)
            self._prepared_key = key
        return self._prepared

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self._prepared, self._prepared_key = None, None  # the loaded weights may reuse the buffer's storage

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None,
                activation: str | None = None) -> torch.Tensor:
        """act(conv(x) + residual); residual and activation ("relu", "gelu") are fused into the kernel."""
        _require_gpu(x, self.packed_weight, True, "DIMQCodebookConv2d")
        if self.activation_centers is not None:
            if residual is not None or activation is not None:
                raise RuntimeError("activation-codebook layers take no fused residual / activation")
            return ops.dimq_conv2d_codebook_act(x, self.packed_weight, self.codebook, self.bits,
                                                self.activation_centers, self.bias, self.weight_shape, self.stride,
                                                self.padding, self.dilation, self.groups, out_dtype=self.out_dtype,
                                                prepared_weight=self.prepared_weight(), variant=self.variant)
        return ops.dimq_conv2d_codebook(x, self.packed_weight, self.codebook, self.bits, self.bias,
                                        self.weight_shape, self.stride, self.padding, self.dilation, self.groups,
                                        out_dtype=self.out_dtype, variant=self.variant,
                                        prepared_weight=self.prepared_weight(), residual=residual,
                                        activation=activation)

    @classmethod
    @torch.no_grad()
    def from_conv(cls, conv: nn.Conv2d, bits: int, *, per_channel: bool = True, codebook_dtype=torch.float32,
                  out_dtype: torch.dtype | None = None) -> "DIMQCodebookConv2d":
        if conv.padding_mode != "zeros":
            raise ValueError("only zero padding is supported")
        w = conv.weight.detach().float()
        K = 1 << int(bits)
        centers = init_centers_per_channel(w, K) if per_channel else init_centers_1d(w, K)
        idx = assign_indices(w, centers)
        packed = pack_indices(idx, bits)
        dev = conv.weight.device
        bias = None if conv.bias is None else conv.bias.detach()
        return cls(packed.to(dev), centers.to(device=dev, dtype=codebook_dtype), bits, tuple(w.shape), bias,
                   stride=conv.stride, padding=conv.padding, dilation=conv.dilation, groups=conv.groups,
                   out_dtype=out_dtype)

    @classmethod
    def from_export_layer(cls, layer: Mapping[str, Any]) -> "DIMQCodebookConv2d":
        return cls(layer["packed_weight"], layer["codebook"], layer["bit_w"], layer["weight_shape"], layer.get("bias"),
                   stride=layer.get("stride", (1, 1)), padding=layer.get("padding", (0, 0)),
                   dilation=layer.get("dilation", (1, 1)), groups=layer.get("groups", 1),
                   activation_centers=layer.get("activation_centers"))


class DIMQLayerNorm(nn.LayerNorm):
    """nn.LayerNorm whose forward runs the HIP LayerNorm kernel (fp16/bf16 CUDA
    inputs, normalized over the last dimension).  Same parameters and state
    dict as nn.LayerNorm; other inputs raise: the CPU reference model converts
    it back to nn.LayerNorm (torch's own op)."""

    out_dtype: torch.dtype | None = None  # the output's dtype (fp16 / bf16); None: the input's

    @classmethod
    def from_layer_norm(cls, ln: nn.LayerNorm, out_dtype: torch.dtype | None = None) -> "DIMQLayerNorm":
        if len(ln.normalized_shape) != 1:
            raise ValueError("DIMQLayerNorm normalizes over the last dimension only")
        new = cls(ln.normalized_shape[0], eps=ln.eps, elementwise_affine=ln.elementwise_affine,
                  bias=ln.bias is not None, device=ln.weight.device if ln.weight is not None else None,
                  dtype=ln.weight.dtype if ln.weight is not None else None)
        new.out_dtype = out_dtype
        if ln.weight is not None:
            new.weight.data.copy_(ln.weight.data)
        if ln.bias is not None:
            new.bias.data.copy_(ln.bias.data)
        return new

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("DIMQLayerNorm runs on CUDA (HIP) tensors only")
        return ops.layer_norm(x, self.weight, self.bias, self.eps, self.out_dtype)


class DIMQMaxPool2d(nn.MaxPool2d):
    """nn.MaxPool2d whose forward runs the HIP max-pool kernel (channels-last
    fp16/bf16 CUDA inputs, dilation 1, floor mode).  Other inputs raise: the
    CPU reference model converts it back to nn.MaxPool2d (torch's own op)."""

    @classmethod
    def from_max_pool(cls, mp: nn.MaxPool2d) -> "DIMQMaxPool2d":
        if mp.dilation not in (1, (1, 1)) or mp.ceil_mode or mp.return_indices:
            raise ValueError("DIMQMaxPool2d supports dilation 1, floor mode and no indices")
        return cls(mp.kernel_size, mp.stride, mp.padding)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("DIMQMaxPool2d runs on CUDA (HIP) tensors only")
        return ops.max_pool2d_nhwc(x, self.kernel_size, self.stride, self.padding)


def make_packed_layer(layer: Mapping[str, Any], *, use_cuda_kernel: bool = True) -> nn.Module:
    """modules.py:153-158, extended with weight-only (format v2) layers."""
    weight_only = (layer.get("activation_quantization") in ("none", "codebook") or layer.get("bit_a", 4) is None
                   or "activation_centers" in layer)
    if layer["type"] == "linear":
        if weight_only:
            return DIMQCodebookLinear.from_export_layer(layer)
        return DIMQLinear.from_export_layer(layer, use_cuda_kernel=use_cuda_kernel)
    if layer["type"] == "conv2d":
        if weight_only:
            return DIMQCodebookConv2d.from_export_layer(layer)
        return DIMQConv2d.from_export_layer(layer, use_cuda_kernel=use_cuda_kernel)
    raise ValueError(f"unsupported packed DIMQ layer type {layer['type']!r}")


def replace_modules_with_packed_dimq(model: nn.Module, packed_state: Mapping[str, Any], *,
                                     use_cuda_kernel: bool = True) -> nn.Module:
    """Replace matching modules with packed DIMQ runtime layers (modules.py:161-172)."""
    for name, layer in packed_state["layers"].items():
        parent, leaf = _resolve_parent(model, name)
        parent._modules[leaf] = make_packed_layer(layer, use_cuda_kernel=use_cuda_kernel)
    return model


def quantize_model_weight_only(model: nn.Module, bits_for: Any, *, per_channel: bool = True,
                               codebook_dtype=torch.float32, out_dtype: torch.dtype | None = None) -> nn.Module:
    """Replace every Conv2d/Linear with its weight-only codebook layer.

    ``bits_for(name, module) -> int | None`` picks the index width per layer
    (None keeps the float layer)."""
    for name, module in list(model.named_modules()):
        if isinstance(module, (nn.Conv2d, nn.Linear)):
            bits = bits_for(name, module)
            if bits is None:
                continue
            parent, leaf = _resolve_parent(model, name) if name else (None, None)
            if isinstance(module, nn.Conv2d):
                new = DIMQCodebookConv2d.from_conv(module, bits, per_channel=per_channel,
                                                   codebook_dtype=codebook_dtype, out_dtype=out_dtype)
            else:
                new = DIMQCodebookLinear.from_linear(module, bits, per_channel=per_channel,
                                                     codebook_dtype=codebook_dtype, out_dtype=out_dtype)
            parent._modules[leaf] = new
    return model


@contextmanager
def decoded_weights(model: nn.Module, rows: int) -> Iterator[None]:
    """For the span of the ``with`` block, the model's weight-only codebook
    Linears run on weights decoded by one batch of launches at entry
    (``ops.predecode_codebook_weights``) instead of decoding them in every
    call: same kernels, same results, fewer launches.  ``rows`` is the number
    of activation rows the Linears will see (batch x tokens); layers whose
    calls at that size do not take the large-M path (where the per-call
    decode happens) are left alone, so small batches decode nothing extra.
    The decode runs at entry on the current stream, so the packed weights and
    codebooks must not change inside the block; nested use is not supported.
    Scope it to what the next few calls read: the GEMMs then find the decoded
    weights still in the GPU's caches.  Measured on ViT-B/16 bs64 (graph
    replay, same process): one batch per encoder block 4.24 ms per forward,
    the per-call decode 4.33 ms, one batch for all 48 Linears 4.41 ms (170 MB
    of decoded weights, mostly evicted before use).
    No counterpart in the reference, whose LUT kernels decode inside every
    call (dimq_cuda_backend/csrc/dimq_gemm_lut.cu)."""
    cands = [m for m in model.modules() if isinstance(m, DIMQCodebookLinear) and m.activation_centers is None
             and m.packed_weight.is_cuda and m._decoded is None]
    layers = []
    if cands:
        from . import _C
        for mod in cands:
            wbytes = _C.lib.dimq_codebook_predecode_bytes(mod.out_features, mod.in_features, mod.bits)
            # the large-M path of an fp16 call needs exactly the decoded weights as its workspace
            if wbytes > 0 and _C.lib.dimq_linear_codebook_workspace_bytes(
                    int(rows), mod.in_features, mod.out_features, mod.bits, _C.F16) == wbytes:
                layers.append(mod)
    try:
        if layers:
            _, views = ops.predecode_codebook_weights(
                [(m.packed_weight, m.codebook, m.bits, m.out_features, m.in_features) for m in layers])
            for mod, v in zip(layers, views):
                mod._decoded = v
        yield
    finally:
        for mod in layers:
            mod._decoded = None


def _resolve_parent(model: nn.Module, layer_name: str):
    parts = layer_name.split(".")
    parent = model
    for part in parts[:-1]:
        parent = parent._modules[part]
    return parent, parts[-1]


def _pair(value):
    if isinstance(value, int):
        return int(value), int(value)
    if len(value) != 2:
        raise ValueError(f"expected pair, got {value!r}")
    return int(value[0]), int(value[1])


__all__ = ["DIMQLinear", "DIMQConv2d", "DIMQCodebookLinear", "DIMQCodebookConv2d", "make_packed_layer",
           "replace_modules_with_packed_dimq", "quantize_model_weight_only", "bits_for_codebook"]
