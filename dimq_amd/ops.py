"""Python entry points for the DIMQ operators (MI355X HIP backend).

Mirrors ``dimq_backend/ops.py`` (reference ``dimq_cuda_backend/dimq_backend/ops.py:12-125``):
same function names, arguments and errors, with ``is_available()`` testing that
the HIP library (``dimq_amd._C``) loads.  The generalised operators for
b-bit / per-channel / weight-only layers are added alongside.
"""

from __future__ import annotations

import importlib
from functools import lru_cache
from typing import Sequence

import torch


@lru_cache(maxsize=1)
def _extension_available() -> bool:
    try:
        importlib.import_module("dimq_amd._C")
    except Exception:
        return False
    return True


def is_available() -> bool:
    """Return whether the compiled HIP library is loadable (ops.py:21-24)."""

    return _extension_available()


def require_extension() -> None:
    if not is_available():
        raise RuntimeError(
            "dimq_amd HIP library is not available. "
            "Build it with `make -C dimq_amd/csrc` (or `python -c 'import __graft_entry__ as g; g.build()'`)."
        )


def pack_u4(indices: torch.Tensor) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.pack_u4(indices)


def unpack_u4(packed: torch.Tensor, numel: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.unpack_u4(packed, int(numel))


def quantize_activation_u4(x: torch.Tensor, act_scale: float, act_zero_point: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.quantize_activation_u4(x, float(act_scale), int(act_zero_point))


def build_product_table(codebook: torch.Tensor, act_scale: float, act_zero_point: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.build_product_table(codebook, float(act_scale), int(act_zero_point))


def dimq_linear_lut(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    codebook: torch.Tensor,
    act_scale: float,
    act_zero_point: int,
    bias: torch.Tensor | None,
    out_features: int,
    in_features: int,
) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.linear_lut(
        x, packed_weight, codebook, float(act_scale), int(act_zero_point), bias, int(out_features), int(in_features)
    )


def dimq_conv2d_lut(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    codebook: torch.Tensor,
    act_scale: float,
    act_zero_point: int,
    bias: torch.Tensor | None,
    weight_shape: Sequence[int],
    stride: Sequence[int],
    padding: Sequence[int],
    dilation: Sequence[int],
    groups: int,
) -> torch.Tensor:
    require_extension()
    out_channels, cin_per_group, kernel_h, kernel_w = [int(v) for v in weight_shape]
    stride_h, stride_w = _pair(stride)
    pad_h, pad_w = _pair(padding)
    dil_h, dil_w = _pair(dilation)
    return torch.ops.dimq.conv2d_lut(
        x, packed_weight, codebook, float(act_scale), int(act_zero_point), bias, out_channels, cin_per_group,
        kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, int(groups),
    )


# ---------------------------------------------------------------------------
# generalised operators (no reference counterpart: the reference is W4A4 only)
# ---------------------------------------------------------------------------

VARIANTS = {"auto": 0, "small_m": 1, "mfma": 2}
ACTIVATIONS = {None: 0, "none": 0, "relu": 1, "gelu": 2}


def pack_bits(indices: torch.Tensor, bits: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.pack_bits(indices, int(bits))


def unpack_bits(packed: torch.Tensor, numel: int, bits: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.unpack_bits(packed, int(numel), int(bits))


def hard_quantize(w: torch.Tensor, centers: torch.Tensor, per_channel: bool = False):
    """Nearest-centre (indices, values), quant/dimq.py:197-221 semantics."""
    require_extension()
    return torch.ops.dimq.hard_quantize(w, centers, bool(per_channel))


def build_product_table_grouped(codebook: torch.Tensor, act_scale: float, act_zero_point: int) -> torch.Tensor:
    require_extension()
    return torch.ops.dimq.build_product_table_grouped(codebook, float(act_scale), int(act_zero_point))


def dimq_linear_codebook(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    codebook: torch.Tensor,
    bits: int,
    bias: torch.Tensor | None,
    out_features: int,
    in_features: int,
    *,
    out_dtype: torch.dtype | None = None,
    variant: str = "auto",
    residual: torch.Tensor | None = None,
    activation: str | None = None,
    decoded: torch.Tensor | None = None,
) -> torch.Tensor:
    """y = act(x @ W_hat^T + bias + residual) with W_hat[n, k] = codebook[n or 0, idx[n, k]].

    ``residual`` (output shape) and ``activation`` ("relu" or "gelu", exact erf
    form) are fused into the kernel's store; without them this is the plain
    weight-only Linear.  ``decoded``: this layer's buffer from
    ``predecode_codebook_weights`` (same packed weights and codebook), used by
    the large-M path in place of its own per-call weight decode."""
    require_extension()
    return torch.ops.dimq.linear_codebook(
        x, packed_weight, codebook, int(bits), bias, int(out_features), int(in_features), out_dtype,
        VARIANTS[variant], residual, ACTIVATIONS[activation], decoded,
    )


def predecode_codebook_weights(layers):
    """Decodes the weights of several codebook Linears in one batch of launches.

    ``layers``: (packed_weight, codebook, bits, out_features, in_features)
    tuples on one GPU.  Returns (buffer, views): views[i] is layer i's decode
    (None when bits is 8 or in_features % 32 != 0), to pass as
    ``dimq_linear_codebook(..., decoded=views[i])`` while the packed weights
    and codebook stay unchanged.  No counterpart in the reference, whose LUT
    kernels decode inside every call."""
    require_extension()
    from . import _C
    return _C.predecode_codebook_weights_impl(layers)


def dimq_conv2d_codebook(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    codebook: torch.Tensor,
    bits: int,
    bias: torch.Tensor | None,
    weight_shape: Sequence[int],
    stride: Sequence[int],
    padding: Sequence[int],
    dilation: Sequence[int],
    groups: int,
    *,
    out_dtype: torch.dtype | None = None,
    variant: str = "auto",
    prepared_weight: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    activation: str | None = None,
) -> torch.Tensor:
    """Weight-only codebook conv2d; NCHW or channels_last input, output in the same memory format.

    ``prepared_weight`` (from :func:`prepare_conv_weight`) enables the LDS-halo
    and large-tile implicit-GEMM kernels for the shapes they support.
    ``residual`` (output shape) and ``activation`` ("relu" / "gelu") are fused
    into the kernel's store: y = act(conv + bias + residual)."""
    require_extension()
    out_channels, cin_per_group, kernel_h, kernel_w = [int(v) for v in weight_shape]
    stride_h, stride_w = _pair(stride)
    pad_h, pad_w = _pair(padding)
    dil_h, dil_w = _pair(dilation)
    return torch.ops.dimq.conv2d_codebook(
        x, packed_weight, codebook, int(bits), bias, out_channels, cin_per_group, kernel_h, kernel_w, stride_h,
        stride_w, pad_h, pad_w, dil_h, dil_w, int(groups), out_dtype, VARIANTS[variant], prepared_weight, residual,
        ACTIVATIONS[activation],
    )


def prepare_conv_weight(packed_weight: torch.Tensor, bits: int, weight_shape: Sequence[int]) -> torch.Tensor | None:
    """Kernel-layout copy of a conv_kcrs packed weight, or None when the shape has no kernel layout."""
    require_extension()
    from . import _C

    out_channels, cin, kernel_h, kernel_w = [int(v) for v in weight_shape]
    if _C.prepared_conv_words(out_channels, cin, kernel_h, kernel_w, int(bits)) <= 0:
        return None
    return torch.ops.dimq.prepare_conv_weight(packed_weight, int(bits), out_channels, cin, kernel_h, kernel_w)


def dimq_linear_codebook_act(x: torch.Tensor, packed_weight: torch.Tensor, codebook: torch.Tensor, bits: int,
                             act_centers: torch.Tensor, bias: torch.Tensor | None, out_features: int,
                             in_features: int, out_dtype: torch.dtype | None = None,
                             variant: str = "auto") -> torch.Tensor:
    """Weight x activation codebook Linear: x quantized to its nearest activation centre (the QAT wrapper's
    activation_centers, quant/dimq_wrapper.py:80-85), then the weight-codebook GEMM."""
    require_extension()
    return torch.ops.dimq.linear_codebook_act(x, packed_weight, codebook, int(bits), act_centers, bias,
                                              int(out_features), int(in_features), out_dtype, VARIANTS[variant])


def build_codebook_product_table(codebook: torch.Tensor, act_values: torch.Tensor) -> torch.Tensor:
    """[rows, Kw, Ka] fp32 table codebook[g][w] * act_values[a] (one rounding): the weight x activation codebook
    products a LUT GEMM gathers from.  act_values: the activation centres as the activations take them (in the
    activations' dtype)."""
    require_extension()
    from . import _C

    return _C.build_codebook_product_table_impl(codebook, act_values)


def dimq_linear_lut_act(act_idx: torch.Tensor, packed_weight: torch.Tensor, codebook: torch.Tensor, bits: int,
                        act_centers: torch.Tensor, x_dtype: torch.dtype, bias: torch.Tensor | None, out_features: int,
                        in_features: int, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Index x index LUT GEMM (M <= 16): y[m, n] = sum_k (C_w[n][w[n, k]] * C_a[a[m, k]]) + bias[n], act_idx the
    uint8 activation-centre indices, C_a rounded to x_dtype (the reference's centers[idx].to(x.dtype))."""
    require_extension()
    from . import _C

    return _C.linear_lut_act_impl(act_idx, packed_weight, codebook, int(bits), act_centers, x_dtype, bias,
                                  int(out_features), int(in_features), out_dtype)


def dimq_conv2d_codebook_act(x: torch.Tensor, packed_weight: torch.Tensor, codebook: torch.Tensor, bits: int,
                             act_centers: torch.Tensor, bias: torch.Tensor | None, weight_shape: Sequence[int],
                             stride=1, padding=0, dilation=1, groups: int = 1, *,
                             out_dtype: torch.dtype | None = None, prepared_weight: torch.Tensor | None = None,
                             variant: str = "auto") -> torch.Tensor:
    """Weight x activation codebook Conv2d: x quantized to its nearest activation centre (the QAT wrapper's
    activation_centers, quant/dimq_wrapper.py:80-85), then the weight-codebook conv."""
    require_extension()
    from . import _C

    oc, cin_g, kh, kw = [int(v) for v in weight_shape]
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    return _C.conv2d_codebook_act_impl(x, packed_weight, codebook, int(bits), act_centers, bias, oc, cin_g, kh, kw,
                                       sh, sw, ph, pw, dh, dw, int(groups), out_dtype, prepared_weight,
                                       VARIANTS[variant])


# ---------------------------------------------------------------------------
# Chained W4A4 layers.  Between layers the activations travel as the fp16
# integers a - zp (a = clamp(rint(x / s) + zp, 0, 15), the reference's u4 code,
# dimq_backend/reference.py:11-21), so a layer's epilogue can quantize its
# output for the next layer instead of the next layer re-reading a float tensor.
def quantize_activation_f16(x: torch.Tensor, act_scale: float, act_zp: int) -> torch.Tensor:
    """fp16 tensor of x's shape holding a - zp: the input form of linear_lut_q / conv2d_lut_q."""
    require_extension()
    from . import _C

    return _C.quantize_activation_f16_impl(x, act_scale, act_zp)


def dimq_linear_lut_q(xq: torch.Tensor, packed_weight: torch.Tensor, codebook: torch.Tensor, act_scale: float,
                      bias: torch.Tensor | None, out_features: int, in_features: int, *,
                      activation: str | None = None, out_act: tuple[float, int] | None = None,
                      out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """linear_lut on pre-quantized activations: y = act(s * sum_k C[w] (a - zp) + bias), xq = a - zp (fp16),
    s = act_scale.  With out_act = (s', zp') the result is returned as the next layer's codes (fp16 q' - zp');
    otherwise as out_dtype (default fp32).  codebook: the 16-entry fp16 codebook of the packed export."""
    require_extension()
    from . import _C

    return _C.linear_lut_q_impl(xq, packed_weight, codebook, act_scale, bias, int(out_features), int(in_features),
                                ACTIVATIONS[activation], out_act, out_dtype)


def dimq_conv2d_lut_q(xq: torch.Tensor, packed_weight: torch.Tensor, codebook: torch.Tensor, act_scale: float,
                      bias: torch.Tensor | None, weight_shape: Sequence[int], stride=1, padding=0, dilation=1,
                      groups: int = 1, *, prepared_weight: torch.Tensor | None = None,
                      activation: str | None = None, out_act: tuple[float, int] | None = None,
                      out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """conv2d_lut on pre-quantized NCHW activations (xq = a - zp, fp16); output NCHW.  prepared_weight: the 4-bit
    kernel layout of prepare_conv_weight (optional).  activation / out_act / out_dtype as dimq_linear_lut_q."""
    require_extension()
    from . import _C

    oc, cin_g, kh, kw = [int(v) for v in weight_shape]
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    return _C.conv2d_lut_q_impl(xq, packed_weight, codebook, act_scale, bias, oc, cin_g, kh, kw, sh, sw, ph, pw, dh,
                                dw, int(groups), prepared_weight, ACTIVATIONS[activation], out_act, out_dtype)


def layer_norm(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
               eps: float = 1e-5, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """LayerNorm over the last dimension on the HIP kernel (fp16/bf16 x; the ViT workload's LayerNorms); the
    output in out_dtype (fp16 / bf16, default x's dtype)."""
    require_extension()
    return torch.ops.dimq.layer_norm(x, int(x.shape[-1]), weight, bias, float(eps), out_dtype)


def max_pool2d_nhwc(x: torch.Tensor, kernel_size, stride=None, padding=0) -> torch.Tensor:
    """2-D max pooling of a channels-last fp16/bf16 tensor on the HIP kernel (the ResNet workload's stem pool)."""
    require_extension()
    kh, kw = _pair(kernel_size)
    sh, sw = _pair(stride if stride is not None else kernel_size)
    ph, pw = _pair(padding)
    return torch.ops.dimq.max_pool2d_nhwc(x, kh, kw, sh, sw, ph, pw)


def _pair(value: Sequence[int] | int) -> tuple[int, int]:
    if isinstance(value, int):
        return int(value), int(value)
    if len(value) != 2:
        raise ValueError(f"expected pair, got {value!r}")
    return int(value[0]), int(value[1])
