"""Loads ``libdimq_hip.so`` (the gfx950 C-ABI library) and registers the ops.

Importing this module is what ``ops.is_available()`` tests, exactly as the
reference's ``dimq_backend/ops.py:12-18`` tests ``import dimq_backend._C``.
The import fails loudly (OSError / RuntimeError) when the library is missing;
nothing here falls back to a CPU implementation.

Ops registered in the ``dimq`` namespace on the CUDA dispatch key (HIP tensors
use it in ROCm PyTorch):

* the reference's six schemas, verbatim (``dimq_cuda_backend/csrc/dimq_ops.cpp:38-43``);
* generalised ops for b in {2,3,4,8}, per-channel codebooks and weight-only
  GEMM/conv (``pack_bits``, ``unpack_bits``, ``hard_quantize``,
  ``build_product_table_grouped``, ``linear_codebook``, ``conv2d_codebook``).

Each op validates its tensors in Python (same messages as the reference's
TORCH_CHECKs), allocates the output with ``torch.empty`` and passes raw device
pointers plus the current HIP stream to the ``extern "C"`` entry point.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # must be imported first: the HIP runtime comes from torch's libamdhip64

_LIB_PATH = Path(__file__).resolve().parent / "libdimq_hip.so"

if not _LIB_PATH.exists():
    raise ImportError(
        f"{_LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
        "or `make -C dimq_amd/csrc`"
    )

lib = ctypes.CDLL(str(_LIB_PATH))

F32, F16, BF16, F64, U8 = 0, 1, 2, 3, 4
NCHW, NHWC = 0, 1
VARIANT_AUTO, VARIANT_SMALL_M, VARIANT_MFMA = 0, 1, 2

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: F64, torch.uint8: U8}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_dbl = ctypes.c_double

_SIGS = {
    "dimq_last_error": (ctypes.c_char_p, []),
    "dimq_abi_version": (_int, []),
    "dimq_pack_u4": (_int, [_vp, _i64, _vp, _vp]),
    "dimq_unpack_u4": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "dimq_quantize_activation_u4": (_int, [_vp, _int, _i64, _dbl, _i64, _vp, _vp]),
    "dimq_build_product_table": (_int, [_vp, _int, _i64, _dbl, _i64, _vp, _vp]),
    "dimq_linear_lut": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _i64, _vp, _int, _i64, _i64, _i64,
                               _vp, _vp]),
    "dimq_conv2d_lut": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _i64, _vp, _int,
                               _i64] + [_i64] * 11 + [_vp, _vp]),
    "dimq_linear_lut_workspace_bytes": (_i64, [_i64, _i64, _int]),
    "dimq_linear_lut_ws": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _i64, _vp, _int, _i64, _i64,
                                  _i64, _vp, _vp, _i64, _vp]),
    "dimq_linear_lut_noalloc": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _i64, _vp, _int, _i64,
                                       _i64, _i64, _vp, _vp]),
    "dimq_conv2d_lut_workspace_bytes": (_i64, [_i64] * 9 + [_int]),
    "dimq_conv2d_lut_ws": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _i64, _vp,
                                  _int, _i64] + [_i64] * 11 + [_vp, _vp, _i64, _vp]),
    "dimq_quantize_activation_f16": (_int, [_vp, _int, _i64, _dbl, _i64, _vp, _vp]),
    "dimq_linear_lut_q": (_int, [_vp, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _vp, _int, _i64, _i64, _i64, _int,
                                 _dbl, _i64, _vp, _int, _vp]),
    "dimq_conv2d_lut_q": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _int, _i64, _dbl, _vp,
                                 _int, _i64] + [_i64] * 11 + [_int, _dbl, _i64, _vp, _int, _vp]),
    "dimq_layer_norm": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _int, _dbl, _vp, _vp]),
    "dimq_layer_norm_ex": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _int, _dbl, _vp, _int, _vp]),
    "dimq_max_pool2d_nhwc": (_int, [_vp, _int] + [_i64] * 10 + [_vp, _vp]),
    "dimq_pack_bits": (_int, [_vp, _i64, _int, _vp, _vp]),
    "dimq_unpack_bits": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "dimq_hard_quantize": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _vp, _vp]),
    "dimq_build_product_table_grouped": (_int, [_vp, _int, _i64, _i64, _dbl, _i64, _vp, _vp]),
    "dimq_linear_codebook": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp, _int, _i64,
                                    _vp, _int, _int, _vp]),
    "dimq_conv2d_prepared_words": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "dimq_conv2d_prepare_weight": (_int, [_vp, _i64, _int, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "dimq_conv2d_codebook": (_int, [_vp, _int, _int, _i64, _i64, _i64, _i64, _vp, _i64, _int, _vp, _i64, _vp, _int,
                                    _i64, _i64, _vp, _int] + [_i64] * 10 + [_vp, _int, _int, _int, _vp]),
    "dimq_linear_codebook_ex": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp, _int,
                                       _i64, _vp, _int, _vp, _int, _int, _int, _vp]),
    "dimq_linear_codebook_workspace_bytes": (_i64, [_i64, _i64, _i64, _int, _int]),
    "dimq_linear_codebook_ex_ws": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp, _int,
                                          _i64, _vp, _int, _vp, _int, _int, _int, _vp, _i64, _vp]),
    "dimq_codebook_predecode_bytes": (_i64, [_i64, _i64, _int]),
    "dimq_codebook_predecode_batch": (_int, [_vp, _int, _vp]),
    "dimq_linear_codebook_predecoded": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp,
                                               _int, _i64, _vp, _int, _vp, _int, _int, _int, _vp, _vp, _i64, _vp]),
    "dimq_linear_codebook_act_workspace_bytes": (_i64, [_i64, _i64]),
    "dimq_linear_codebook_act": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp, _i64, _vp,
                                        _int, _i64, _vp, _int, _int, _vp, _i64, _vp]),
    "dimq_build_codebook_product_table": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _vp, _vp]),
    "dimq_linear_lut_act": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _vp, _int, _i64, _i64, _vp, _i64, _int, _vp,
                                   _int, _i64, _vp, _int, _vp]),
    "dimq_conv2d_codebook_act_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "dimq_conv2d_codebook_act": (_int, [_vp, _int, _int, _i64, _i64, _i64, _i64, _vp, _i64, _int, _vp, _i64, _vp,
                                        _int, _i64, _i64, _vp, _i64, _vp, _int] + [_i64] * 10 +
                                 [_vp, _int, _int, _int, _vp, _i64, _vp]),
    "dimq_conv2d_codebook_ex": (_int, [_vp, _int, _int, _i64, _i64, _i64, _i64, _vp, _i64, _int, _vp, _i64, _vp,
                                       _int, _i64, _i64, _vp, _int] + [_i64] * 10 +
                                [_vp, _int, _int, _vp, _int, _int, _int, _vp]),
    "dimq_qat_workspace_bytes": (_i64, [_i64, _i64]),
    "dimq_softmin_loss_forward": (_int, [_vp, _int, _i64, _vp, _i64, _dbl, _int, _vp, _vp, _vp, _i64, _vp]),
    "dimq_softmin_loss_backward": (_int, [_vp, _int, _i64, _vp, _i64, _dbl, _int, _vp, _vp, _vp, _int, _vp, _vp, _i64,
                                          _vp]),
    "dimq_soft_dequantize_forward": (_int, [_vp, _int, _i64, _vp, _i64, _dbl, _vp, _vp, _vp]),
    "dimq_soft_dequantize_backward": (_int, [_vp, _int, _i64, _vp, _i64, _dbl, _vp, _vp, _int, _vp, _int, _vp, _vp,
                                             _i64, _vp]),
    "dimq_separation_loss": (_int, [_vp, _int, _i64, _vp, _i64, _dbl, _dbl, _vp, _vp, _vp, _i64, _vp]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)  # AttributeError here = the library lacks a declared entry point
    _fn.restype = _res
    _fn.argtypes = _args


def exported_symbols() -> list[str]:
    return sorted(_SIGS)


def _check(rc: int) -> None:
    if rc != 0:
        msg = lib.dimq_last_error().decode(errors="replace")
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _dtype(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}") from None


def _require_cuda(t: torch.Tensor, msg: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(msg)


# ---------------------------------------------------------------------------
# reference ops (csrc/dimq_pack.cu, dimq_product_table.cu, dimq_gemm_lut.cu, dimq_conv2d_lut.cu)
# ---------------------------------------------------------------------------

def pack_u4_impl(indices: torch.Tensor) -> torch.Tensor:
    _require_cuda(indices, "pack_u4 expects a CUDA tensor")
    if indices.dtype != torch.uint8:
        raise RuntimeError("pack_u4 expects uint8 indices")
    flat = indices.contiguous().view(-1)
    out = torch.empty(((flat.numel() + 1) // 2,), dtype=torch.uint8, device=flat.device)
    with torch.cuda.device(flat.device):
        _check(lib.dimq_pack_u4(_ptr(flat), flat.numel(), _ptr(out), _stream(flat.device)))
    return out


def unpack_u4_impl(packed: torch.Tensor, numel: int) -> torch.Tensor:
    _require_cuda(packed, "unpack_u4 expects a CUDA tensor")
    if packed.dtype != torch.uint8:
        raise RuntimeError("unpack_u4 expects uint8 packed data")
    if numel < 0:
        raise RuntimeError("numel must be non-negative")
    if packed.numel() < (numel + 1) // 2:
        raise RuntimeError("packed tensor is too small for requested numel")
    flat = packed.contiguous().view(-1)
    out = torch.empty((numel,), dtype=torch.uint8, device=flat.device)
    with torch.cuda.device(flat.device):
        _check(lib.dimq_unpack_u4(_ptr(flat), flat.numel(), numel, _ptr(out), _stream(flat.device)))
    return out


def quantize_activation_u4_impl(x: torch.Tensor, act_scale: float, act_zp: int) -> torch.Tensor:
    _require_cuda(x, "quantize_activation_u4 expects a CUDA tensor")
    if not x.is_floating_point():
        raise RuntimeError("quantize_activation_u4 expects floating input")
    xc = x.contiguous()
    out = torch.empty(xc.shape, dtype=torch.uint8, device=xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_quantize_activation_u4(_ptr(xc), _dtype(xc), xc.numel(), float(act_scale), int(act_zp),
                                               _ptr(out), _stream(xc.device)))
    return out


def build_product_table_impl(codebook: torch.Tensor, act_scale: float, act_zp: int) -> torch.Tensor:
    _require_cuda(codebook, "build_product_table expects a CUDA tensor")
    if not codebook.is_floating_point():
        raise RuntimeError("build_product_table expects floating codebook")
    cb = codebook.contiguous().view(-1)
    table = torch.empty((16, 16), dtype=torch.float32, device=cb.device)
    with torch.cuda.device(cb.device):
        _check(lib.dimq_build_product_table(_ptr(cb), _dtype(cb), cb.numel(), float(act_scale), int(act_zp),
                                            _ptr(table), _stream(cb.device)))
    return table


def _bias_args(bias: torch.Tensor | None, n: int, what: str):
    if bias is None:
        return None, None, F32, 0
    _require_cuda(bias, "bias must be CUDA when provided")
    if bias.numel() != n:
        raise RuntimeError(f"bias numel must equal {what}")
    b = bias.contiguous()
    return b, _ptr(b), _dtype(b), b.numel()


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    """Device workspace of the W4A4 fast path (None when the call needs none).

    Allocated from torch's caching allocator on the current stream, so
    back-to-back calls reuse the same block without a hipMalloc.
    """
    if nbytes <= 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


def linear_lut_impl(x, packed_w, codebook, act_scale, act_zp, bias, out_features, in_features):
    _require_cuda(x, "linear_lut expects CUDA input")
    _require_cuda(packed_w, "linear_lut expects CUDA packed_weight")
    _require_cuda(codebook, "linear_lut expects CUDA codebook")
    if not x.is_floating_point():
        raise RuntimeError("linear_lut expects floating input")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if not codebook.is_floating_point():
        raise RuntimeError("codebook must be floating point")
    if codebook.numel() != 16:
        raise RuntimeError("codebook must have 16 entries for W4")
    if out_features <= 0 or in_features <= 0:
        raise RuntimeError("linear dimensions must be positive")
    if x.numel() % in_features != 0:
        raise RuntimeError("input numel must be divisible by in_features")
    if x.dim() == 0 or x.size(-1) != in_features:
        raise RuntimeError("input last dimension must equal in_features")
    xc = x.contiguous()
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous().view(-1)
    b, bp, bdt, bn = _bias_args(bias, out_features, "out_features")
    M = xc.numel() // in_features
    y = torch.empty((M, out_features), dtype=torch.float32, device=xc.device)
    ws = _workspace(lib.dimq_linear_lut_workspace_bytes(M, in_features, _dtype(cb)), xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_linear_lut_ws(_ptr(xc), _dtype(xc), M, _ptr(pw), pw.numel(), _ptr(cb), _dtype(cb), cb.numel(),
                                      float(act_scale), int(act_zp), bp, bdt, bn, out_features, in_features, _ptr(y),
                                      _ptr(ws), 0 if ws is None else ws.numel(), _stream(xc.device)))
    return y.view(*x.shape[:-1], out_features)


def conv2d_lut_impl(x, packed_w, codebook, act_scale, act_zp, bias, out_channels, in_channels_per_group, kernel_h,
                    kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups):
    _require_cuda(x, "conv2d_lut expects CUDA input")
    if x.dim() != 4:
        raise RuntimeError("conv2d_lut expects NCHW input")
    _require_cuda(packed_w, "conv2d_lut expects CUDA packed_weight")
    _require_cuda(codebook, "conv2d_lut expects CUDA codebook")
    if not x.is_floating_point():
        raise RuntimeError("conv2d_lut expects floating input")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if not codebook.is_floating_point():
        raise RuntimeError("codebook must be floating point")
    xc = x.contiguous()
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous().view(-1)
    B, C, H, W = xc.shape
    b, bp, bdt, bn = _bias_args(bias, out_channels, "out_channels")
    oh = (H + 2 * pad_h - dilation_h * (kernel_h - 1) - 1) // stride_h + 1 if stride_h > 0 else 0
    ow = (W + 2 * pad_w - dilation_w * (kernel_w - 1) - 1) // stride_w + 1 if stride_w > 0 else 0
    y = torch.empty((B, out_channels, max(oh, 0), max(ow, 0)), dtype=torch.float32, device=xc.device)
    ws = None
    if y.numel() > 0:
        ws = _workspace(lib.dimq_conv2d_lut_workspace_bytes(B, C, H, W, out_channels, in_channels_per_group, kernel_h,
                                                            kernel_w, groups, _dtype(cb)), xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_conv2d_lut_ws(_ptr(xc), _dtype(xc), B, C, H, W, _ptr(pw), pw.numel(), _ptr(cb), _dtype(cb),
                                      cb.numel(), float(act_scale), int(act_zp), bp, bdt, bn, out_channels,
                                      in_channels_per_group, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w,
                                      dilation_h, dilation_w, groups, _ptr(y), _ptr(ws),
                                      0 if ws is None else ws.numel(), _stream(xc.device)))
    return y


# ---------------------------------------------------------------------------
# generalised ops
# ---------------------------------------------------------------------------

def pack_bits_impl(indices: torch.Tensor, bits: int) -> torch.Tensor:
    _require_cuda(indices, "pack_bits expects a CUDA tensor")
    if indices.dtype != torch.uint8:
        raise RuntimeError("pack_bits expects uint8 indices")
    flat = indices.contiguous().view(-1)
    out = torch.empty(((flat.numel() * bits + 7) // 8,), dtype=torch.uint8, device=flat.device)
    with torch.cuda.device(flat.device):
        _check(lib.dimq_pack_bits(_ptr(flat), flat.numel(), int(bits), _ptr(out), _stream(flat.device)))
    return out


def unpack_bits_impl(packed: torch.Tensor, numel: int, bits: int) -> torch.Tensor:
    _require_cuda(packed, "unpack_bits expects a CUDA tensor")
    if packed.dtype != torch.uint8:
        raise RuntimeError("unpack_bits expects uint8 packed data")
    if numel < 0:
        raise RuntimeError("numel must be non-negative")
    flat = packed.contiguous().view(-1)
    out = torch.empty((numel,), dtype=torch.uint8, device=flat.device)
    with torch.cuda.device(flat.device):
        _check(lib.dimq_unpack_bits(_ptr(flat), flat.numel(), numel, int(bits), _ptr(out), _stream(flat.device)))
    return out


def hard_quantize_impl(w: torch.Tensor, centers: torch.Tensor, per_channel: bool):
    _require_cuda(w, "hard_quantize expects a CUDA tensor")
    _require_cuda(centers, "hard_quantize expects CUDA centers")
    wc = w.contiguous()
    if wc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        wc = wc.float()
    c = centers.detach().float().contiguous()
    if per_channel:
        if c.dim() != 2 or wc.dim() == 0 or c.size(0) != wc.size(0):
            raise RuntimeError("per-channel centers must be [out_channels, K]")
        rows, K = c.size(0), c.size(1)
    else:
        rows, K = 1, c.numel()
    row_len = wc.numel() // rows if rows else 0
    idx = torch.empty(wc.shape, dtype=torch.uint8, device=wc.device)
    vals = torch.empty(wc.shape, dtype=wc.dtype, device=wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_hard_quantize(_ptr(wc), _dtype(wc), rows, row_len, _ptr(c), K, int(bool(per_channel)),
                                      _ptr(idx), _ptr(vals), _stream(wc.device)))
    return idx, vals


def build_product_table_grouped_impl(codebook: torch.Tensor, act_scale: float, act_zp: int) -> torch.Tensor:
    _require_cuda(codebook, "build_product_table expects a CUDA tensor")
    cb = codebook.contiguous()
    G, Kc = (1, cb.numel()) if cb.dim() <= 1 else (cb.size(0), cb.numel() // max(cb.size(0), 1))
    out = torch.empty((G, Kc, 16), dtype=torch.float32, device=cb.device)
    with torch.cuda.device(cb.device):
        _check(lib.dimq_build_product_table_grouped(_ptr(cb), _dtype(cb), G, Kc, float(act_scale), int(act_zp),
                                                    _ptr(out), _stream(cb.device)))
    return out


def _cb_shape(codebook: torch.Tensor, n: int):
    if codebook.dim() == 2 and codebook.size(0) == n and n != 1:
        return codebook.size(0), codebook.size(1)
    if codebook.dim() == 2 and codebook.size(0) == 1:
        return 1, codebook.size(1)
    if codebook.dim() <= 1:
        return 1, codebook.numel()
    raise RuntimeError("codebook must be [K] (per layer) or [out_features, K] (per channel)")


def _residual_args(residual: torch.Tensor | None, y: torch.Tensor, mf=torch.contiguous_format):
    """Residual of the fused epilogue: y's shape, moved into y's memory order."""
    if residual is None:
        return None, None, F32
    _require_cuda(residual, "residual must be CUDA when provided")
    if tuple(residual.shape) != tuple(y.shape):
        raise RuntimeError(f"residual shape {tuple(residual.shape)} must equal the output shape {tuple(y.shape)}")
    if not residual.is_floating_point():
        raise RuntimeError("residual must be floating point")
    r = residual.contiguous(memory_format=mf)
    return r, _ptr(r), _dtype(r)


def linear_codebook_impl(x, packed_w, codebook, bits, bias, out_features, in_features, out_dtype=None, variant=0,
                         residual=None, activation=0, decoded=None):
    _require_cuda(x, "linear_codebook expects CUDA input")
    _require_cuda(packed_w, "linear_codebook expects CUDA packed_weight")
    _require_cuda(codebook, "linear_codebook expects CUDA codebook")
    if x.dim() == 0 or x.size(-1) != in_features:
        raise RuntimeError("input last dimension must equal in_features")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    xc = x.contiguous()
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    rows, size = _cb_shape(cb, out_features)
    b, bp, bdt, _ = _bias_args(bias, out_features, "out_features")
    odt = x.dtype if out_dtype is None else out_dtype
    M = xc.numel() // in_features if in_features else 0
    y = torch.empty((M, out_features), dtype=odt, device=xc.device)
    if residual is not None and tuple(residual.shape) != (*x.shape[:-1], out_features):
        raise RuntimeError(f"residual shape {tuple(residual.shape)} must equal the output shape "
                           f"{(*x.shape[:-1], out_features)}")
    r, rp, rdt = _residual_args(None if residual is None else residual.reshape(M, out_features), y)
    ws = _workspace(lib.dimq_linear_codebook_workspace_bytes(M, in_features, out_features, int(bits), _dtype(xc)),
                    xc.device)
    with torch.cuda.device(xc.device):
        if decoded is None:
            _check(lib.dimq_linear_codebook_ex_ws(_ptr(xc), _dtype(xc), M, in_features, _ptr(pw), pw.numel(),
                                                  int(bits), _ptr(cb), _dtype(cb), rows, size, bp, bdt, out_features,
                                                  _ptr(y), _dtype(y), rp, rdt, int(activation), int(variant),
                                                  _ptr(ws), 0 if ws is None else ws.numel(), _stream(xc.device)))
        else:
            _require_cuda(decoded, "decoded weights must be CUDA")
            if decoded.dtype != torch.uint8 or decoded.numel() < lib.dimq_codebook_predecode_bytes(
                    out_features, in_features, int(bits)):
                raise RuntimeError("decoded must be the uint8 buffer predecode_codebook_weights made for this layer")
            _check(lib.dimq_linear_codebook_predecoded(_ptr(xc), _dtype(xc), M, in_features, _ptr(pw), pw.numel(),
                                                       int(bits), _ptr(cb), _dtype(cb), rows, size, bp, bdt,
                                                       out_features, _ptr(y), _dtype(y), rp, rdt, int(activation),
                                                       int(variant), _ptr(decoded), _ptr(ws),
                                                       0 if ws is None else ws.numel(), _stream(xc.device)))
    return y.view(*x.shape[:-1], out_features)


class PredecodeJob(ctypes.Structure):
    """DimqPredecodeJob of include/dimq_hip.h."""
    _fields_ = [("packed_w", _vp), ("packed_numel", _i64), ("bits", _int), ("codebook", _vp), ("cb_dtype", _int),
                ("cb_rows", _i64), ("cb_size", _i64), ("out_features", _i64), ("in_features", _i64),
                ("decoded", _vp)]


def predecode_codebook_weights_impl(layers):
    """Decodes every (packed_w, codebook, bits, out_features, in_features) of ``layers`` with one
    dimq_codebook_predecode_batch call: one uint8 device buffer, and per layer a 256-byte aligned view of
    dimq_codebook_predecode_bytes(...) bytes (None for a layer the batch cannot decode: bits 8, in_features
    not a multiple of 32)."""
    if not layers:
        return None, []
    dev = layers[0][0].device
    sizes = [int(lib.dimq_codebook_predecode_bytes(int(n), int(k), int(b))) for (_, _, b, n, k) in layers]
    total = sum(sizes)
    if total == 0:
        return None, [None] * len(layers)
    buf = torch.empty(total + 256, dtype=torch.uint8, device=dev)
    off = (-buf.data_ptr()) % 256
    views, jobs, keep = [], [], []
    for (pw, cb, b, n, k), nbytes in zip(layers, sizes):
        if nbytes == 0:
            views.append(None)
            continue
        _require_cuda(pw, "predecode expects CUDA packed weights")
        _require_cuda(cb, "predecode expects CUDA codebooks")
        if pw.device != dev or cb.device != dev:
            raise RuntimeError("predecode: all layers must be on one device")
        pwc, cbc = pw.contiguous().view(-1), cb.contiguous()
        rows, size = _cb_shape(cbc, int(n))
        keep += [pwc, cbc]
        v = buf[off:off + nbytes]
        views.append(v)
        jobs.append(PredecodeJob(_ptr(pwc), pwc.numel(), int(b), _ptr(cbc), _dtype(cbc), rows, size, int(n), int(k),
                                 _ptr(v)))
        off += nbytes
    arr = (PredecodeJob * len(jobs))(*jobs)
    with torch.cuda.device(dev):
        _check(lib.dimq_codebook_predecode_batch(ctypes.cast(arr, _vp), len(jobs), _stream(dev)))
    return buf, views


def linear_codebook_act_impl(x, packed_w, codebook, bits, act_centers, bias, out_features, in_features,
                             out_dtype=None, variant=0):
    _require_cuda(x, "linear_codebook_act expects CUDA input")
    _require_cuda(packed_w, "linear_codebook_act expects CUDA packed_weight")
    _require_cuda(codebook, "linear_codebook_act expects CUDA codebook")
    _require_cuda(act_centers, "linear_codebook_act expects CUDA activation centres")
    if x.dim() == 0 or x.size(-1) != in_features:
        raise RuntimeError("input last dimension must equal in_features")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    xc = x.contiguous()
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    ac = act_centers.detach().reshape(-1).float().contiguous()
    rows, size = _cb_shape(cb, out_features)
    b, bp, bdt, _ = _bias_args(bias, out_features, "out_features")
    odt = x.dtype if out_dtype is None else out_dtype
    M = xc.numel() // in_features if in_features else 0
    y = torch.empty((M, out_features), dtype=odt, device=xc.device)
    ws = _workspace(lib.dimq_linear_codebook_act_workspace_bytes(M, in_features), xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_linear_codebook_act(_ptr(xc), _dtype(xc), M, in_features, _ptr(pw), pw.numel(), int(bits),
                                            _ptr(cb), _dtype(cb), rows, size, _ptr(ac), ac.numel(), bp, bdt,
                                            out_features, _ptr(y), _dtype(y), int(variant), _ptr(ws),
                                            0 if ws is None else ws.numel(), _stream(xc.device)))
    return y.view(*x.shape[:-1], out_features)


# ---------------------------------------------------------------------------
# chained W4A4 layers: activations as the fp16 integers a - zp between layers
def quantize_activation_f16_impl(x, act_scale, act_zp):
    _require_cuda(x, "quantize_activation expects CUDA input")
    xc = x.contiguous()
    out = torch.empty(xc.shape, dtype=torch.float16, device=xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_quantize_activation_f16(_ptr(xc), _dtype(xc), xc.numel(), float(act_scale), int(act_zp),
                                                _ptr(out), _stream(xc.device)))
    return out


def _q_out(out_act, out_dtype):
    if out_act is None:
        return 0.0, 0, (torch.float32 if out_dtype is None else out_dtype)
    s, zp = out_act
    if out_dtype not in (None, torch.float16):
        raise RuntimeError("a quantized output is written as fp16 codes")
    return float(s), int(zp), torch.float16


def linear_lut_q_impl(xq, packed_w, codebook, act_scale, bias, out_features, in_features, activation=0,
                      out_act=None, out_dtype=None):
    _require_cuda(xq, "linear_lut_q expects CUDA input")
    if xq.dtype != torch.float16:
        raise RuntimeError("linear_lut_q expects the fp16 activation codes a - zp")
    if xq.dim() == 0 or xq.size(-1) != in_features:
        raise RuntimeError("input last dimension must equal in_features")
    xc = xq.contiguous()
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    b, bp, bdt, bn = _bias_args(bias, out_features, "out_features")
    qs, qzp, odt = _q_out(out_act, out_dtype)
    M = xc.numel() // in_features if in_features else 0
    y = torch.empty((M, out_features), dtype=odt, device=xc.device)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_linear_lut_q(_ptr(xc), M, _ptr(pw), pw.numel(), _ptr(cb), _dtype(cb), cb.numel(),
                                     float(act_scale), bp, bdt, bn, out_features, in_features, int(activation), qs,
                                     qzp, _ptr(y), _dtype(y), _stream(xc.device)))
    return y.view(*xq.shape[:-1], out_features)


def conv2d_lut_q_impl(xq, packed_w, codebook, act_scale, bias, out_channels, in_channels_per_group, kernel_h,
                      kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups, prepared_w=None,
                      activation=0, out_act=None, out_dtype=None):
    _require_cuda(xq, "conv2d_lut_q expects CUDA input")
    if xq.dtype != torch.float16 or xq.dim() != 4:
        raise RuntimeError("conv2d_lut_q expects NCHW fp16 activation codes a - zp")
    xc = xq.contiguous()
    B, C, H, W = xc.shape
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    b, bp, bdt, bn = _bias_args(bias, out_channels, "out_channels")
    qs, qzp, odt = _q_out(out_act, out_dtype)
    OH = (H + 2 * pad_h - dilation_h * (kernel_h - 1) - 1) // stride_h + 1
    OW = (W + 2 * pad_w - dilation_w * (kernel_w - 1) - 1) // stride_w + 1
    y = torch.empty((B, out_channels, OH, OW), dtype=odt, device=xc.device)
    pr = None if prepared_w is None else prepared_w.contiguous()
    with torch.cuda.device(xc.device):
        _check(lib.dimq_conv2d_lut_q(_ptr(xc), B, C, H, W, _ptr(pw), pw.numel(), _ptr(pr),
                                     0 if pr is None else pr.numel(), _ptr(cb), _dtype(cb), cb.numel(),
                                     float(act_scale), bp, bdt, bn, out_channels, in_channels_per_group, kernel_h,
                                     kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups,
                                     int(activation), qs, qzp, _ptr(y), _dtype(y), _stream(xc.device)))
    return y


def build_codebook_product_table_impl(codebook, act_values):
    _require_cuda(codebook, "build_codebook_product_table expects CUDA codebook")
    cb = codebook.contiguous()
    ca = act_values.detach().reshape(-1).float().contiguous().to(cb.device)
    rows = cb.shape[0] if cb.dim() == 2 else 1
    kw = cb.shape[-1]
    table = torch.empty((rows, kw, ca.numel()), dtype=torch.float32, device=cb.device)
    with torch.cuda.device(cb.device):
        _check(lib.dimq_build_codebook_product_table(_ptr(cb), _dtype(cb), rows, kw, _ptr(ca), ca.numel(),
                                                     _ptr(table), _stream(cb.device)))
    return table


def linear_lut_act_impl(act_idx, packed_w, codebook, bits, act_centers, x_dtype, bias, out_features, in_features,
                        out_dtype=torch.float32):
    _require_cuda(act_idx, "linear_lut_act expects CUDA activation indices")
    if act_idx.dtype != torch.uint8 or act_idx.size(-1) != in_features:
        raise RuntimeError("activation indices must be uint8 [..., in_features]")
    ai = act_idx.contiguous()
    if ai.data_ptr() % 16:
        ai = ai.clone()  # 16-byte index loads
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    ac = act_centers.detach().reshape(-1).float().contiguous()
    rows, size = _cb_shape(cb, out_features)
    b, bp, bdt, _ = _bias_args(bias, out_features, "out_features")
    M = ai.numel() // in_features
    y = torch.empty((M, out_features), dtype=out_dtype, device=ai.device)
    with torch.cuda.device(ai.device):
        _check(lib.dimq_linear_lut_act(_ptr(ai), M, in_features, _ptr(pw), pw.numel(), int(bits), _ptr(cb), _dtype(cb),
                                       rows, size, _ptr(ac), ac.numel(), _DT[x_dtype], bp, bdt, out_features, _ptr(y),
                                       _dtype(y), _stream(ai.device)))
    return y.view(*act_idx.shape[:-1], out_features)


def conv2d_codebook_act_impl(x, packed_w, codebook, bits, act_centers, bias, out_channels, in_channels_per_group,
                             kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups,
                             out_dtype=None, prepared_w=None, variant=0):
    _require_cuda(x, "conv2d_codebook_act expects CUDA input")
    if x.dim() != 4:
        raise RuntimeError("conv2d_codebook_act expects NCHW-shaped input")
    nhwc = x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous()
    mf = torch.channels_last if nhwc else torch.contiguous_format
    xc = x.contiguous(memory_format=mf)
    B, C, H, W = xc.shape
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    ac = act_centers.detach().reshape(-1).float().contiguous()
    rows, size = _cb_shape(cb, out_channels)
    b, bp, bdt, _ = _bias_args(bias, out_channels, "out_channels")
    OH = (H + 2 * pad_h - dilation_h * (kernel_h - 1) - 1) // stride_h + 1
    OW = (W + 2 * pad_w - dilation_w * (kernel_w - 1) - 1) // stride_w + 1
    odt = x.dtype if out_dtype is None else out_dtype
    y = torch.empty((B, out_channels, OH, OW), dtype=odt, device=xc.device, memory_format=mf)
    ws = _workspace(lib.dimq_conv2d_codebook_act_workspace_bytes(B, C, H, W), xc.device)
    pr = None if prepared_w is None else prepared_w.contiguous()
    lay = NHWC if nhwc else NCHW
    with torch.cuda.device(xc.device):
        _check(lib.dimq_conv2d_codebook_act(_ptr(xc), _dtype(xc), lay, B, C, H, W, _ptr(pw), pw.numel(), int(bits),
                                            _ptr(pr), 0 if pr is None else pr.numel(), _ptr(cb), _dtype(cb), rows,
                                            size, _ptr(ac), ac.numel(), bp, bdt, out_channels, kernel_h, kernel_w,
                                            stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups,
                                            _ptr(y), _dtype(y), lay, int(variant), _ptr(ws),
                                            0 if ws is None else ws.numel(), _stream(xc.device)))
    return y


def prepare_conv_weight_impl(packed_w, bits, out_channels, in_channels, kernel_h, kernel_w):
    _require_cuda(packed_w, "prepare_conv_weight expects a CUDA tensor")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    words = int(lib.dimq_conv2d_prepared_words(out_channels, in_channels, kernel_h, kernel_w, int(bits)))
    if words <= 0:
        raise RuntimeError(f"no kernel layout for C={in_channels} KH={kernel_h} KW={kernel_w} bits={bits}")
    pw = packed_w.contiguous().view(-1)
    out = torch.empty((words,), dtype=torch.int32, device=pw.device)
    with torch.cuda.device(pw.device):
        _check(lib.dimq_conv2d_prepare_weight(_ptr(pw), pw.numel(), int(bits), out_channels, in_channels, kernel_h,
                                              kernel_w, _ptr(out), words, _stream(pw.device)))
    return out


def prepared_conv_words(out_channels, in_channels, kernel_h, kernel_w, bits) -> int:
    return int(lib.dimq_conv2d_prepared_words(out_channels, in_channels, kernel_h, kernel_w, int(bits)))


def conv2d_codebook_impl(x, packed_w, codebook, bits, bias, out_channels, in_channels_per_group, kernel_h, kernel_w,
                         stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups, out_dtype=None, variant=0,
                         prepared_w=None, residual=None, activation=0):
    _require_cuda(x, "conv2d_codebook expects CUDA input")
    if x.dim() != 4:
        raise RuntimeError("conv2d_codebook expects a 4-D input")
    _require_cuda(packed_w, "conv2d_codebook expects CUDA packed_weight")
    _require_cuda(codebook, "conv2d_codebook expects CUDA codebook")
    if packed_w.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    B, C, H, W = x.shape
    if C != in_channels_per_group * groups:
        raise RuntimeError("input channels do not match weight/groups")
    channels_last = (not x.is_contiguous()) and x.is_contiguous(memory_format=torch.channels_last)
    if channels_last:
        xc, layout = x, NHWC
    else:
        xc, layout = x.contiguous(), NCHW
    pw = packed_w.contiguous().view(-1)
    cb = codebook.contiguous()
    rows, size = _cb_shape(cb, out_channels)
    b, bp, bdt, _ = _bias_args(bias, out_channels, "out_channels")
    oh = (H + 2 * pad_h - dilation_h * (kernel_h - 1) - 1) // stride_h + 1 if stride_h > 0 else 0
    ow = (W + 2 * pad_w - dilation_w * (kernel_w - 1) - 1) // stride_w + 1 if stride_w > 0 else 0
    odt = x.dtype if out_dtype is None else out_dtype
    mf = torch.channels_last if channels_last else torch.contiguous_format
    y = torch.empty((B, out_channels, max(oh, 0), max(ow, 0)), dtype=odt, device=xc.device, memory_format=mf)
    if prepared_w is not None:
        _require_cuda(prepared_w, "prepared_w must be CUDA when provided")
        prep = prepared_w.contiguous()
        prep_ptr, prep_words = _ptr(prep), prep.numel()
    else:
        prep_ptr, prep_words = None, 0
    r, rp, rdt = _residual_args(residual, y, mf)
    with torch.cuda.device(xc.device):
        _check(lib.dimq_conv2d_codebook_ex(_ptr(xc), _dtype(xc), layout, B, C, H, W, _ptr(pw), pw.numel(), int(bits),
                                           prep_ptr, prep_words, _ptr(cb), _dtype(cb), rows, size, bp, bdt,
                                           out_channels, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w,
                                           dilation_h, dilation_w, groups, _ptr(y), _dtype(y), layout, rp, rdt,
                                           int(activation), int(variant), _stream(xc.device)))
    return y


def layer_norm_impl(x, normalized_size, weight, bias, eps, out_dtype=None):
    """LayerNorm over the last dimension (support op of the ViT workload); output in out_dtype (fp16 / bf16,
    default x's dtype)."""
    _require_cuda(x, "layer_norm expects CUDA input")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("layer_norm expects fp16 or bf16 input")
    D = int(normalized_size)
    if x.dim() == 0 or x.size(-1) != D:
        raise RuntimeError("layer_norm: last input dimension must equal the normalized size")
    xv = x.reshape(-1, D) if x.dim() != 2 else x
    if xv.stride(-1) != 1 or xv.stride(0) % 8 != 0 or xv.data_ptr() % 16 != 0:
        xv = xv.contiguous()
    wdt = F32
    for t in (weight, bias):
        if t is not None:
            _require_cuda(t, "layer_norm weight and bias must be CUDA tensors")
            if t.numel() != D:
                raise RuntimeError("layer_norm weight and bias must have the normalized size")
    if weight is not None and bias is not None and weight.dtype != bias.dtype:
        bias = bias.to(weight.dtype)
    w = weight.contiguous() if weight is not None else None
    b = bias.contiguous() if bias is not None else None
    if w is not None or b is not None:
        wdt = _dtype(w if w is not None else b)
    odt = x.dtype if out_dtype is None else out_dtype
    if odt not in (torch.float16, torch.bfloat16):
        raise RuntimeError("layer_norm writes fp16 or bf16 output")
    y = torch.empty(xv.shape, dtype=odt, device=x.device)
    with torch.cuda.device(x.device):
        _check(lib.dimq_layer_norm_ex(_ptr(xv), _dtype(xv), xv.shape[0], D, xv.stride(0), _ptr(w), _ptr(b), wdt,
                                      float(eps), _ptr(y), _dtype(y), _stream(x.device)))
    return y.view(x.shape)


def max_pool2d_impl(x, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w):
    """2-D max pooling of a channels-last fp16/bf16 tensor (support op of the ResNet workload)."""
    _require_cuda(x, "max_pool2d expects CUDA input")
    if x.dim() != 4 or not x.is_contiguous(memory_format=torch.channels_last):
        raise RuntimeError("max_pool2d expects a channels-last 4-D input")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("max_pool2d expects fp16 or bf16 input")
    B, C, H, W = x.shape
    oh = (H + 2 * pad_h - kernel_h) // stride_h + 1 if stride_h > 0 else 0
    ow = (W + 2 * pad_w - kernel_w) // stride_w + 1 if stride_w > 0 else 0
    y = torch.empty((B, C, max(oh, 0), max(ow, 0)), dtype=x.dtype, device=x.device,
                    memory_format=torch.channels_last)
    with torch.cuda.device(x.device):
        _check(lib.dimq_max_pool2d_nhwc(_ptr(x), _dtype(x), B, C, H, W, kernel_h, kernel_w, stride_h, stride_w, pad_h,
                                        pad_w, _ptr(y), _stream(x.device)))
    return y


# ---------------------------------------------------------------------------
# torch.library registration
# ---------------------------------------------------------------------------

_SCHEMAS = {
    # verbatim from dimq_cuda_backend/csrc/dimq_ops.cpp:38-43
    "pack_u4": ("pack_u4(Tensor indices) -> Tensor", pack_u4_impl),
    "unpack_u4": ("unpack_u4(Tensor packed, int numel) -> Tensor", unpack_u4_impl),
    "quantize_activation_u4": ("quantize_activation_u4(Tensor x, float act_scale, int act_zp) -> Tensor",
                               quantize_activation_u4_impl),
    "build_product_table": ("build_product_table(Tensor codebook, float act_scale, int act_zp) -> Tensor",
                            build_product_table_impl),
    "linear_lut": ("linear_lut(Tensor x, Tensor packed_w, Tensor codebook, float act_scale, int act_zp, Tensor? bias, "
                   "int out_features, int in_features) -> Tensor", linear_lut_impl),
    "conv2d_lut": ("conv2d_lut(Tensor x, Tensor packed_w, Tensor codebook, float act_scale, int act_zp, Tensor? bias, "
                   "int out_channels, int in_channels_per_group, int kernel_h, int kernel_w, int stride_h, "
                   "int stride_w, int pad_h, int pad_w, int dilation_h, int dilation_w, int groups) -> Tensor",
                   conv2d_lut_impl),
    # generalised ops
    "pack_bits": ("pack_bits(Tensor indices, int bits) -> Tensor", pack_bits_impl),
    "unpack_bits": ("unpack_bits(Tensor packed, int numel, int bits) -> Tensor", unpack_bits_impl),
    "hard_quantize": ("hard_quantize(Tensor w, Tensor centers, bool per_channel) -> (Tensor, Tensor)",
                      hard_quantize_impl),
    "build_product_table_grouped": ("build_product_table_grouped(Tensor codebook, float act_scale, int act_zp) "
                                    "-> Tensor", build_product_table_grouped_impl),
    "linear_codebook": ("linear_codebook(Tensor x, Tensor packed_w, Tensor codebook, int bits, Tensor? bias, "
                        "int out_features, int in_features, ScalarType? out_dtype=None, int variant=0, "
                        "Tensor? residual=None, int activation=0, Tensor? decoded=None) -> Tensor",
                        linear_codebook_impl),
    "conv2d_codebook": ("conv2d_codebook(Tensor x, Tensor packed_w, Tensor codebook, int bits, Tensor? bias, "
                        "int out_channels, int in_channels_per_group, int kernel_h, int kernel_w, int stride_h, "
                        "int stride_w, int pad_h, int pad_w, int dilation_h, int dilation_w, int groups, "
                        "ScalarType? out_dtype=None, int variant=0, Tensor? prepared_w=None, Tensor? residual=None, "
                        "int activation=0) -> Tensor",
                        conv2d_codebook_impl),
    "prepare_conv_weight": ("prepare_conv_weight(Tensor packed_w, int bits, int out_channels, int in_channels, "
                            "int kernel_h, int kernel_w) -> Tensor", prepare_conv_weight_impl),
    "linear_codebook_act": ("linear_codebook_act(Tensor x, Tensor packed_w, Tensor codebook, int bits, "
                            "Tensor act_centers, Tensor? bias, int out_features, int in_features, "
                            "ScalarType? out_dtype=None, int variant=0) -> Tensor", linear_codebook_act_impl),
    # support op of the end-to-end ViT workload
    "layer_norm": ("layer_norm(Tensor x, int normalized_size, Tensor? weight, Tensor? bias, float eps, "
                   "ScalarType? out_dtype=None) -> Tensor",
                   layer_norm_impl),
    "max_pool2d_nhwc": ("max_pool2d_nhwc(Tensor x, int kernel_h, int kernel_w, int stride_h, int stride_w, int pad_h, "
                        "int pad_w) -> Tensor", max_pool2d_impl),
}


def _register() -> torch.library.Library:
    lib_def = torch.library.Library("dimq", "DEF")
    for name, (schema, impl) in _SCHEMAS.items():
        lib_def.define(schema)
        lib_def.impl(name, impl, "CUDA")
    return lib_def


_LIBRARY = _register()


# The reference extension's module-level functions (csrc/dimq_ops.cpp:55-62,
# its PYBIND11_MODULE block): the same six names and positional arguments as
# the registered ops, callable as dimq_backend._C.linear_lut(...) without the
# dispatcher.  They are the op implementations themselves.
pack_u4 = pack_u4_impl
unpack_u4 = unpack_u4_impl
quantize_activation_u4 = quantize_activation_u4_impl
build_product_table = build_product_table_impl
linear_lut = linear_lut_impl
conv2d_lut = conv2d_lut_impl


# ---------------------------------------------------------------------------
# QAT kernels (quant/dimq.py:197-296): host wrappers used by dimq_amd.qat
def _qat_inputs(w, centers):
    _require_cuda(w, "QAT kernels expect CUDA weights")
    _require_cuda(centers, "QAT kernels expect CUDA centers")
    if w.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise RuntimeError("weights must be fp32, fp16, bf16 or fp64")
    wc = w.detach().contiguous()
    c = centers.detach().reshape(-1).float().contiguous()
    if c.numel() == 0:
        raise ValueError("centers must be non-empty")
    if c.numel() > 256:
        raise RuntimeError("at most 256 centers are supported")
    return wc, c


def _qat_ws(n, K, device):
    return torch.empty(int(lib.dimq_qat_workspace_bytes(n, K)), dtype=torch.uint8, device=device)


def softmin_loss_forward_impl(w, centers, tau, mean):
    """(loss fp32 scalar, aux [n, 2] fp32: (dmin_i, log s_i) for the backward)."""
    wc, c = _qat_inputs(w, centers)
    n = wc.numel()
    aux = torch.empty((n, 2), dtype=torch.float32, device=wc.device)
    loss = torch.empty((), dtype=torch.float32, device=wc.device)
    ws = _qat_ws(n, c.numel(), wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_softmin_loss_forward(_ptr(wc), _dtype(wc), n, _ptr(c), c.numel(), float(tau), int(bool(mean)),
                                             _ptr(aux), _ptr(loss), _ptr(ws), ws.numel(), _stream(wc.device)))
    return loss, aux


def softmin_loss_backward_impl(w, centers, tau, aux, grad_loss):
    """(grad_w in w's dtype, grad_centers fp32) of the sum reduction for the upstream scalar grad_loss."""
    wc, c = _qat_inputs(w, centers)
    n = wc.numel()
    g = grad_loss.detach().reshape(()).float().contiguous()
    gw = torch.empty_like(wc)
    gc = torch.empty(c.numel(), dtype=torch.float32, device=wc.device)
    ws = _qat_ws(n, c.numel(), wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_softmin_loss_backward(_ptr(wc), _dtype(wc), n, _ptr(c), c.numel(), float(tau), 0, _ptr(aux),
                                              _ptr(g), _ptr(gw), _dtype(gw), _ptr(gc), _ptr(ws), ws.numel(),
                                              _stream(wc.device)))
    return gw, gc


def soft_dequantize_forward_impl(w, centers, tau):
    wc, c = _qat_inputs(w, centers)
    n = wc.numel()
    out = torch.empty_like(wc)
    aux = torch.empty((n, 2), dtype=torch.float32, device=wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_soft_dequantize_forward(_ptr(wc), _dtype(wc), n, _ptr(c), c.numel(), float(tau), _ptr(out),
                                                _ptr(aux), _stream(wc.device)))
    return out, aux


def soft_dequantize_backward_impl(w, centers, tau, aux, grad_out):
    wc, c = _qat_inputs(w, centers)
    n = wc.numel()
    go = grad_out.detach().contiguous()
    gw = torch.empty_like(wc)
    gc = torch.empty(c.numel(), dtype=torch.float32, device=wc.device)
    ws = _qat_ws(n, c.numel(), wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_soft_dequantize_backward(_ptr(wc), _dtype(wc), n, _ptr(c), c.numel(), float(tau), _ptr(aux),
                                                 _ptr(go), _dtype(go), _ptr(gw), _dtype(gw), _ptr(gc), _ptr(ws),
                                                 ws.numel(), _stream(wc.device)))
    return gw, gc


def separation_loss_impl(w, centers, eta, eps):
    """(loss fp32 scalar, d loss / d centers fp32) -- the margin uses std(w), no gradient to w."""
    wc, c = _qat_inputs(w, centers)
    n = wc.numel()
    loss = torch.empty((), dtype=torch.float32, device=wc.device)
    gc = torch.empty(c.numel(), dtype=torch.float32, device=wc.device)
    ws = _qat_ws(n, c.numel(), wc.device)
    with torch.cuda.device(wc.device):
        _check(lib.dimq_separation_loss(_ptr(wc), _dtype(wc), n, _ptr(c), c.numel(), float(eta), float(eps),
                                        _ptr(loss), _ptr(gc), _ptr(ws), ws.numel(), _stream(wc.device)))
    return loss, gc
