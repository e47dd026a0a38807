"""CPU oracle for the DIMQ packed-index inference path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker.  The product (``dimq_amd``) never imports, links or calls it.

Two kinds of oracle live here:

* byte / integer / table arithmetic (pack, unpack, nearest-centre assignment,
  u4 activation quantization, product table, W4A4 LUT Linear/Conv2d) is a plain C
  restatement in ``dimq_oracle.c`` (built by ``oracle/Makefile`` into
  ``oracle/_build/libdimq_oracle.so``) driven through ctypes on numpy arrays;
* floating-point GEMM/conv parity uses the reference's own parity target,
  "dequantize then ``F.linear`` / ``F.conv2d`` in fp32 on the CPU"
  (``dimq_backend/reference.py:91-144``, ``quant/dimq_wrapper.py:189-197,237-240``),
  i.e. torch's CPU library routines over the dequantized weight.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libdimq_oracle.so"
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)


def build() -> Path:
    """Compile the C oracle (gcc) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(_LIB_PATH))
    lib.dimq_oracle_packed_nbytes.restype = ctypes.c_int64
    lib.dimq_oracle_packed_nbytes.argtypes = [ctypes.c_int64, ctypes.c_int]
    lib.dimq_oracle_pack_bits.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int, _u8p]
    lib.dimq_oracle_unpack_bits.restype = ctypes.c_int
    lib.dimq_oracle_unpack_bits.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _u8p]
    lib.dimq_oracle_hard_quantize.argtypes = [
        _f32p, ctypes.c_int64, ctypes.c_int64, _f32p, ctypes.c_int, ctypes.c_int, _u8p, _f32p]
    lib.dimq_oracle_quantize_act_u4.argtypes = [_f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, _u8p]
    lib.dimq_oracle_product_table.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, _f32p]
    lib.dimq_oracle_dequantize.restype = ctypes.c_int
    lib.dimq_oracle_dequantize.argtypes = [
        _u8p, ctypes.c_int64, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, _f32p]
    lib.dimq_oracle_linear_lut.argtypes = [
        _f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _u8p, _f32p, ctypes.c_float, ctypes.c_int,
        _f32p, _f32p]
    lib.dimq_oracle_conv2d_lut.argtypes = (
        [_f32p] + [ctypes.c_int] * 4 + [_u8p, _f32p, ctypes.c_float, ctypes.c_int, _f32p] + [ctypes.c_int] * 11
        + [_f32p])
    _lib = lib
    return lib


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, a.ctypes.data_as(_u8p)


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _np(t):
    """torch tensor or array-like -> numpy (CPU)."""
    if hasattr(t, "detach"):
        t = t.detach().cpu()
        if str(t.dtype) in ("torch.bfloat16", "torch.float16", "torch.float64"):
            t = t.float()
        return t.numpy()
    return np.asarray(t)


def packed_nbytes(n: int, bits: int) -> int:
    return int(_load().dimq_oracle_packed_nbytes(int(n), int(bits)))


def pack_bits(indices, bits: int) -> np.ndarray:
    """LSB-first b-bit packing (dimq_backend/export.py:38-55 generalised)."""
    idx, p = _u8(_np(indices).reshape(-1))
    out = np.zeros(max(packed_nbytes(idx.size, bits), 1), dtype=np.uint8)
    _load().dimq_oracle_pack_bits(p, idx.size, int(bits), out.ctypes.data_as(_u8p))
    return out[: packed_nbytes(idx.size, bits)]


def unpack_bits(packed, n: int, bits: int) -> np.ndarray:
    """Inverse of pack_bits (dimq_backend/export.py:58-78 generalised)."""
    pk, p = _u8(_np(packed).reshape(-1))
    out = np.zeros(max(int(n), 1), dtype=np.uint8)
    rc = _load().dimq_oracle_unpack_bits(p, pk.size, int(n), int(bits), out.ctypes.data_as(_u8p))
    if rc != 0:
        raise ValueError("packed tensor is too small for requested numel")
    return out[: int(n)]


def hard_quantize(w, centers, per_channel: bool | None = None):
    """Nearest-centre index assignment (quant/dimq.py:197-221).

    ``w`` is [rows, row_len] (any shape is flattened to one row when
    ``centers`` is 1-D); ``centers`` is [K] (per layer) or [rows, K]
    (per output channel).  Returns (uint8 indices, fp32 values)."""
    w = _np(w).astype(np.float32)
    c = _np(centers).astype(np.float32)
    if per_channel is None:
        per_channel = c.ndim == 2
    if per_channel:
        rows = c.shape[0]
        K = c.shape[1]
    else:
        rows = 1
        K = c.size
    shape = w.shape
    w2, wp = _f32(w.reshape(rows, -1))
    c2, cp = _f32(c.reshape(-1))
    idx = np.zeros(w2.size, dtype=np.uint8)
    val = np.zeros(w2.size, dtype=np.float32)
    _load().dimq_oracle_hard_quantize(wp, rows, w2.shape[1], cp, K, int(per_channel),
                                      idx.ctypes.data_as(_u8p), val.ctypes.data_as(_f32p))
    return idx.reshape(shape), val.reshape(shape)


def quantize_act_u4(x, scale: float, zp: int) -> np.ndarray:
    """dimq_backend/reference.py:11-21 (x is taken as x.float())."""
    x = _np(x).astype(np.float32)
    xa, xp = _f32(x.reshape(-1))
    out = np.zeros(max(xa.size, 1), dtype=np.uint8)
    _load().dimq_oracle_quantize_act_u4(xp, xa.size, float(np.float32(scale)), int(zp), out.ctypes.data_as(_u8p))
    return out[: xa.size].reshape(x.shape)


def product_table(codebook, scale: float, zp: int) -> np.ndarray:
    """dimq_backend/reference.py:32-44; [Kw,16] for a 1-D codebook, [G,Kw,16] for [G,Kw]."""
    cb = _np(codebook).astype(np.float32)
    G, Kw = (1, cb.size) if cb.ndim == 1 else cb.shape
    ca, cp = _f32(cb.reshape(-1))
    out = np.zeros(G * Kw * 16, dtype=np.float32)
    _load().dimq_oracle_product_table(cp, G, Kw, float(np.float32(scale)), int(zp), out.ctypes.data_as(_f32p))
    return out.reshape((Kw, 16) if cb.ndim == 1 else (G, Kw, 16))


def dequantize(packed, bits: int, codebook, N: int, K: int) -> np.ndarray:
    """dimq_backend/reference.py:47-56: W_hat[n,k] = C[idx] (C[n, idx] per channel)."""
    pk, pp = _u8(_np(packed).reshape(-1))
    cb = _np(codebook).astype(np.float32)
    if cb.ndim == 2 and cb.shape[0] not in (1, int(N)):
        raise ValueError(f"codebook rows {cb.shape[0]} must be 1 or {int(N)}")
    per_channel = cb.ndim == 2 and cb.shape[0] != 1  # a [1, E] codebook is the per-layer one
    Kc = cb.shape[-1]
    ca, cp = _f32(cb.reshape(-1))
    out = np.zeros(max(int(N) * int(K), 1), dtype=np.float32)
    rc = _load().dimq_oracle_dequantize(pp, pk.size, int(bits), cp, Kc, int(per_channel), int(N), int(K),
                                        out.ctypes.data_as(_f32p))
    if rc != 0:
        raise ValueError("packed weight too small or index outside the codebook")
    return out[: int(N) * int(K)].reshape(int(N), int(K))


def linear_lut(x, packed_w, codebook16, scale, zp, bias, out_features, in_features) -> np.ndarray:
    """W4A4 LUT Linear, dimq_backend/reference.py:59-88."""
    x = _np(x).astype(np.float32)
    lead = x.shape[:-1]
    xa, xp = _f32(x.reshape(-1, int(in_features)))
    pk, pp = _u8(_np(packed_w).reshape(-1))
    cb, cp = _f32(_np(codebook16).astype(np.float32).reshape(-1))
    assert cb.size == 16
    if bias is not None:
        ba, bp = _f32(_np(bias).astype(np.float32).reshape(-1))
    else:
        bp = None
    M = xa.shape[0]
    y = np.zeros((max(M, 1), int(out_features)), dtype=np.float32)
    _load().dimq_oracle_linear_lut(xp, M, int(out_features), int(in_features), pp, cp,
                                   float(np.float32(scale)), int(zp), bp, y.ctypes.data_as(_f32p))
    return y[:M].reshape(*lead, int(out_features))


def conv2d_lut(x, packed_w, codebook16, scale, zp, bias, weight_shape, stride=(1, 1), padding=(0, 0),
               dilation=(1, 1), groups=1) -> np.ndarray:
    """W4A4 LUT Conv2d (NCHW), dimq_backend/reference.py:147-205."""
    x = _np(x).astype(np.float32)
    B, C, H, W = x.shape
    OC, ICg, KH, KW = [int(v) for v in weight_shape]
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    xa, xp = _f32(x)
    pk, pp = _u8(_np(packed_w).reshape(-1))
    cb, cp = _f32(_np(codebook16).astype(np.float32).reshape(-1))
    ba, bp = _f32(_np(bias).astype(np.float32).reshape(-1)) if bias is not None else (None, None)
    y = np.zeros(max(B * OC * OH * OW, 1), dtype=np.float32)
    _load().dimq_oracle_conv2d_lut(xp, B, C, H, W, pp, cp, float(np.float32(scale)), int(zp), bp, OC, ICg, KH, KW,
                                   sh, sw, ph, pw, dh, dw, int(groups), y.ctypes.data_as(_f32p))
    return y[: B * OC * OH * OW].reshape(B, OC, OH, OW)


def _pair(v):
    if isinstance(v, int):
        return v, v
    return int(v[0]), int(v[1])


# ---------------------------------------------------------------------------
# Floating-point parity target: dequantize, then torch CPU fp32 F.linear/F.conv2d
# (dimq_backend/reference.py:91-144; quant/dimq_wrapper.py:189-197,237-240).
# ---------------------------------------------------------------------------

def linear_dequant_reference(x, packed_w, bits, codebook, out_features, in_features, bias=None):
    import torch
    import torch.nn.functional as F

    w_hat = torch.from_numpy(dequantize(packed_w, bits, codebook, out_features, in_features))
    xb = x.detach().cpu().float()
    b = None if bias is None else bias.detach().cpu().float()
    return F.linear(xb, w_hat, b)


def conv2d_dequant_reference(x, packed_w, bits, codebook, weight_shape, bias=None, stride=1, padding=0,
                             dilation=1, groups=1):
    import torch
    import torch.nn.functional as F

    OC = int(weight_shape[0])
    Kr = int(np.prod([int(v) for v in weight_shape[1:]]))
    w_hat = torch.from_numpy(dequantize(packed_w, bits, codebook, OC, Kr)).reshape(
        *[int(v) for v in weight_shape])
    b = None if bias is None else bias.detach().cpu().float()
    return F.conv2d(x.detach().cpu().float(), w_hat, b, _pair(stride), _pair(padding), _pair(dilation), int(groups))


def linear_a4_dequant_reference(x, packed_w, codebook16, scale, zp, out_features, in_features, bias=None):
    """dimq_backend/reference.py:91-110: dequantized A4 activations x dequantized W4."""
    import torch
    import torch.nn.functional as F

    q = quantize_act_u4(x, scale, zp)
    x_hat = np.float32(scale) * (q.astype(np.float32) - np.float32(zp))
    w_hat = dequantize(packed_w, 4, _np(codebook16).astype(np.float32).reshape(-1), out_features, in_features)
    b = None if bias is None else bias.detach().cpu().float()
    return F.linear(torch.from_numpy(x_hat), torch.from_numpy(w_hat), b)


def conv2d_a4_dequant_reference(x, packed_w, codebook16, scale, zp, weight_shape, bias=None, stride=1, padding=0,
                                dilation=1, groups=1):
    """dimq_backend/reference.py:113-144."""
    import torch
    import torch.nn.functional as F

    q = quantize_act_u4(x, scale, zp)
    x_hat = np.float32(scale) * (q.astype(np.float32) - np.float32(zp))
    OC = int(weight_shape[0])
    Kr = int(np.prod([int(v) for v in weight_shape[1:]]))
    w_hat = dequantize(packed_w, 4, _np(codebook16).astype(np.float32).reshape(-1), OC, Kr).reshape(
        *[int(v) for v in weight_shape])
    b = None if bias is None else bias.detach().cpu().float()
    return F.conv2d(torch.from_numpy(x_hat), torch.from_numpy(w_hat), b, _pair(stride), _pair(padding),
                    _pair(dilation), int(groups))


def rel_err(y, ref) -> float:
    """max|y - ref| / max|ref|, the parity metric for floating-point outputs."""
    y = _np(y).astype(np.float64)
    ref = _np(ref).astype(np.float64)
    denom = np.abs(ref).max() if ref.size else 0.0
    if denom == 0.0:
        return float(np.abs(y - ref).max()) if y.size else 0.0
    return float(np.abs(y - ref).max() / denom)



def dequantized_model(qmodel):
    """CPU fp32 copy of a model whose weight-only codebook layers are replaced by
    plain nn.Linear / nn.Conv2d holding W_hat = C[idx] (reference.py:47-56): the
    dequantize-then-F.linear/F.conv2d reference of an end-to-end forward."""
    import copy

    import torch
    import torch.nn as nn

    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear, DIMQLayerNorm, DIMQMaxPool2d

    m = copy.deepcopy(qmodel).cpu().float()
    for name, mod in list(m.named_modules()):
        if isinstance(mod, (DIMQLayerNorm, DIMQMaxPool2d)):  # HIP support ops -> torch's own ops
            if isinstance(mod, DIMQLayerNorm):
                new = nn.LayerNorm(mod.normalized_shape, eps=mod.eps, elementwise_affine=mod.elementwise_affine,
                                   bias=mod.bias is not None)
                new.load_state_dict(mod.state_dict())
            else:
                new = nn.MaxPool2d(mod.kernel_size, mod.stride, mod.padding)
            parent = m
            parts = name.split(".")
            for part in parts[:-1]:
                parent = parent._modules[part]
            parent._modules[parts[-1]] = new
            continue
        if isinstance(mod, DIMQCodebookLinear):
            new = nn.Linear(mod.in_features, mod.out_features, bias=mod.bias is not None)
            w = dequantize(mod.packed_weight, mod.bits, mod.codebook.float(), mod.out_features, mod.in_features)
            new.weight.data = torch.from_numpy(w)
        elif isinstance(mod, DIMQCodebookConv2d):
            oc, cin, kh, kw = mod.weight_shape
            new = nn.Conv2d(cin * mod.groups, oc, (kh, kw), mod.stride, mod.padding, mod.dilation, mod.groups,
                            bias=mod.bias is not None)
            w = dequantize(mod.packed_weight, mod.bits, mod.codebook.float(), oc, cin * kh * kw)
            new.weight.data = torch.from_numpy(w).reshape(oc, cin, kh, kw)
        else:
            continue
        if mod.bias is not None:
            new.bias.data = mod.bias.detach().float().cpu()
        parent = m
        parts = name.split(".")
        for part in parts[:-1]:
            parent = parent._modules[part]
        parent._modules[parts[-1]] = new
    return m.eval()
