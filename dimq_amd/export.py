"""Packed-checkpoint export for DIMQ inference on the HIP backend.

Mirrors ``dimq_backend/export.py`` (reference ``dimq_cuda_backend/dimq_backend/export.py:20-344``):
the same public functions, argument names, errors and the ``dimq_packed_lut``
format.  Export is host-side data preparation, as in the reference: tensors on
a GPU go through the HIP kernels (``dimq_hard_quantize`` / ``dimq_pack_bits`` /
``dimq_unpack_bits``), CPU tensors (a compact checkpoint loaded with
``map_location="cpu"``) through the same arithmetic in torch on the host, so
the exporter also runs where no GPU is visible.  Both give the same bytes
(``tests/test_export.py``).

Format extension (``format_version`` 2), written only when a layer needs it:
``bit_w`` in {2,3,4,8}, ``codebook_granularity`` "per_layer" | "per_channel"
(``codebook`` [K] or [out_channels, K]), ``activation_quantization`` "none"
for weight-only layers, or "codebook" with the layer's ``activation_centers``
(fp32 [Ka]) and ``bit_a`` when the compact layer carries the QAT wrapper's
activation codebook (``quant/export_dimq.py:81-86``), ``weight_encoding``
"packed_lsb_first_indices".  A compact checkpoint whose layers all hold 16
per-layer centres exports to the reference's version-1 layout unchanged (its
uniform u4 activations; ``weight_only=True`` keeps activation codebooks).
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any, Mapping

import torch
import torch.nn as nn

from . import ops

QMIN_U4 = 0
QMAX_U4 = 15
SUPPORTED_BITS = (2, 3, 4, 8)


def bits_for_codebook(n_centers: int) -> int:
    """Smallest supported index width that holds n_centers codes."""
    for b in SUPPORTED_BITS:
        if n_centers <= (1 << b):
            return b
    raise ValueError(f"at most 256 centers are supported, got {n_centers}")


_HOST_CHUNK = 1 << 18  # weights per host argmin pass (bounds its [chunk, K] distance matrix)


@torch.no_grad()
def _nearest_host(w: torch.Tensor, centers: torch.Tensor) -> torch.Tensor:
    """uint8 argmin_c (w - c)^2 (first minimum) of fp32 weights w against one [K] codebook."""
    flat = w.reshape(-1)
    out = torch.empty(flat.shape, dtype=torch.uint8)
    for s in range(0, flat.numel(), _HOST_CHUNK):
        out[s:s + _HOST_CHUNK] = (flat[s:s + _HOST_CHUNK, None] - centers[None, :]).pow(2).argmin(dim=1)
    return out.reshape(w.shape)


@torch.no_grad()
def assign_weight_indices(weight: torch.Tensor, codebook: torch.Tensor) -> torch.Tensor:
    """Nearest learned centre for every weight (export.py:24-35); per-layer codebook of <= 16 entries."""
    centers = codebook.detach().float().reshape(-1)
    if centers.numel() > 16:
        raise ValueError(f"packed u4 export supports at most 16 centers, got {centers.numel()}")
    if centers.numel() == 0:
        raise ValueError("codebook must not be empty")
    w = weight.detach().float()
    if w.is_cuda:
        idx, _ = ops.hard_quantize(w, centers.to(w.device), False)
        return idx.reshape(weight.shape)
    return _nearest_host(w, centers.cpu()).reshape(weight.shape)


@torch.no_grad()
def _pack_host(flat: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first b-bit stream of uint8 indices (index i in bits [b*i, b*i + b)), torch on the host."""
    if bits == 8:
        return flat.clone()
    n = flat.numel()
    nbytes = (n * bits + 7) // 8
    bitv = torch.zeros(nbytes * 8, dtype=torch.uint8)
    bitv[: n * bits] = ((flat[:, None] >> torch.arange(bits, dtype=torch.uint8)) & 1).reshape(-1)
    place = (1 << torch.arange(8, dtype=torch.int32))[None, :]
    return (bitv.reshape(nbytes, 8).to(torch.int32) * place).sum(dim=1).to(torch.uint8)


@torch.no_grad()
def _unpack_host(packed: torch.Tensor, numel: int, bits: int) -> torch.Tensor:
    """Inverse of _pack_host."""
    if bits == 8:
        return packed[:numel].clone()
    bitv = ((packed[:, None] >> torch.arange(8, dtype=torch.uint8)) & 1).reshape(-1)[: numel * bits]
    place = (1 << torch.arange(bits, dtype=torch.int32))[None, :]
    return (bitv.reshape(numel, bits).to(torch.int32) * place).sum(dim=1).to(torch.uint8)


@torch.no_grad()
def pack_u4_indices(indices: torch.Tensor) -> torch.Tensor:
    """``packed[j] = indices[2*j] | (indices[2*j + 1] << 4)`` (export.py:38-55)."""
    return pack_indices(indices, 4)


@torch.no_grad()
def unpack_u4_indices(packed: torch.Tensor, numel: int, *, shape=None) -> torch.Tensor:
    """Inverse of :func:`pack_u4_indices` (export.py:58-78)."""
    return unpack_indices(packed, numel, 4, shape=shape)


@torch.no_grad()
def pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first b-bit packing: index i occupies bits [b*i, b*i+b)."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}, got {bits}")
    flat = indices.detach().contiguous().reshape(-1)
    if flat.numel() == 0:
        return flat.new_empty((0,), dtype=torch.uint8)
    if flat.is_floating_point() or flat.is_complex():
        raise ValueError("indices must be an integer tensor")
    lo, hi = int(flat.min().item()), int(flat.max().item())
    if lo < 0 or hi > (1 << bits) - 1:
        if bits == 4:
            raise ValueError("u4 indices must be in [0, 15]")
        raise ValueError(f"{bits}-bit indices must be in [0, {(1 << bits) - 1}]")
    flat = flat.to(torch.uint8)
    return ops.pack_bits(flat, bits) if flat.is_cuda else _pack_host(flat, bits)


@torch.no_grad()
def unpack_indices(packed: torch.Tensor, numel: int, bits: int, *, shape=None) -> torch.Tensor:
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}, got {bits}")
    flat = packed.detach().contiguous().reshape(-1).to(torch.uint8)
    if numel < 0:
        raise ValueError("numel must be non-negative")
    needed = (numel * bits + 7) // 8
    if flat.numel() < needed:
        raise ValueError(f"packed tensor has {flat.numel()} bytes, expected at least {needed}")
    if numel == 0:
        out = flat.new_empty((0,), dtype=torch.uint8)
    elif flat.is_cuda:
        out = ops.unpack_bits(flat[:needed], numel, bits)
    else:
        out = _unpack_host(flat[:needed], numel, bits)
    if shape is not None:
        out = out.reshape(tuple(shape))
    return out


def activation_qparams_from_minmax(min_val: float, max_val: float, *, qmin: int = QMIN_U4, qmax: int = QMAX_U4,
                                   eps: float = 1e-8) -> dict[str, Any]:
    """Per-tensor uniform affine qparams from an observed range (export.py:81-111)."""
    min_val = float(min_val)
    max_val = float(max_val)
    if not torch.isfinite(torch.tensor([min_val, max_val])).all():
        raise ValueError("activation min/max must be finite")
    if min_val > max_val:
        min_val, max_val = max_val, min_val
    if max_val - min_val < eps:
        scale = 1.0
        zero_point = 0
    else:
        scale = max((max_val - min_val) / float(qmax - qmin), eps)
        zero_point = int(round(qmin - min_val / scale))
        zero_point = max(qmin, min(qmax, zero_point))
    return {"bit_a": 4, "scale": float(scale), "zero_point": int(zero_point), "qmin": int(qmin), "qmax": int(qmax),
            "granularity": "per_tensor"}


def default_activation_qparams() -> dict[str, Any]:
    """Uncalibrated fallback qparams (export.py:114-125)."""
    return {"bit_a": 4, "scale": 1.0, "zero_point": 8, "qmin": QMIN_U4, "qmax": QMAX_U4, "granularity": "per_tensor",
            "source": "default_uncalibrated"}


def load_activation_qparams(path: str | Path) -> dict[str, dict[str, Any]]:
    data = json.loads(Path(path).read_text())
    if not isinstance(data, dict):
        raise ValueError("activation qparams JSON must contain a mapping")
    return {str(key): _normalize_act_qparams(value) for key, value in data.items()}


def infer_module_hparams(model: nn.Module) -> dict[str, dict[str, Any]]:
    """Conv2d/Linear metadata keyed by module name (export.py:137-156)."""
    hparams: dict[str, dict[str, Any]] = {}
    for name, module in model.named_modules():
        if isinstance(module, nn.Conv2d):
            hparams[name] = {
                "type": "conv2d",
                "stride": list(_pair(module.stride)),
                "padding": list(_pair(module.padding)),
                "dilation": list(_pair(module.dilation)),
                "groups": int(module.groups),
                "bias": module.bias.detach().cpu() if module.bias is not None else None,
            }
        elif isinstance(module, nn.Linear):
            hparams[name] = {"type": "linear",
                             "bias": module.bias.detach().cpu() if module.bias is not None else None}
    return hparams


@torch.no_grad()
def export_packed_dimq_checkpoint(
    compact_checkpoint: str | Path | Mapping[str, Any],
    output_path: str | Path,
    *,
    act_qparams: Mapping[str, Mapping[str, Any]] | str | Path | None = None,
    layer_hparams: Mapping[str, Mapping[str, Any]] | None = None,
    model_name: str = "dimq_packed_lut",
    codebook_dtype: torch.dtype = torch.float16,
    weight_only: bool | None = None,
) -> dict[str, Any]:
    """Compact checkpoint -> ``dimq_packed_lut`` (export.py:159-260).

    ``weight_only``: None (default) keeps the reference's W4A4 layout when
    every layer has 16 per-layer centres and writes weight-only layers
    otherwise; True forces weight-only layers; False requires W4A4.
    """
    if isinstance(compact_checkpoint, Mapping):
        compact = dict(compact_checkpoint)
        source_path = None
    else:
        source_path = str(compact_checkpoint)
        compact = torch.load(Path(compact_checkpoint), map_location="cpu", weights_only=True)
    if compact.get("format") != "dimq_compact":
        raise ValueError(f"expected a dimq_compact checkpoint, got {compact.get('format')!r}")

    layers_in = compact["layers"]
    reference_layout = all(torch.as_tensor(l["centers"]).numel() == 16 and torch.as_tensor(l["centers"]).dim() <= 1
                           for l in layers_in.values())
    if weight_only is None:
        weight_only = not reference_layout
    if not weight_only and not reference_layout:
        for name, layer in layers_in.items():
            n = torch.as_tensor(layer["centers"]).numel()
            if n != 16:
                raise ValueError(f"{name} has {n} centers; this W4A4 backend expects 16 learned centers")

    qparams_map = _load_or_normalize_qparams(act_qparams) if not weight_only else {}
    hparams_map = {str(k): dict(v) for k, v in (layer_hparams or {}).items()}
    non_quantized = compact.get("non_quantized_state_dict", {})

    layers: dict[str, dict[str, Any]] = {}
    for name, layer in layers_in.items():
        centers = layer["centers"].detach().float()
        per_channel = centers.dim() == 2 and centers.shape[0] > 1
        if not per_channel:
            centers = centers.reshape(-1)
        n_centers = centers.shape[-1]
        indices = layer["indices"].detach()
        if int(indices.min().item()) < 0 or int(indices.max().item()) >= n_centers:
            if n_centers == 16:
                raise ValueError(f"{name} contains indices outside [0, 15]")
            raise ValueError(f"{name} contains indices outside [0, {n_centers - 1}]")
        bits = 4 if not weight_only else bits_for_codebook(n_centers)
        indices = indices.to(torch.uint8)
        shape = [int(dim) for dim in layer["shape"]]
        layer_type = _infer_layer_type(shape, hparams_map.get(name))
        bias = _find_bias(name, non_quantized, hparams_map.get(name))
        packed = pack_indices(indices, bits).cpu()

        entry: dict[str, Any] = {
            "name": name,
            "type": layer_type,
            "bit_w": bits,
            "weight_shape": shape,
            "weight_numel": int(indices.numel()),
            "packed_weight": packed,
            "packed_indices": packed,
            "codebook": centers.to(dtype=codebook_dtype).cpu(),
            "codebook_granularity": "per_channel" if per_channel else "per_layer",
            "bias": bias.detach().cpu().to(dtype=codebook_dtype) if bias is not None else None,
        }
        if weight_only and layer.get("activation_centers") is not None:
            # the QAT wrapper's activation codebook (quant/export_dimq.py:81-86): kept as is, applied at run time
            ac = torch.as_tensor(layer["activation_centers"]).detach().float().reshape(-1).cpu()
            entry["bit_a"] = int(layer.get("activation_bits", bits_for_codebook(ac.numel())))
            entry["activation_quantization"] = "codebook"
            entry["activation_centers"] = ac
        elif weight_only:
            entry["bit_a"] = None
            entry["activation_quantization"] = "none"
        else:
            aq = _select_qparams(name, qparams_map)
            entry.update({
                "bit_a": 4,
                "act_scale": float(aq["scale"]),
                "act_zero_point": int(aq["zero_point"]),
                "act_qmin": int(aq.get("qmin", QMIN_U4)),
                "act_qmax": int(aq.get("qmax", QMAX_U4)),
                "activation_qparams": aq,
            })
        if layer_type == "linear":
            entry["layout"] = "linear_nk"
            entry["out_features"] = shape[0]
            entry["in_features"] = shape[1]
        else:
            hp = hparams_map.get(name, {})
            entry["layout"] = "conv_kcrs"
            entry["out_channels"] = shape[0]
            entry["in_channels_per_group"] = shape[1]
            entry["kernel_size"] = shape[2:4]
            entry["stride"] = list(_pair(hp.get("stride", (1, 1))))
            entry["padding"] = list(_pair(hp.get("padding", _default_padding(shape))))
            entry["dilation"] = list(_pair(hp.get("dilation", (1, 1))))
            entry["groups"] = int(hp.get("groups", 1))
        layers[name] = entry

    state = {
        "format": "dimq_packed_lut",
        "format_version": 2 if weight_only else 1,
        "model_name": model_name,
        "source_checkpoint": source_path,
        "source_format": compact.get("format"),
        "source_extra": compact.get("extra", {}),
        "model_meta": compact.get("model_meta", {}),
        "quant_cfg": compact.get("quant_cfg", {}),
        "weight_encoding": "packed_lsb_first_indices" if weight_only else "packed_u4_indices",
        "activation_quantization": ("uniform_affine_u4" if not weight_only else
                                    "codebook" if any("activation_centers" in l for l in layers.values()) else "none"),
        "layers": layers,
        "non_quantized_state_dict": non_quantized,
    }
    output_path = Path(output_path)
    output_path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(state, output_path)
    return state


def _pair(value: Any) -> tuple[int, int]:
    if isinstance(value, int):
        return (int(value), int(value))
    if isinstance(value, torch.Size):
        value = tuple(value)
    if isinstance(value, (tuple, list)) and len(value) == 2:
        return (int(value[0]), int(value[1]))
    raise ValueError(f"expected an int or pair, got {value!r}")


def _default_padding(shape: list[int]) -> tuple[int, int]:
    if len(shape) != 4:
        return (0, 0)
    return (int(shape[2]) // 2, int(shape[3]) // 2)


def _infer_layer_type(shape: list[int], hparams: Mapping[str, Any] | None) -> str:
    if hparams and hparams.get("type") in {"conv2d", "linear"}:
        return str(hparams["type"])
    if len(shape) == 2:
        return "linear"
    if len(shape) == 4:
        return "conv2d"
    raise ValueError(f"cannot infer layer type from weight shape {shape}")


def _find_bias(name: str, non_quantized: Mapping[str, torch.Tensor], hparams: Mapping[str, Any] | None):
    if hparams and hparams.get("bias") is not None:
        return hparams["bias"]
    bias = non_quantized.get(f"{name}.bias")
    if bias is not None:
        return bias
    return None


def _load_or_normalize_qparams(qparams) -> dict[str, dict[str, Any]]:
    if qparams is None:
        return {"__default__": default_activation_qparams()}
    if isinstance(qparams, (str, Path)):
        return load_activation_qparams(qparams)
    return {str(key): _normalize_act_qparams(value) for key, value in qparams.items()}


def _select_qparams(name: str, qparams_map: Mapping[str, Mapping[str, Any]]) -> dict[str, Any]:
    if name in qparams_map:
        return _normalize_act_qparams(qparams_map[name])
    if "__default__" in qparams_map:
        return _normalize_act_qparams(qparams_map["__default__"])
    raise KeyError(f"missing activation qparams for layer {name!r}")


def _normalize_act_qparams(value: Mapping[str, Any]) -> dict[str, Any]:
    if "scale" not in value or "zero_point" not in value:
        raise ValueError("activation qparams must include scale and zero_point")
    scale = float(value["scale"])
    if scale <= 0.0:
        raise ValueError("activation scale must be positive")
    zero_point = int(value["zero_point"])
    qmin = int(value.get("qmin", QMIN_U4))
    qmax = int(value.get("qmax", QMAX_U4))
    if qmin != QMIN_U4 or qmax != QMAX_U4:
        raise ValueError("this backend currently supports only u4 activation range [0, 15]")
    if zero_point < qmin or zero_point > qmax:
        raise ValueError("activation zero_point must be in [0, 15]")
    out = dict(value)
    out.update({"bit_a": 4, "scale": scale, "zero_point": zero_point, "qmin": qmin, "qmax": qmax,
                "granularity": value.get("granularity", "per_tensor")})
    return out
