"""dimq_amd — MI355X (gfx950) HIP backend for DIMQ packed-index inference.

Public API mirrors ``dimq_backend/__init__.py`` of the reference
(``dimq_cuda_backend/dimq_backend/__init__.py:3-37``), plus the weight-only,
b-bit, per-channel codebook layers and ops.  The CPU reference functions of
the reference package (``dimq_linear_reference`` ...) are test oracles and
live in ``oracle/``, not here.
"""

from .export import (
    activation_qparams_from_minmax,
    assign_weight_indices,
    bits_for_codebook,
    default_activation_qparams,
    export_packed_dimq_checkpoint,
    infer_module_hparams,
    load_activation_qparams,
    pack_indices,
    pack_u4_indices,
    unpack_indices,
    unpack_u4_indices,
)
from .modules import (
    DIMQCodebookConv2d,
    DIMQCodebookLinear,
    DIMQConv2d,
    DIMQLinear,
    make_packed_layer,
    quantize_model_weight_only,
    replace_modules_with_packed_dimq,
)
from .ops import build_product_table, is_available, quantize_activation_u4
from .codebook import hard_quantize_weight, init_centers_1d, init_centers_per_channel

__all__ = [
    "DIMQCodebookConv2d",
    "DIMQCodebookLinear",
    "DIMQConv2d",
    "DIMQLinear",
    "activation_qparams_from_minmax",
    "assign_weight_indices",
    "bits_for_codebook",
    "build_product_table",
    "default_activation_qparams",
    "export_packed_dimq_checkpoint",
    "hard_quantize_weight",
    "infer_module_hparams",
    "init_centers_1d",
    "init_centers_per_channel",
    "is_available",
    "load_activation_qparams",
    "make_packed_layer",
    "pack_indices",
    "pack_u4_indices",
    "quantize_activation_u4",
    "quantize_model_weight_only",
    "replace_modules_with_packed_dimq",
    "unpack_indices",
    "unpack_u4_indices",
]
