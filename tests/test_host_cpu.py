"""CPU-only checks of the host side: the C-ABI library's exports, its host-only
entry points and error returns, the torch.library registration, and the
host-side codebook initialisation (quant/dimq.py:88-194)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dimq_hip.h"


def _header_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\s*\*)\s+(dimq_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        decls[m.group(1)] = len(params)
    return decls


@pytest.fixture(scope="module")
def capi():
    from dimq_amd import _C
    return _C


def test_header_declares_every_entry_point_the_binding_uses(capi):
    decls = _header_decls()
    assert len(decls) >= 16
    assert set(decls) == set(capi.exported_symbols())
    for name, nargs in decls.items():
        assert len(capi._SIGS[name][1]) == nargs, name


def test_library_exports_every_declared_symbol(capi):
    lib = ctypes.CDLL(str(capi._LIB_PATH))
    for name in _header_decls():
        assert hasattr(lib, name), name


def test_host_only_entry_points(capi):
    lib = capi.lib
    assert lib.dimq_abi_version() == 2
    # LDS-halo layout words: OC * 2 lane groups * ceil(T/4) words-groups * bits, T = KH*KW*C/16,
    # followed by the tap-major layout: OC * C * KH * KW * bits / 32
    assert lib.dimq_conv2d_prepared_words(64, 64, 3, 3, 2) == 64 * 2 * 9 * 2 + 64 * 64 * 9 * 2 // 32
    assert lib.dimq_conv2d_prepared_words(128, 128, 1, 1, 4) == 128 * 2 * 2 * 4 + 128 * 128 * 4 // 32
    assert lib.dimq_conv2d_prepared_words(3, 64, 1, 1, 3) == 20 + 3 * 64 * 3 // 32  # halo part 18 -> 20 words
    assert lib.dimq_conv2d_prepared_words(64, 64, 3, 3, 8) == 0      # bits without a kernel layout
    assert lib.dimq_conv2d_prepared_words(64, 48, 3, 3, 2) == 0      # channels without a kernel layout
    assert lib.dimq_conv2d_prepared_words(64, 64, 5, 5, 2) == 64 * 64 * 25 * 2 // 32   # tap-major GEMM layout
    assert lib.dimq_conv2d_prepared_words(512, 256, 3, 3, 2) == 512 * 256 * 9 * 2 // 32
    assert lib.dimq_conv2d_prepared_words(512, 256, 1, 1, 4) == 512 * 256 * 4 // 32


def test_w4a4_workspace_sizes(capi):
    lib = capi.lib
    F16, F32 = capi.F16, capi.F32
    up = lambda b: (b + 255) // 256 * 256
    # linear_lut: the activations as fp16 a - zp, only for fp16 codebooks
    assert lib.dimq_linear_lut_workspace_bytes(1576, 768, F16) == up(1576 * 768 * 2)
    assert lib.dimq_linear_lut_workspace_bytes(1576, 768, F32) == 0
    assert lib.dimq_linear_lut_workspace_bytes(0, 768, F16) == 0
    # conv2d_lut: the activations + the 4-bit LDS-halo weight layout where the shape has one
    halo_words = 64 * 2 * 9 * 4  # OC * 2 lane groups * ceil(T/4) * bits, T = 9 * 64 / 16
    assert lib.dimq_conv2d_lut_workspace_bytes(32, 64, 56, 56, 64, 64, 3, 3, 1, F16) == \
        up(32 * 64 * 56 * 56 * 2) + halo_words * 4
    assert lib.dimq_conv2d_lut_workspace_bytes(2, 6, 11, 7, 4, 3, 3, 2, 2, F16) == up(2 * 6 * 11 * 7 * 2)
    assert lib.dimq_conv2d_lut_workspace_bytes(32, 64, 56, 56, 64, 64, 3, 3, 1, F32) == 0


def test_linear_workspace_sizes_and_act_codebook_errors(capi):
    lib = capi.lib
    up = lambda b: (b + 255) // 256 * 256
    # below the large-M path (M >= 2048) only the decode shapes (M <= 16) use a workspace
    ws = lib.dimq_linear_codebook_workspace_bytes
    assert ws(1576, 768, 3072, 4, capi.F32) == 0
    assert ws(1576, 768, 3072, 4, capi.BF16) == 0
    assert ws(17, 4096, 4096, 3, capi.BF16) == 0
    # decode GEMV, 4 < M <= 16: bf16 x with K in {1024, 2048, 4096} takes the one-launch bf16 kernel (no
    # workspace); other shapes keep fp32 partial sums of the k splits (k ranges of 1024)
    assert ws(16, 4096, 4096, 3, capi.BF16) == 0
    assert ws(16, 4096, 4096, 3, capi.F16) == up(4 * 16 * 4096 * 4)
    assert ws(9, 8192, 192, 2, capi.F16) == up(8 * 9 * 192 * 4)
    assert ws(9, 8192, 192, 2, capi.BF16) == up(8 * 9 * 192 * 4)
    assert ws(16, 4096, 4000, 3, capi.BF16) == 0   # N % 64 != 0: one k range per work-group
    assert ws(4, 4096, 4096, 3, capi.BF16) == 0    # M <= 4, K 4096: one k range per work-group
    assert ws(4, 8192, 4096, 3, capi.BF16) == up(2 * 4 * 4096 * 4)  # M <= 4: k ranges of 4096
    assert ws(16, 4096, 4096, 8, capi.BF16) == 0
    assert lib.dimq_linear_codebook_act_workspace_bytes(300, 768) == up(300 * 768 * 4)
    assert lib.dimq_linear_codebook_act_workspace_bytes(0, 768) == 0
    args = [None, capi.F32, 4, 64, None, 128, 4, None, capi.F32, 1, 16]
    tail = [None, capi.F32, 8, None, capi.F32, 0, None, 0, None]
    assert lib.dimq_linear_codebook_act(*args, None, 300, *tail) == 1
    assert lib.dimq_last_error() == b"activation codebook must hold between 1 and 256 centres"
    assert lib.dimq_linear_codebook_act(*args, None, 16, *tail) == 1
    assert lib.dimq_last_error() == b"activation codebook is required"


def test_predecode_sizes_and_job_errors(capi):
    """Batched weight pre-decode: bytes per layer (fp16 W_hat, then N fp32 row factors, each 256-byte
    aligned), 0 for layers it cannot decode, and job checks that fail before any launch."""
    import ctypes
    lib = capi.lib
    up = lambda b: (b + 255) // 256 * 256
    assert lib.dimq_codebook_predecode_bytes(768, 768, 4) == up(768 * 768 * 2) + up(768 * 4)
    assert lib.dimq_codebook_predecode_bytes(300, 96, 3) == up(300 * 96 * 2) + up(300 * 4)
    assert lib.dimq_codebook_predecode_bytes(768, 80, 4) == 0      # in_features % 32 != 0
    assert lib.dimq_codebook_predecode_bytes(768, 768, 8) == 0     # 8-bit codebooks are not pre-decoded
    # the large-M fp16 path's workspace is exactly the decoded weights
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 768, 3072, 4, capi.F16) == \
        lib.dimq_codebook_predecode_bytes(3072, 768, 4)
    assert lib.dimq_codebook_predecode_batch(None, 0, None) == 0   # nothing to do, no launch
    job = capi.PredecodeJob(256, 64 * 64, 8, 512, capi.F32, 64, 256, 64, 64, 1024)
    arr = (capi.PredecodeJob * 1)(job)
    assert lib.dimq_codebook_predecode_batch(ctypes.cast(arr, ctypes.c_void_p), 1, None) != 0
    assert b"bits 2-4" in lib.dimq_last_error()
    arr[0].bits, arr[0].cb_size, arr[0].decoded = 4, 16, 1040
    assert lib.dimq_codebook_predecode_batch(ctypes.cast(arr, ctypes.c_void_p), 1, None) != 0
    assert b"256-byte aligned" in lib.dimq_last_error()
    arr[0].decoded, arr[0].cb_rows = 1024, 3
    assert lib.dimq_codebook_predecode_batch(ctypes.cast(arr, ctypes.c_void_p), 1, None) != 0
    assert b"per channel" in lib.dimq_last_error()
    arr[0].cb_rows, arr[0].packed_numel = 64, 100
    assert lib.dimq_codebook_predecode_batch(ctypes.cast(arr, ctypes.c_void_p), 1, None) != 0
    assert b"too small" in lib.dimq_last_error()


def test_support_op_argument_errors(capi):
    lib = capi.lib
    assert lib.dimq_layer_norm(None, capi.F32, 4, 768, 768, None, None, capi.F32, 1e-6, None, None) == 1
    assert lib.dimq_last_error() == b"layer_norm expects fp16 or bf16 input"
    assert lib.dimq_layer_norm(None, capi.BF16, 4, 100, 100, None, None, capi.F32, 1e-6, None, None) == 1
    assert b"multiple of 8" in lib.dimq_last_error()
    assert lib.dimq_layer_norm(None, capi.BF16, 4, 768, 512, None, None, capi.F32, 1e-6, None, None) == 1
    assert b"row stride" in lib.dimq_last_error()
    assert lib.dimq_max_pool2d_nhwc(None, capi.F16, 1, 12, 4, 4, 3, 3, 2, 2, 1, 1, None, None) == 1
    assert b"multiple of 8" in lib.dimq_last_error()
    assert lib.dimq_max_pool2d_nhwc(None, capi.F16, 1, 16, 4, 4, 3, 3, 2, 2, 2, 2, None, None) == 1
    assert lib.dimq_last_error() == b"pad should be at most half of effective kernel size"


def test_argument_errors_return_codes_without_touching_the_gpu(capi):
    lib = capi.lib
    assert lib.dimq_pack_bits(None, 0, 5, None, None) == 2                 # DIMQ_ERR_UNSUPPORTED
    assert b"bits must be one of 2, 3, 4, 8" in lib.dimq_last_error()
    assert lib.dimq_unpack_bits(None, 1, 16, 4, None, None) == 1           # DIMQ_ERR_INVALID
    assert lib.dimq_last_error() == b"packed tensor is too small for requested numel"  # dimq_pack.cu:73
    assert lib.dimq_pack_bits(None, -1, 4, None, None) == 1
    assert lib.dimq_pack_bits(None, 8, 4, None, None) == 1                 # null pointers with numel > 0


def test_ops_have_no_cpu_kernel(capi):
    # the reference registers CUDA impls only (dimq_ops.cpp:46-53): CPU tensors raise a dispatcher error
    with pytest.raises(NotImplementedError):
        torch.ops.dimq.pack_u4(torch.zeros(4, dtype=torch.uint8))
    with pytest.raises(NotImplementedError):
        torch.ops.dimq.unpack_u4(torch.zeros(2, dtype=torch.uint8), 4)


def test_reference_schemas_registered_verbatim(capi):
    # dimq_cuda_backend/csrc/dimq_ops.cpp:37-42
    schemas = {
        "pack_u4": "pack_u4(Tensor indices) -> Tensor",
        "unpack_u4": "unpack_u4(Tensor packed, int numel) -> Tensor",
        "quantize_activation_u4": "quantize_activation_u4(Tensor x, float act_scale, int act_zp) -> Tensor",
        "build_product_table": "build_product_table(Tensor codebook, float act_scale, int act_zp) -> Tensor",
        "linear_lut": "linear_lut(Tensor x, Tensor packed_w, Tensor codebook, float act_scale, int act_zp, "
                      "Tensor? bias, int out_features, int in_features) -> Tensor",
        "conv2d_lut": "conv2d_lut(Tensor x, Tensor packed_w, Tensor codebook, float act_scale, int act_zp, "
                      "Tensor? bias, int out_channels, int in_channels_per_group, int kernel_h, int kernel_w, "
                      "int stride_h, int stride_w, int pad_h, int pad_w, int dilation_h, int dilation_w, "
                      "int groups) -> Tensor",
    }
    for name, schema in schemas.items():
        got = str(getattr(torch.ops.dimq, name).default._schema)
        assert got.replace("dimq::", "") == schema


def test_extension_module_functions_match_the_schemas(capi):
    """csrc/dimq_ops.cpp:55-62: the extension also exposes the six ops as module-level functions taking the
    schema's arguments in order; a CPU tensor gets the CUDA-only error, as from the compiled extension."""
    import inspect
    for name in ("pack_u4", "unpack_u4", "quantize_activation_u4", "build_product_table", "linear_lut",
                 "conv2d_lut"):
        fn = getattr(capi, name)
        schema = getattr(torch.ops.dimq, name).default._schema
        assert list(inspect.signature(fn).parameters) == [a.name for a in schema.arguments], name
    with pytest.raises(RuntimeError, match="pack_u4 expects a CUDA tensor"):
        capi.pack_u4(torch.zeros(4, dtype=torch.uint8))


# ---------------------------------------------------------------------------
# codebook initialisation (host)
# ---------------------------------------------------------------------------

def test_quantile_centers_closed_form():
    from dimq_amd.codebook import init_centers_1d
    w = torch.arange(5, dtype=torch.float32)            # quantiles at 1/4, 1/2, 3/4 -> 1, 2, 3
    c = init_centers_1d(w, 3, "quantile")
    assert torch.allclose(c, torch.tensor([1.0, 2.0, 3.0]), atol=1e-6)


def test_postprocess_spreads_duplicate_centers_and_keeps_mean():
    from dimq_amd.codebook import init_centers_1d
    g = torch.Generator().manual_seed(7)
    w = torch.randn(147, generator=g)                  # ResNet stem row: 256 centres > 147 weights
    c = init_centers_1d(w, 256, "quantile")
    q = torch.quantile(w, torch.linspace(0, 1, 258)[1:-1])
    assert c.shape == (256,)
    assert bool((c[1:] > c[:-1]).all())                # strictly increasing after the min-gap pass
    assert abs(float(c.mean() - q.mean())) < 1e-6      # re-centred on the quantiles' mean
    gap = float(torch.maximum(w.max() - w.min(), w.std(unbiased=False))) * 1e-6
    assert float((c[1:] - c[:-1]).min()) >= gap * 0.5


def test_constant_row_min_gap_behaviour():
    from dimq_amd.codebook import init_centers_1d
    # span = sigma = 0 -> min_gap = 1e-6 * 1e-6 = 1e-12 (quant/dimq.py:182-190)
    c0 = init_centers_1d(torch.zeros(10), 4, "quantile")
    assert bool((c0[1:] > c0[:-1]).all())
    assert torch.allclose(c0[1:] - c0[:-1], torch.full((3,), 1e-12), rtol=1e-3, atol=0)
    assert abs(float(c0.mean())) < 1e-15
    # at 0.25 the 1e-12 gap is below fp32 resolution: the centres stay equal, as in the reference
    c1 = init_centers_1d(torch.full((10,), 0.25), 4, "quantile")
    assert torch.equal(c1, torch.full((4,), 0.25))


def test_per_channel_init_rows():
    from dimq_amd.codebook import init_centers_per_channel
    g = torch.Generator().manual_seed(3)
    w = torch.randn(48, 16, 3, 3, generator=g) * 0.05
    w[5] = 0.125                                       # a constant row: every quantile equal
    w[9, 0, 0, 0] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        init_centers_per_channel(w, 4)
    w[9, 0, 0, 0] = 0.0
    pc = init_centers_per_channel(w, 4)
    rows = w.reshape(48, -1)
    q = torch.quantile(rows, torch.linspace(0, 1, 6)[1:-1], dim=1).T
    live = [r for r in range(48) if r != 5]
    # distinct quantiles: the spread is a no-op, the codebook is torch.quantile's
    assert torch.equal(pc[live], q[live])
    # constant row: gap = 1e-6 * max(span, std) clamped to 1e-6 -> 1e-12, below fp32 resolution at 0.125
    assert torch.equal(pc[5], torch.full((4,), 0.125))


def test_init_rejects_other_initialisers():
    from dimq_amd.codebook import init_centers_1d, init_centers_per_channel
    with pytest.raises(ValueError, match="quantile"):
        init_centers_1d(torch.randn(10), 3, "kmeans")
    with pytest.raises(ValueError, match="quantile"):
        init_centers_per_channel(torch.randn(4, 10), 3, "linspace_minmax")


def test_init_subsamples_large_tensors_with_randperm():
    from dimq_amd.codebook import init_centers_1d
    g = torch.Generator().manual_seed(11)
    w = torch.randn(250_000, generator=g)
    torch.manual_seed(123)
    c = init_centers_1d(w, 8, "quantile")
    torch.manual_seed(123)
    sample = w[torch.randperm(w.numel())[:200_000]]    # quant/dimq.py:111-113
    assert torch.equal(c, torch.quantile(sample, torch.linspace(0, 1, 10)[1:-1]))


def test_benchmark_cuda_needs_a_gpu():
    """benchmark_cuda (dimq_backend/benchmark.py:10-26) times with HIP events; without a GPU it raises."""
    from dimq_amd.benchmark import benchmark_cuda
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible (the GPU test covers the timing)")
    with pytest.raises(RuntimeError, match="GPU"):
        benchmark_cuda(lambda: None, warmup=1, repeat=1)
