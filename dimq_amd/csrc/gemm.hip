// Host side of the codebook Linear: argument checks (with the reference's
// messages where one exists, csrc/dimq_gemm_lut.cu:66-79), tile selection and
// launch.
#include <mutex>

#include "gemm_big.h"
#include "gemm_kernel.h"
#include "gemv_fast.h"

namespace dimq {
namespace {

constexpr int64_t kCUs = 256;

}  // namespace

// gemm_pd.hip: the pre-decoded-weight path for large M (weights decoded once
// per call into the workspace, then an fp16 GEMM fed by global_load_lds).
int64_t predecoded_ws_bytes(int64_t M, int64_t K, int64_t N, int bits, int x_dtype);
int launch_predecoded(const GemmArgs& p, int bits, int x_dtype, void* ws, int64_t ws_bytes, hipStream_t s,
                      const void* decoded = nullptr);
int64_t predecoded_w_bytes(int64_t N, int64_t K, int bits);
int launch_predecode_jobs(const DimqPredecodeJob* jobs, int count, hipStream_t s);

// Fast-path tiles need K % 128 == 0, aligned rows/streams and a Linear layout.
int gemm_fast_tile(int tile, const GemmArgs& p, int bits) {
  if (bits == 8 || p.conv || !p.fast_b || !p.vec_a || p.K % kKM != 0) return tile;
  if (tile == kTile128x64) return kTileFast128x64;
  if (tile == kTile64x32) return kTileFast64x32;
  return tile;
}

// Large-tile kernels (gemm_big.h) for Linear shapes with M > 64, K % 64 == 0
// and aligned rows/streams.  Measured on the ViT-B/16 shapes (M = 12,608) and
// cfg1: the deep-pipeline tile (7, 64x128) is fastest for K < 2048, the 2x2
// 128x128 tile (2) for K >= 2048.  Returns -1 when the shape does not qualify.
int gemm_big_tile(const GemmArgs& p, int bits, int x_dtype, int variant) {
  if (variant == DIMQ_VARIANT_SMALL_M || p.conv || !(bits == 2 || bits == 3 || bits == 4)) return -1;
  const int mode = epi_mode(p.epi);  // epilogues the large tiles are instantiated for
  const bool qmode = x_dtype == DIMQ_F16 && (mode == kEpiQuant || mode == (kEpiRelu | kEpiQuant) ||
                                             mode == (kEpiGelu | kEpiQuant));
  if (!(mode == kEpiNone || mode == kEpiRelu || mode == kEpiGelu || mode == kEpiRes || qmode)) return -1;
  if (p.M <= 64 || p.K % 64 != 0 || !p.fast_b || !p.vec_a) return -1;
  // 256x256 shared-decode tiles for large M (measured on the ViT-B/16 shapes at
  // M 12,608, bf16: qkv 84 vs 104 us, proj 40 vs 50, fc1 114 vs 134, fc2 104 vs
  // 133 against the best 128x128 tile); below M 2048 the 128x128 tiles fill
  // the CUs better (M 1000: 17 vs 30 us).
  if (p.M >= 2048 && x_dtype != DIMQ_F32) return 10;  // fp32 activations spill its registers
  return p.K >= 2048 ? 2 : 7;
}

int gemm_pick_tile(int64_t M, int64_t N, int variant) {
  if (variant == DIMQ_VARIANT_SMALL_M) return M <= 16 ? kTileGemv : kTile16x16;
  if (variant == DIMQ_VARIANT_AUTO && M <= 16) return kTileGemv;
  const int64_t big = ((M + 127) / 128) * ((N + 255) / 256);
  if (big >= kCUs) return kTile128x64;
  return kTile64x32;
}

namespace {

template <bool A4>
int dispatch(const GemmArgs& p, int bits, int xt, int tile, hipStream_t s) {
#define DIMQ_XT_CASES(B)                                                   \
  switch (xt) {                                                            \
    case DIMQ_F32: return launch_gemm_tile<B, DIMQ_F32, A4>(p, tile, s);   \
    case DIMQ_F16: return launch_gemm_tile<B, DIMQ_F16, A4>(p, tile, s);   \
    case DIMQ_BF16: return launch_gemm_tile<B, DIMQ_BF16, A4>(p, tile, s); \
  }                                                                        \
  break;
  if constexpr (A4) {
    switch (xt) {
      case DIMQ_F32: return launch_gemm_tile<4, DIMQ_F32, true>(p, tile, s);
      case DIMQ_F16: return launch_gemm_tile<4, DIMQ_F16, true>(p, tile, s);
      case DIMQ_BF16: return launch_gemm_tile<4, DIMQ_BF16, true>(p, tile, s);
      case DIMQ_F64: return launch_gemm_tile<4, DIMQ_F64, true>(p, tile, s);
    }
  } else {
    switch (bits) {
      case 2: DIMQ_XT_CASES(2)
      case 3: DIMQ_XT_CASES(3)
      case 4: DIMQ_XT_CASES(4)
      case 8: DIMQ_XT_CASES(8)
    }
  }
#undef DIMQ_XT_CASES
  return set_error(DIMQ_ERR_UNSUPPORTED, "unsupported dtype/bit-width combination (x dtype %d, bits %d)", xt, bits);
}

}  // namespace

int gemm_dispatch(const GemmArgs& p, int bits, int xt, bool a4, int tile, hipStream_t s) {
  return a4 ? dispatch<true>(p, bits, xt, tile, s) : dispatch<false>(p, bits, xt, tile, s);
}

int linear_codebook_impl(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed_w,
                         int bits, const void* codebook, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                         const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype, int64_t ldy,
                         const Epi& epi, int variant, hipStream_t s, float acc_scale = 1.0f,
                         void* workspace = nullptr, int64_t workspace_bytes = 0, const void* decoded = nullptr) {
  GemmArgs p{};
  p.epi = epi;
  p.acc_scale = acc_scale;
  p.x = x;
  p.M = M;
  p.K = K;
  p.ldx = ldx;
  p.w = packed_w;
  p.N = N;
  p.cb = codebook;
  p.cb_dt = cb_dtype;
  p.cb_rows = cb_rows;
  p.cb_size = static_cast<int>(cb_size);
  p.bias = bias;
  p.bias_dt = bias_dtype;
  p.y = y;
  p.y_dt = y_dtype;
  p.ldy = ldy;
  p.act_scale = 1.0f;
  p.act_zp = 0;
  p.fast_b = (K % 32 == 0) && aligned(packed_w, 16);
  const int xs = dtype_size(x_dtype);
  p.vec_a = aligned(x, 16) && ((ldx * xs) % 16 == 0);
  p.groups = 1;
  if (M == 0 || N == 0) return DIMQ_OK;
  if ((workspace != nullptr || decoded != nullptr) && variant != DIMQ_VARIANT_SMALL_M) {
    const int rc = launch_predecoded(p, bits, x_dtype, workspace, workspace_bytes, s, decoded);
    if (rc >= 0) return rc;
  }
  const int big = gemm_big_tile(p, bits, x_dtype, variant);
  if (big >= 0) {
    switch (bits) {
      case 2: return launch_big_b2(p, x_dtype, big, s);
      case 3: return launch_big_b3(p, x_dtype, big, s);
      default: return launch_big_b4(p, x_dtype, big, s);
    }
  }
  int tile = gemm_fast_tile(gemm_pick_tile(M, N, variant), p, bits);
  if (tile < 0 || tile >= kTileCount) tile = gemm_pick_tile(M, N, variant);
  if (tile >= kTileFast128x64 && gemm_fast_tile(kTile64x32, p, bits) == kTile64x32) tile = gemm_pick_tile(M, N, variant);
  if (tile == kTileGemv && (M > 16 || bits == 8)) tile = gemm_pick_tile(M, N, DIMQ_VARIANT_MFMA);
  // 8-bit: 16-row tiles when the 64-row ones would leave most CUs idle
  // (ResNet-18 fc, M 128 x N 1000: 32 work-groups on 64-row tiles, 128 on
  // 16-row tiles; measured 28.9 -> 23.4 us per call)
  if (bits == 8 && tile == kTile64x32 && ((M + 63) / 64) * ((N + 63) / 64) < kCUs / 2) tile = kTile16x16;
  if (tile == kTileGemv && gemv_direct_ok(p, bits, x_dtype)) {
    switch (bits) {
      case 2: return launch_gemv_direct<2>(p, s);
      case 3: return launch_gemv_direct<3>(p, s);
      default: return launch_gemv_direct<4>(p, s);
    }
  }
  if (tile == kTileGemv) {
    const bool ws_ok = workspace != nullptr && aligned(workspace, 16);
    GemvPlan pl;
    bool planned = gemv_plan(p, bits, ws_ok, pl);
    if (planned && gemv_partial_bytes(p, pl) > (ws_ok ? workspace_bytes : 0)) planned = gemv_plan(p, bits, false, pl);
    if (planned) {
      float* part = static_cast<float*>(workspace);
      switch (bits) {
        case 2: return launch_gemv_stream<2>(p, x_dtype, pl, part, s);
        case 3: return launch_gemv_stream<3>(p, x_dtype, pl, part, s);
        default: return launch_gemv_stream<4>(p, x_dtype, pl, part, s);
      }
    }
  }
  return dispatch<false>(p, bits, x_dtype, tile, s);
}

}  // namespace dimq

using namespace dimq;

static int linear_codebook_checked(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                   int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                                   int64_t cb_size, const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                                   const void* residual, int residual_dtype, int activation, int variant, void* stream,
                                   void* workspace, int64_t workspace_bytes, const void* decoded = nullptr);

extern "C" int dimq_linear_codebook(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                    int64_t packed_numel, int bits, const void* codebook, int cb_dtype,
                                    int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype, int64_t N,
                                    void* y, int y_dtype, int variant, void* stream) {
  return dimq_linear_codebook_ex(x, x_dtype, M, K, packed_w, packed_numel, bits, codebook, cb_dtype, cb_rows, cb_size,
                                 bias, bias_dtype, N, y, y_dtype, nullptr, 0, DIMQ_ACT_NONE, variant, stream);
}

// Workspace of dimq_linear_codebook_ex_ws: the decode shapes (M <= 16)
// whose k range is split over work-groups keep their fp32 partial sums there;
// large-M shapes with fp16 activations keep the weights decoded to fp16.
extern "C" int64_t dimq_linear_codebook_workspace_bytes(int64_t M, int64_t K, int64_t N, int bits, int x_dtype) {
  const int64_t pd = predecoded_ws_bytes(M, K, N, bits, x_dtype);
  if (pd > 0) return pd;
  if (M <= 0 || M > 16 || K <= 0 || N <= 0 || !(bits == 2 || bits == 3 || bits == 4)) return 0;
  GemmArgs p{};
  p.M = M;
  p.K = K;
  p.N = N;
  p.fast_b = p.vec_a = true;
  if (gemv_direct_ok(p, bits, x_dtype)) return 0;  // no split k
  GemvPlan pl;
  if (!gemv_plan(p, bits, true, pl)) return 0;
  return (gemv_partial_bytes(p, pl) + 255) / 256 * 256;
}

extern "C" int dimq_linear_codebook_ex_ws(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                          int64_t packed_numel, int bits, const void* codebook, int cb_dtype,
                                          int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype,
                                          int64_t N, void* y, int y_dtype, const void* residual, int residual_dtype,
                                          int activation, int variant, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  DIMQ_CHECK(workspace_bytes >= 0, "workspace_bytes must be non-negative");
  const bool decode = (M >= 1 && M <= 16) || predecoded_ws_bytes(M, K, N, bits, x_dtype) > 0;
  return linear_codebook_checked(x, x_dtype, M, K, packed_w, packed_numel, bits, codebook, cb_dtype, cb_rows, cb_size,
                                 bias, bias_dtype, N, y, y_dtype, residual, residual_dtype, activation, variant,
                                 stream, decode ? workspace : nullptr, decode ? workspace_bytes : 0);
}

extern "C" int64_t dimq_codebook_predecode_bytes(int64_t out_features, int64_t in_features, int bits) {
  return predecoded_w_bytes(out_features, in_features, bits);
}

extern "C" int dimq_codebook_predecode_batch(const DimqPredecodeJob* jobs, int count, void* stream) {
  DIMQ_CHECK(count >= 0 && (count == 0 || jobs != nullptr), "jobs must hold count entries");
  for (int j = 0; j < count; ++j) {
    const DimqPredecodeJob& J = jobs[j];
    if (predecoded_w_bytes(J.out_features, J.in_features, J.bits) == 0)
      return set_error(DIMQ_ERR_UNSUPPORTED, "job %d: pre-decode needs bits 2-4 and in_features %% 32 == 0", j);
    DIMQ_CHECK(J.packed_w != nullptr && J.codebook != nullptr && J.decoded != nullptr, "job %d: null pointer", j);
    DIMQ_CHECK(aligned(J.packed_w, 16), "job %d: packed_w must be 16-byte aligned", j);
    DIMQ_CHECK(aligned(J.decoded, 256), "job %d: decoded must be 256-byte aligned", j);
    DIMQ_CHECK(is_float_dtype(J.cb_dtype), "job %d: codebook must be floating point", j);
    DIMQ_CHECK(J.cb_rows == 1 || J.cb_rows == J.out_features,
               "job %d: codebook must have 1 (per layer) or out_features (per channel) rows", j);
    DIMQ_CHECK(J.cb_size >= 1 && J.cb_size <= (1 << J.bits), "job %d: codebook rows must hold 1 to 2^bits entries", j);
    DIMQ_CHECK(J.packed_numel >= (J.out_features * J.in_features * J.bits + 7) / 8,
               "job %d: packed_weight is too small for out_features * in_features", j);
  }
  return launch_predecode_jobs(jobs, count, as_stream(stream));
}

extern "C" int dimq_linear_codebook_predecoded(const void* x, int x_dtype, int64_t M, int64_t K,
                                               const uint8_t* packed_w, int64_t packed_numel, int bits,
                                               const void* codebook, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                                               const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                                               const void* residual, int residual_dtype, int activation, int variant,
                                               const void* decoded, void* workspace, int64_t workspace_bytes,
                                               void* stream) {
  DIMQ_CHECK(workspace_bytes >= 0, "workspace_bytes must be non-negative");
  DIMQ_CHECK(decoded == nullptr || aligned(decoded, 256), "decoded must be 256-byte aligned");
  const bool decode = (M >= 1 && M <= 16) || predecoded_ws_bytes(M, K, N, bits, x_dtype) > 0;
  return linear_codebook_checked(x, x_dtype, M, K, packed_w, packed_numel, bits, codebook, cb_dtype, cb_rows, cb_size,
                                 bias, bias_dtype, N, y, y_dtype, residual, residual_dtype, activation, variant,
                                 stream, decode ? workspace : nullptr, decode ? workspace_bytes : 0, decoded);
}

extern "C" int64_t dimq_linear_codebook_act_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return (M * K * 4 + 255) / 256 * 256;
}

// Activations replaced by their nearest activation-codebook centre in x's
// dtype (centers[idx].to(x.dtype), quant/dimq.py:217; one element-wise pass
// into the workspace), then the weight-codebook tiles on them, under their
// fp16 range guard: the dequantize-then-MFMA form of the weight x activation
// codebook product.
extern "C" int dimq_linear_codebook_act(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                        int64_t packed_numel, int bits, const void* codebook, int cb_dtype,
                                        int64_t cb_rows, int64_t cb_size, const float* act_centers, int64_t n_act,
                                        const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype, int variant,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  DIMQ_CHECK(x_dtype == DIMQ_F32 || x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16,
             "linear_codebook_act expects fp32, fp16 or bf16 input");
  DIMQ_CHECK(n_act >= 1 && n_act <= 256, "activation codebook must hold between 1 and 256 centres");
  DIMQ_CHECK(act_centers != nullptr, "activation codebook is required");
  DIMQ_CHECK(M >= 0 && N > 0 && K > 0, "linear dimensions must be positive");
  if (M == 0) return DIMQ_OK;
  const int64_t need = dimq_linear_codebook_act_workspace_bytes(M, K);
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= need && aligned(workspace, 16),
             "workspace must be 16-byte aligned and hold dimq_linear_codebook_act_workspace_bytes bytes");
  // DIMQ_VARIANT_SMALL_M: activation indices into the workspace, then the
  // index x index LUT gather (the weight and activation codebooks' product
  // table formed per work-group); otherwise the dequantize-then-GEMM form,
  // the faster one on MI355X at every M
  const bool gather = variant == DIMQ_VARIANT_SMALL_M && lut_act_supported(M, K, bits, cb_rows, n_act) &&
                      aligned(packed_w, 4) && is_float_dtype(cb_dtype) && (cb_rows == 1 || cb_rows == N) &&
                      cb_size >= 1 && cb_size <= (1 << bits) && packed_numel >= (N * K * bits + 7) / 8;
  if (gather) {
    uint8_t* idx = static_cast<uint8_t*>(workspace);
    int r = dimq_hard_quantize(x, x_dtype, 1, M * K, act_centers, n_act, 0, idx, nullptr, stream);
    if (r != DIMQ_OK) return r;
    DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
    DIMQ_CHECK(y_dtype == DIMQ_F32 || y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16,
               "linear_codebook output dtype must be fp32, fp16 or bf16");
    return launch_lut_act(idx, M, K, packed_w, bits, codebook, cb_dtype, cb_rows, cb_size, act_centers, n_act, x_dtype,
                          bias, bias_dtype, N, y, y_dtype, /*clamp=*/false, as_stream(stream));
  }
  const int rc = launch_act_codebook(x, x_dtype, M * K, act_centers, static_cast<int>(n_act), workspace,
                                     as_stream(stream));
  if (rc != DIMQ_OK) return rc;
  return dimq_linear_codebook_ex(workspace, x_dtype, M, K, packed_w, packed_numel, bits, codebook, cb_dtype, cb_rows, cb_size,
                                 bias, bias_dtype, N, y, y_dtype, nullptr, 0, DIMQ_ACT_NONE, variant, stream);
}

extern "C" int dimq_linear_codebook_ex(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                       int64_t packed_numel, int bits, const void* codebook, int cb_dtype,
                                       int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype, int64_t N,
                                       void* y, int y_dtype, const void* residual, int residual_dtype,
                                       int activation, int variant, void* stream) {
  return linear_codebook_checked(x, x_dtype, M, K, packed_w, packed_numel, bits, codebook, cb_dtype, cb_rows, cb_size,
                                 bias, bias_dtype, N, y, y_dtype, residual, residual_dtype, activation, variant, stream,
                                 nullptr, 0);
}

// Argument checks of the weight-only Linear, then the kernels; `workspace`
// (nullable) may hold the decode GEMV's split-k partial sums.
static int linear_codebook_checked(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                   int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                                   int64_t cb_size, const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                                   const void* residual, int residual_dtype, int activation, int variant, void* stream,
                                   void* workspace, int64_t workspace_bytes, const void* decoded) {
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 8))
    return set_error(DIMQ_ERR_UNSUPPORTED, "bits must be one of 2, 3, 4, 8 (got %d)", bits);
  DIMQ_CHECK(x_dtype == DIMQ_F32 || x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16,
             "linear_codebook expects fp32, fp16 or bf16 input");
  DIMQ_CHECK(y_dtype == DIMQ_F32 || y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16,
             "linear_codebook output dtype must be fp32, fp16 or bf16");
  DIMQ_CHECK(is_float_dtype(cb_dtype), "codebook must be floating point");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  DIMQ_CHECK(M >= 0 && N > 0 && K > 0, "linear dimensions must be positive");
  DIMQ_CHECK(cb_rows == 1 || cb_rows == N, "codebook must have 1 (per layer) or out_features (per channel) rows");
  DIMQ_CHECK(cb_size >= 1 && cb_size <= (1 << bits), "codebook rows must hold between 1 and 2^bits entries");
  DIMQ_CHECK(packed_numel >= (N * K * bits + 7) / 8, "packed_weight is too small for out_features * in_features");
  DIMQ_CHECK(variant >= DIMQ_VARIANT_AUTO && variant <= DIMQ_VARIANT_MFMA, "unknown kernel variant %d", variant);
  DIMQ_CHECK(residual == nullptr || is_float_dtype(residual_dtype), "residual must be floating point");
  DIMQ_CHECK(activation >= DIMQ_ACT_NONE && activation <= DIMQ_ACT_GELU, "unknown activation %d", activation);
  const Epi epi{residual, residual_dtype, activation, residual != nullptr && aligned(residual, 16)};
  return linear_codebook_impl(x, x_dtype, M, K, K, packed_w, bits, codebook, cb_dtype, cb_rows, cb_size, bias,
                              bias_dtype, N, y, y_dtype, N, epi, variant, as_stream(stream), 1.0f, workspace,
                              workspace_bytes, decoded);
}

extern "C" int64_t dimq_linear_lut_workspace_bytes(int64_t M, int64_t in_features, int cb_dtype) {
  if (cb_dtype != DIMQ_F16 || M <= 0 || in_features <= 0) return 0;
  return (M * in_features * 2 + 255) / 256 * 256;
}

extern "C" int dimq_linear_lut(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                               const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale,
                               int64_t act_zp, const void* bias, int bias_dtype, int64_t bias_numel,
                               int64_t out_features, int64_t in_features, float* y, void* stream) {
  return dimq_linear_lut_ws(x, x_dtype, M, packed_w, packed_numel, codebook, cb_dtype, cb_numel, act_scale, act_zp,
                            bias, bias_dtype, bias_numel, out_features, in_features, y, nullptr, 0, stream);
}

// With an fp16 codebook (the reference exporter's default, export.py
// codebook_dtype) and a workspace of M*K fp16: the activations become the
// exact fp16 integers a - zp (one element-wise pass), then the weight-only
// kernels run on them with the 16-entry codebook and act_scale on the
// accumulator, so the call takes the same fast tiles as linear_codebook.
// Otherwise the generic A4 tiles (hi + lo fp16 codebook planes).
// Argument checks of linear_lut, with the messages of the reference's
// TORCH_CHECKs (csrc/dimq_gemm_lut.cu:66-79).
static int check_linear_lut(int x_dtype, int64_t M, int64_t packed_numel, int cb_dtype, int64_t cb_numel,
                            double act_scale, int64_t act_zp, const void* bias, int bias_dtype, int64_t bias_numel,
                            int64_t out_features, int64_t in_features) {
  DIMQ_CHECK(is_float_dtype(x_dtype), "linear_lut expects floating input");
  DIMQ_CHECK(is_float_dtype(cb_dtype), "codebook must be floating point");
  DIMQ_CHECK(cb_numel == 16, "codebook must have 16 entries for W4");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  DIMQ_CHECK(act_zp >= 0 && act_zp <= 15, "act_zero_point must be in [0, 15]");
  DIMQ_CHECK(out_features > 0 && in_features > 0, "linear dimensions must be positive");
  DIMQ_CHECK(M >= 0, "input numel must be divisible by in_features");
  DIMQ_CHECK(packed_numel >= (out_features * in_features + 1) / 2,
             "packed_weight is too small for out_features * in_features");
  if (bias) DIMQ_CHECK(bias_numel == out_features, "bias numel must equal out_features");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  return DIMQ_OK;
}

extern "C" int dimq_linear_lut_ws(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w,
                                  int64_t packed_numel, const void* codebook, int cb_dtype, int64_t cb_numel,
                                  double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                                  int64_t bias_numel, int64_t out_features, int64_t in_features, float* y,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  const int rc0 = check_linear_lut(x_dtype, M, packed_numel, cb_dtype, cb_numel, act_scale, act_zp, bias, bias_dtype,
                                   bias_numel, out_features, in_features);
  if (rc0 != DIMQ_OK) return rc0;
  DIMQ_CHECK(workspace_bytes >= 0, "workspace_bytes must be non-negative");
  if (M == 0) return DIMQ_OK;
  const int64_t need = dimq_linear_lut_workspace_bytes(M, in_features, cb_dtype);
  if (workspace != nullptr && need > 0 && workspace_bytes >= need && aligned(workspace, 16)) {
    uint16_t* q = static_cast<uint16_t*>(workspace);
    const hipStream_t st = as_stream(stream);
    const int rc = launch_quantize_a4_f16(x, x_dtype, M * in_features, static_cast<float>(act_scale),
                                          static_cast<int>(act_zp), q, st);
    if (rc != DIMQ_OK) return rc;
    return linear_codebook_impl(q, DIMQ_F16, M, in_features, in_features, packed_w, 4, codebook, cb_dtype, 1, 16,
                                bias, bias_dtype, out_features, y, DIMQ_F32, out_features, Epi{}, DIMQ_VARIANT_AUTO,
                                st, static_cast<float>(act_scale));
  }
  GemmArgs p{};
  p.x = x;
  p.M = M;
  p.K = in_features;
  p.ldx = in_features;
  p.w = packed_w;
  p.N = out_features;
  p.cb = codebook;
  p.cb_dt = cb_dtype;
  p.cb_rows = 1;
  p.cb_size = 16;
  p.bias = bias;
  p.bias_dt = bias_dtype;
  p.y = y;
  p.y_dt = DIMQ_F32;
  p.ldy = out_features;
  p.act_scale = static_cast<float>(act_scale);
  p.act_zp = static_cast<int>(act_zp);
  p.fast_b = (in_features % 32 == 0) && aligned(packed_w, 16);
  p.vec_a = aligned(x, 16) && ((in_features * dtype_size(x_dtype)) % 16 == 0);
  p.groups = 1;
  const int tile = (x_dtype != DIMQ_F64) ? gemm_fast_tile(kTile64x32, p, 4) : kTile64x32;
  return dispatch<true>(p, 4, x_dtype, tile, as_stream(stream));
}

extern "C" int dimq_linear_lut_q(const uint16_t* xq, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                                 const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale,
                                 const void* bias, int bias_dtype, int64_t bias_numel, int64_t out_features,
                                 int64_t in_features, int activation, double out_act_scale, int64_t out_act_zp,
                                 void* y, int y_dtype, void* stream) {
  int rc = check_linear_lut(DIMQ_F16, M, packed_numel, cb_dtype, cb_numel, act_scale, 0, bias, bias_dtype, bias_numel,
                            out_features, in_features);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(cb_dtype == DIMQ_F16, "linear_lut_q takes the fp16 codebook of the packed export");
  Epi epi;
  rc = lut_q_epilogue(activation, out_act_scale, out_act_zp, y_dtype, epi);
  if (rc != DIMQ_OK) return rc;
  if (M == 0) return DIMQ_OK;
  return linear_codebook_impl(xq, DIMQ_F16, M, in_features, in_features, packed_w, 4, codebook, cb_dtype, 1, 16, bias,
                              bias_dtype, out_features, y, y_dtype, out_features, epi, DIMQ_VARIANT_AUTO,
                              as_stream(stream), static_cast<float>(act_scale));
}

// ---------------------------------------------------------------------------
// dimq_linear_lut_noalloc: dimq_linear_lut_ws with the library's own scratch
// in place of a caller workspace, for callers that cannot allocate.  The
// scratch is one file-scope device array per GPU (a copy on every device the
// library runs on, held until the process ends); host code reaches it only
// through the address hipGetSymbolAddress returns for the current device.
// Every call on a GPU shares that GPU's copy: calls that overlap on one GPU
// (other streams, other host threads) race on it.

constexpr int64_t kNoAllocScratchBytes = 16ll << 20;  // M * in_features <= 8,388,608 fp16 activations

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device with that device current; nullptr (and the HIP error) on failure.
static void* scratch_address(hipError_t* err) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= 64) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    addr[dev] = p;
  }
  return addr[dev];
}

extern "C" int dimq_linear_lut_noalloc(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w,
                                       int64_t packed_numel, const void* codebook, int cb_dtype, int64_t cb_numel,
                                       double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                                       int64_t bias_numel, int64_t out_features, int64_t in_features, float* y,
                                       void* stream) {
  const int rc = check_linear_lut(x_dtype, M, packed_numel, cb_dtype, cb_numel, act_scale, act_zp, bias, bias_dtype,
                                  bias_numel, out_features, in_features);
  if (rc != DIMQ_OK) return rc;
  const int64_t need = dimq_linear_lut_workspace_bytes(M, in_features, cb_dtype);
  if (need > kNoAllocScratchBytes)
    return set_error(DIMQ_ERR_INVALID,
                     "linear_lut_noalloc: M * in_features = %lld exceeds the scratch limit of %lld activations",
                     (long long)(M * in_features), (long long)(kNoAllocScratchBytes / 2));
  void* ws = nullptr;
  if (need > 0) {
    hipError_t err = hipSuccess;
    ws = scratch_address(&err);
    if (ws == nullptr)
      return set_error(DIMQ_ERR_HIP, "linear_lut_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(err));
  }
  return dimq_linear_lut_ws(x, x_dtype, M, packed_w, packed_numel, codebook, cb_dtype, cb_numel, act_scale, act_zp,
                            bias, bias_dtype, bias_numel, out_features, in_features, y, ws, need, stream);
}
