// Host side of the codebook Conv2d ops: argument checks (reference messages
// from csrc/dimq_conv2d_lut.cu:105-134) and launch of the implicit-GEMM
// kernels (im2col gathered on the fly, never materialised).
#include "gemm_big.h"

namespace dimq {
namespace {

struct ConvShape {
  int64_t B, C, H, W, OC, ICg, KH, KW, sh, sw, ph, pw, dh, dw, groups, OH, OW;
};

int check_conv(const ConvShape& s) {
  DIMQ_CHECK(s.OC > 0 && s.ICg > 0, "channel counts must be positive");
  DIMQ_CHECK(s.KH > 0 && s.KW > 0, "kernel size must be positive");
  DIMQ_CHECK(s.sh > 0 && s.sw > 0, "stride must be positive");
  DIMQ_CHECK(s.dh > 0 && s.dw > 0, "dilation must be positive");
  DIMQ_CHECK(s.groups > 0, "groups must be positive");
  DIMQ_CHECK(s.ph >= 0 && s.pw >= 0, "padding must be non-negative");
  DIMQ_CHECK(s.B >= 0 && s.H >= 0 && s.W >= 0, "input sizes must be non-negative");
  DIMQ_CHECK(s.C == s.ICg * s.groups, "input channels do not match weight/groups");
  DIMQ_CHECK(s.OC % s.groups == 0, "out_channels must be divisible by groups");
  DIMQ_CHECK(s.OH >= 0 && s.OW >= 0, "computed negative output size");
  return DIMQ_OK;
}

GemmArgs conv_args(const ConvShape& s, const void* x, int x_layout, const uint8_t* w, const void* cb, int cb_dt,
                   int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dt, void* y, int y_dt, int y_layout) {
  GemmArgs p{};
  p.x = x;
  p.M = s.B * s.OH * s.OW;
  p.K = s.ICg * s.KH * s.KW;
  p.ldx = 0;
  p.w = w;
  p.N = s.OC / s.groups;
  p.cb = cb;
  p.cb_dt = cb_dt;
  p.cb_rows = cb_rows;
  p.cb_size = static_cast<int>(cb_size);
  p.bias = bias;
  p.bias_dt = bias_dt;
  p.y = y;
  p.y_dt = y_dt;
  p.ldy = 0;
  p.act_scale = 1.0f;
  p.act_zp = 0;
  p.fast_b = (p.K % 32 == 0) && aligned(w, 16);
  p.vec_a = 0;
  p.conv = 1;
  p.x_layout = x_layout;
  p.y_layout = y_layout;
  p.cB = s.B;
  p.cC = s.C;
  p.cH = s.H;
  p.cW = s.W;
  p.cOH = s.OH;
  p.cOW = s.OW;
  p.cOC = s.OC;
  p.cICg = s.ICg;
  p.cKH = static_cast<int>(s.KH);
  p.cKW = static_cast<int>(s.KW);
  p.csh = static_cast<int>(s.sh);
  p.csw = static_cast<int>(s.sw);
  p.cph = static_cast<int>(s.ph);
  p.cpw = static_cast<int>(s.pw);
  p.cdh = static_cast<int>(s.dh);
  p.cdw = static_cast<int>(s.dw);
  p.groups = static_cast<int>(s.groups);
  return p;
}

// ---- implicit-GEMM conv on the large-tile GEMM kernels (C % 64 == 0)
// Weight layout: the conv_kcrs stream re-packed tap-major, index (oc, kh, kw, c)
// at k = (kh*KW + kw)*C + c, same bits (no expansion).
bool gemm_conv_weight_supported(int64_t C, int64_t KH, int64_t KW, int bits) {
  return (bits == 2 || bits == 3 || bits == 4) && C > 0 && C % 64 == 0 && KH > 0 && KW > 0;
}

// The prepared weight holds every kernel layout the shape has, one after the
// other: [LDS-halo layout, padded to 16 bytes][tap-major layout].
int64_t halo_part_words(int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits) {
  if (!halo_weight_supported(C, KH, KW, bits)) return 0;
  return (halo_prepared_words(OC, C, KH, KW, bits) + 3) / 4 * 4;
}

int64_t gemm_part_words(int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits) {
  if (!gemm_conv_weight_supported(C, KH, KW, bits)) return 0;
  return OC * C * KH * KW * bits / 32;  // C % 64 == 0: whole words
}

// Which kernel a conv with both layouts takes (measured on ResNet-18's layers
// at batch 128): the LDS-halo kernel only for stride-1 KxK convs of fewer
// than 128 channels (64 vs 110 us at C = 64, 56x56), where its halo reuse
// beats the GEMM's 64-wide k stages; the implicit GEMM for the rest (stride 2
// C = 128: 38 vs 115 us; 1x1: 20-30 vs 35-39 us; C >= 128 stride 1: equal).
bool prefer_gemm_conv(int64_t C, int64_t KH, int64_t KW, int64_t stride) {
  return !(C < 128 && stride == 1 && KH * KW > 1);
}

template <int BITS>
__global__ void prepare_tapmajor_kernel(const uint8_t* __restrict__ src, int64_t src_bytes, int C, int KH, int KW,
                                        int64_t groups32, uint32_t* __restrict__ out) {
  const int64_t gi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gi >= groups32) return;
  const int64_t K = static_cast<int64_t>(C) * KH * KW;
  uint32_t words[BITS];
#pragma unroll
  for (int w = 0; w < BITS; ++w) words[w] = 0u;
  for (int j = 0; j < 32; ++j) {
    const int64_t f = gi * 32 + j;
    const int64_t oc = f / K;
    const int r = static_cast<int>(f - oc * K);
    const int tap = r / C;
    const int c = r - tap * C;
    const int kh = tap / KW;
    const int kw = tap - kh * KW;
    const int64_t bit = (((oc * C + c) * KH + kh) * KW + kw) * BITS;
    const int64_t byte = bit >> 3;
    const int sh = static_cast<int>(bit & 7);
    uint32_t v = static_cast<uint32_t>(src[byte]) >> sh;
    if (sh + BITS > 8 && byte + 1 < src_bytes) v |= static_cast<uint32_t>(src[byte + 1]) << (8 - sh);
    v &= (1u << BITS) - 1u;
    const int fb = j * BITS;
    words[fb >> 5] |= v << (fb & 31);
    if ((fb & 31) + BITS > 32) words[(fb >> 5) + 1] |= v >> (32 - (fb & 31));
  }
#pragma unroll
  for (int w = 0; w < BITS; ++w) out[gi * BITS + w] = words[w];
}

int launch_prepare_tapmajor(const uint8_t* src, int64_t src_bytes, int64_t OC, int64_t C, int64_t KH, int64_t KW,
                            int bits, uint32_t* out, hipStream_t s) {
  const int64_t groups32 = OC * C * KH * KW / 32;
  const unsigned blocks = static_cast<unsigned>((groups32 + 255) / 256);
  switch (bits) {
    case 2: hipLaunchKernelGGL(prepare_tapmajor_kernel<2>, dim3(blocks), dim3(256), 0, s, src, src_bytes, (int)C,
                               (int)KH, (int)KW, groups32, out); break;
    case 3: hipLaunchKernelGGL(prepare_tapmajor_kernel<3>, dim3(blocks), dim3(256), 0, s, src, src_bytes, (int)C,
                               (int)KH, (int)KW, groups32, out); break;
    default: hipLaunchKernelGGL(prepare_tapmajor_kernel<4>, dim3(blocks), dim3(256), 0, s, src, src_bytes, (int)C,
                                (int)KH, (int)KW, groups32, out); break;
  }
  return check_launch("prepare_conv_weight (tap-major)");
}


// Tile of the implicit-GEMM conv: 128x128 when that fills every CU, else 64x128.
// At most 128 output channels, or a single 64-wide k stage (K <= 64), also
// take 64x128 (ResNet-18 bs128, same process: layer2 3x3 C 128 56.9 -> 49.8
// us, with the residual 59.9 -> 52.9; layer2 downsample 1x1/2 C 64 20.3 ->
// 18.0); at layer3 (N 256) both tiles measured alike, at layer4 (N 512) the
// 128x128 grid does not fill the CUs and 64x128 is faster (58.3 against 69.4).
int gemm_conv_tile(int64_t M, int64_t N, int64_t K) {
  if (K <= 64 || N <= 128) return 1;
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  return t128 >= device_cus() ? 0 : 1;
}

ConvShape make_shape(int64_t B, int64_t C, int64_t H, int64_t W, int64_t OC, int64_t ICg, int64_t KH, int64_t KW,
                     int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int64_t groups) {
  ConvShape s{B, C, H, W, OC, ICg, KH, KW, sh, sw, ph, pw, dh, dw, groups, 0, 0};
  if (sh > 0 && sw > 0) {
    s.OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
    s.OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  }
  return s;
}

}  // namespace

// CUs of the current device (cached per device).
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace dimq

using namespace dimq;

// Device workspace of the W4A4 fast path: the activations as fp16 a - zp
// (NCHW) and, for shapes the LDS-halo kernel runs, its 4-bit weight layout.
// 0 = no fast path (the codebook is not fp16).
static int64_t lut_act_bytes(int64_t B, int64_t C, int64_t H, int64_t W) { return (B * C * H * W * 2 + 255) / 256 * 256; }

extern "C" int64_t dimq_conv2d_lut_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t out_channels,
                                                   int64_t in_channels_per_group, int64_t kernel_h,
                                                   int64_t kernel_w, int64_t groups, int cb_dtype) {
  if (cb_dtype != DIMQ_F16 || B <= 0 || C <= 0 || H <= 0 || W <= 0 || out_channels <= 0) return 0;
  const int64_t hw = (groups == 1 && in_channels_per_group == C)
                         ? halo_part_words(out_channels, C, kernel_h, kernel_w, 4) : 0;
  return lut_act_bytes(B, C, H, W) + hw * 4;
}

extern "C" int dimq_conv2d_lut(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                               const uint8_t* packed_w, int64_t packed_numel, const void* codebook, int cb_dtype,
                               int64_t cb_numel, double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                               int64_t bias_numel, int64_t out_channels, int64_t in_channels_per_group,
                               int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                               int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, float* y,
                               void* stream) {
  return dimq_conv2d_lut_ws(x, x_dtype, B, C, H, W, packed_w, packed_numel, codebook, cb_dtype, cb_numel, act_scale,
                            act_zp, bias, bias_dtype, bias_numel, out_channels, in_channels_per_group, kernel_h,
                            kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups, y, nullptr, 0,
                            stream);
}

// With an fp16 codebook and the workspace above: activations quantized once
// to the exact fp16 integers a - zp, then the weight-only conv kernels with
// act_scale on the accumulator (the LDS-halo kernel where the shape allows,
// its weight layout built into the workspace; else the generic implicit GEMM).
// Otherwise the generic A4 kernel (hi + lo fp16 codebook planes).
extern "C" int dimq_conv2d_lut_ws(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                                  const uint8_t* packed_w, int64_t packed_numel, const void* codebook, int cb_dtype,
                                  int64_t cb_numel, double act_scale, int64_t act_zp, const void* bias,
                                  int bias_dtype, int64_t bias_numel, int64_t out_channels,
                                  int64_t in_channels_per_group, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                  int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h,
                                  int64_t dilation_w, int64_t groups, float* y, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  DIMQ_CHECK(is_float_dtype(x_dtype), "conv2d_lut expects floating input");
  DIMQ_CHECK(is_float_dtype(cb_dtype), "codebook must be floating point");
  DIMQ_CHECK(cb_numel == 16, "codebook must have 16 entries for W4");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  DIMQ_CHECK(act_zp >= 0 && act_zp <= 15, "act_zero_point must be in [0, 15]");
  const ConvShape s = make_shape(B, C, H, W, out_channels, in_channels_per_group, kernel_h, kernel_w, stride_h,
                                 stride_w, pad_h, pad_w, dilation_h, dilation_w, groups);
  const int rc = check_conv(s);
  if (rc != DIMQ_OK) return rc;
  const int64_t wnumel = s.OC * s.ICg * s.KH * s.KW;
  DIMQ_CHECK(packed_numel >= (wnumel + 1) / 2, "packed_weight is too small for requested conv weight shape");
  if (bias) DIMQ_CHECK(bias_numel == out_channels, "bias numel must equal out_channels");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  DIMQ_CHECK(workspace_bytes >= 0, "workspace_bytes must be non-negative");
  if (s.B * s.OC * s.OH * s.OW == 0) return DIMQ_OK;
  const hipStream_t st = as_stream(stream);
  const int64_t need = dimq_conv2d_lut_workspace_bytes(s.B, s.C, s.H, s.W, s.OC, s.ICg, s.KH, s.KW, s.groups,
                                                       cb_dtype);
  if (workspace != nullptr && need > 0 && workspace_bytes >= need && aligned(workspace, 16)) {
    const float sc = static_cast<float>(act_scale);
    uint16_t* q = static_cast<uint16_t*>(workspace);
    const int64_t hw = (s.groups == 1) ? halo_part_words(s.OC, s.C, s.KH, s.KW, 4) : 0;
    if (hw > 0 && halo_eligible(s.C, s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, s.groups, s.OH, s.OW, 4, DIMQ_F16,
                                kEpiNone, DIMQ_NCHW)) {
      // the weight layout and the quantized activations in one launch
      uint32_t* kw = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + lut_act_bytes(s.B, s.C, s.H, s.W));
      const int r = launch_w4a4_conv_inputs(packed_w, s.OC, s.C, s.KH, s.KW, kw, x, x_dtype, s.B * s.C * s.H * s.W,
                                            sc, static_cast<int>(act_zp), q, st);
      if (r != DIMQ_OK) return r;
      return launch_conv_halo(q, DIMQ_F16, DIMQ_NCHW, s.B, s.C, s.H, s.W, kw, 4, codebook, cb_dtype, 1, 16, bias,
                              bias_dtype, s.OC, s.KH, s.KW, s.sh, s.ph, s.pw, s.OH, s.OW, y, DIMQ_F32, DIMQ_NCHW,
                              Epi{}, st, sc);
    }
    const int r = launch_quantize_a4_f16(x, x_dtype, s.B * s.C * s.H * s.W, sc, static_cast<int>(act_zp), q, st);
    if (r != DIMQ_OK) return r;
    GemmArgs p = conv_args(s, q, DIMQ_NCHW, packed_w, codebook, cb_dtype, 1, 16, bias, bias_dtype, y, DIMQ_F32,
                           DIMQ_NCHW);
    p.acc_scale = sc;
    int tile = gemm_pick_tile(p.M, p.N, DIMQ_VARIANT_AUTO);
    if (tile == kTileGemv) tile = kTile16x16;  // the GEMV kernel has no im2col/group support
    return gemm_dispatch(p, 4, DIMQ_F16, false, tile, st);
  }
  GemmArgs p = conv_args(s, x, DIMQ_NCHW, packed_w, codebook, cb_dtype, 1, 16, bias, bias_dtype, y, DIMQ_F32,
                         DIMQ_NCHW);
  p.act_scale = static_cast<float>(act_scale);
  p.act_zp = static_cast<int>(act_zp);
  return gemm_dispatch(p, 4, x_dtype, true, kTile64x32, st);
}

// Quantized-activation form of conv2d_lut: xq holds the input as the fp16
// integers a - zp (NCHW), y is NCHW.  With a prepared weight (the 4-bit
// LDS-halo layout of dimq_conv2d_prepare_weight) the halo kernels run where
// the shape allows; otherwise the generic implicit GEMM.
extern "C" int dimq_conv2d_lut_q(const uint16_t* xq, int64_t B, int64_t C, int64_t H, int64_t W,
                                 const uint8_t* packed_w, int64_t packed_numel, const uint32_t* prepared_w,
                                 int64_t prepared_words, const void* codebook, int cb_dtype, int64_t cb_numel,
                                 double act_scale, const void* bias, int bias_dtype, int64_t bias_numel,
                                 int64_t out_channels, int64_t in_channels_per_group, int64_t kernel_h,
                                 int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 int64_t dilation_h, int64_t dilation_w, int64_t groups, int activation,
                                 double out_act_scale, int64_t out_act_zp, void* y, int y_dtype, void* stream) {
  DIMQ_CHECK(cb_dtype == DIMQ_F16, "conv2d_lut_q takes the fp16 codebook of the packed export");
  DIMQ_CHECK(cb_numel == 16, "codebook must have 16 entries for W4");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  const ConvShape s = make_shape(B, C, H, W, out_channels, in_channels_per_group, kernel_h, kernel_w, stride_h,
                                 stride_w, pad_h, pad_w, dilation_h, dilation_w, groups);
  int rc = check_conv(s);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(packed_numel >= (s.OC * s.ICg * s.KH * s.KW + 1) / 2,
             "packed_weight is too small for requested conv weight shape");
  if (bias) DIMQ_CHECK(bias_numel == out_channels, "bias numel must equal out_channels");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  Epi epi;
  rc = lut_q_epilogue(activation, out_act_scale, out_act_zp, y_dtype, epi);
  if (rc != DIMQ_OK) return rc;
  if (s.B * s.OC * s.OH * s.OW == 0) return DIMQ_OK;
  const hipStream_t st = as_stream(stream);
  const float sc = static_cast<float>(act_scale);
  const int64_t hw = (prepared_w && s.groups == 1) ? halo_part_words(s.OC, s.C, s.KH, s.KW, 4) : 0;
  if (prepared_w) DIMQ_CHECK(prepared_words >= hw, "prepared weight buffer is too small");
  if (hw > 0 && aligned(xq, 16) &&
      halo_eligible(s.C, s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, s.groups, s.OH, s.OW, 4, DIMQ_F16, epi_mode(epi),
                    DIMQ_NCHW)) {
    return launch_conv_halo(xq, DIMQ_F16, DIMQ_NCHW, s.B, s.C, s.H, s.W, prepared_w, 4, codebook, cb_dtype, 1, 16,
                            bias, bias_dtype, s.OC, s.KH, s.KW, s.sh, s.ph, s.pw, s.OH, s.OW, y, y_dtype, DIMQ_NCHW,
                            epi, st, sc);
  }
  GemmArgs p = conv_args(s, xq, DIMQ_NCHW, packed_w, codebook, cb_dtype, 1, 16, bias, bias_dtype, y, y_dtype,
                         DIMQ_NCHW);
  p.acc_scale = sc;
  p.epi = epi;
  int tile = gemm_pick_tile(p.M, p.N, DIMQ_VARIANT_AUTO);
  if (tile == kTileGemv) tile = kTile16x16;  // the GEMV kernel has no im2col/group support
  return gemm_dispatch(p, 4, DIMQ_F16, false, tile, st);
}

// Weight x activation codebook Conv2d: x replaced by its nearest activation
// centre in x's dtype (the QAT wrapper's fake_quant_activation before
// F.conv2d, quant/dimq_wrapper.py:80-85,189-197), then the weight-codebook
// conv on it (dequantize-then-MFMA).  Workspace: B*C*H*W elements of x's
// dtype, fp32 at most.
extern "C" int64_t dimq_conv2d_codebook_act_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W) {
  if (B <= 0 || C <= 0 || H <= 0 || W <= 0) return 0;
  return (B * C * H * W * 4 + 255) / 256 * 256;
}

extern "C" int dimq_conv2d_codebook_act(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H,
                                        int64_t W, const uint8_t* packed_w, int64_t packed_numel, int bits,
                                        const uint32_t* prepared_w, int64_t prepared_words, const void* codebook,
                                        int cb_dtype, int64_t cb_rows, int64_t cb_size, const float* act_centers,
                                        int64_t n_act, const void* bias, int bias_dtype, int64_t out_channels,
                                        int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                                        int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w,
                                        int64_t groups, void* y, int y_dtype, int y_layout, int variant,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  DIMQ_CHECK(x_dtype == DIMQ_F32 || x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16,
             "conv2d_codebook_act expects fp32, fp16 or bf16 input");
  DIMQ_CHECK(n_act >= 1 && n_act <= 256, "activation codebook must hold between 1 and 256 centres");
  DIMQ_CHECK(act_centers != nullptr, "activation codebook is required");
  DIMQ_CHECK(B >= 0 && C > 0 && H >= 0 && W >= 0, "input sizes must be non-negative");
  const int64_t need = dimq_conv2d_codebook_act_workspace_bytes(B, C, H, W);
  if (need == 0) return DIMQ_OK;
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= need && aligned(workspace, 16),
             "workspace must be 16-byte aligned and hold dimq_conv2d_codebook_act_workspace_bytes bytes");
  const int rc = launch_act_codebook(x, x_dtype, B * C * H * W, act_centers, static_cast<int>(n_act), workspace,
                                     as_stream(stream));
  if (rc != DIMQ_OK) return rc;
  return dimq_conv2d_codebook_ex(workspace, x_dtype, x_layout, B, C, H, W, packed_w, packed_numel, bits, prepared_w,
                                 prepared_words, codebook, cb_dtype, cb_rows, cb_size, bias, bias_dtype, out_channels,
                                 kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups,
                                 y, y_dtype, y_layout, nullptr, 0, DIMQ_ACT_NONE, variant, stream);
}

extern "C" int64_t dimq_conv2d_prepared_words(int64_t out_channels, int64_t in_channels, int64_t kernel_h,
                                              int64_t kernel_w, int bits) {
  if (out_channels <= 0) return 0;
  return halo_part_words(out_channels, in_channels, kernel_h, kernel_w, bits) +
         gemm_part_words(out_channels, in_channels, kernel_h, kernel_w, bits);
}

extern "C" int dimq_conv2d_prepare_weight(const uint8_t* packed_w, int64_t packed_numel, int bits,
                                          int64_t out_channels, int64_t in_channels, int64_t kernel_h,
                                          int64_t kernel_w, uint32_t* prepared_w, int64_t prepared_words,
                                          void* stream) {
  const int64_t hw = halo_part_words(out_channels, in_channels, kernel_h, kernel_w, bits);
  const int64_t gw = gemm_part_words(out_channels, in_channels, kernel_h, kernel_w, bits);
  if (hw + gw == 0)
    return set_error(DIMQ_ERR_UNSUPPORTED, "no kernel layout for C=%lld KH=%lld KW=%lld bits=%d",
                     (long long)in_channels, (long long)kernel_h, (long long)kernel_w, bits);
  DIMQ_CHECK(out_channels > 0, "channel counts must be positive");
  const int64_t wnumel = out_channels * in_channels * kernel_h * kernel_w;
  DIMQ_CHECK(packed_numel >= (wnumel * bits + 7) / 8, "packed_weight is too small for requested conv weight shape");
  DIMQ_CHECK(prepared_words >= hw + gw, "prepared weight buffer is too small");
  if (hw) {
    const int rc = launch_prepare(packed_w, out_channels, in_channels, kernel_h, kernel_w, bits, prepared_w,
                                  as_stream(stream));
    if (rc != DIMQ_OK) return rc;
  }
  if (gw)
    return launch_prepare_tapmajor(packed_w, packed_numel, out_channels, in_channels, kernel_h, kernel_w, bits,
                                   prepared_w + hw, as_stream(stream));
  return DIMQ_OK;
}

extern "C" int dimq_conv2d_codebook(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H,
                                    int64_t W, const uint8_t* packed_w, int64_t packed_numel, int bits,
                                    const uint32_t* prepared_w, int64_t prepared_words, const void* codebook,
                                    int cb_dtype, int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype,
                                    int64_t out_channels, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                    int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h,
                                    int64_t dilation_w, int64_t groups, void* y, int y_dtype, int y_layout,
                                    int variant, void* stream) {
  return dimq_conv2d_codebook_ex(x, x_dtype, x_layout, B, C, H, W, packed_w, packed_numel, bits, prepared_w,
                                 prepared_words, codebook, cb_dtype, cb_rows, cb_size, bias, bias_dtype,
                                 out_channels, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, dilation_h,
                                 dilation_w, groups, y, y_dtype, y_layout, nullptr, 0, DIMQ_ACT_NONE, variant,
                                 stream);
}

extern "C" int dimq_conv2d_codebook_ex(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H,
                                       int64_t W, const uint8_t* packed_w, int64_t packed_numel, int bits,
                                       const uint32_t* prepared_w, int64_t prepared_words, const void* codebook,
                                       int cb_dtype, int64_t cb_rows, int64_t cb_size, const void* bias,
                                       int bias_dtype, int64_t out_channels, int64_t kernel_h, int64_t kernel_w,
                                       int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                       int64_t dilation_h, int64_t dilation_w, int64_t groups, void* y, int y_dtype,
                                       int y_layout, const void* residual, int residual_dtype, int activation,
                                       int variant, void* stream) {
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 8))
    return set_error(DIMQ_ERR_UNSUPPORTED, "bits must be one of 2, 3, 4, 8 (got %d)", bits);
  DIMQ_CHECK(x_dtype == DIMQ_F32 || x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16,
             "conv2d_codebook expects fp32, fp16 or bf16 input");
  DIMQ_CHECK(y_dtype == DIMQ_F32 || y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16,
             "conv2d_codebook output dtype must be fp32, fp16 or bf16");
  DIMQ_CHECK(x_layout == DIMQ_NCHW || x_layout == DIMQ_NHWC, "unknown input layout %d", x_layout);
  DIMQ_CHECK(y_layout == DIMQ_NCHW || y_layout == DIMQ_NHWC, "unknown output layout %d", y_layout);
  DIMQ_CHECK(is_float_dtype(cb_dtype), "codebook must be floating point");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  DIMQ_CHECK(groups > 0, "groups must be positive");
  const ConvShape s = make_shape(B, C, H, W, out_channels, groups > 0 ? C / groups : 0, kernel_h, kernel_w, stride_h,
                                 stride_w, pad_h, pad_w, dilation_h, dilation_w, groups);
  const int rc = check_conv(s);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(cb_rows == 1 || cb_rows == out_channels,
             "codebook must have 1 (per layer) or out_channels (per channel) rows");
  DIMQ_CHECK(cb_size >= 1 && cb_size <= (1 << bits), "codebook rows must hold between 1 and 2^bits entries");
  const int64_t wnumel = s.OC * s.ICg * s.KH * s.KW;
  DIMQ_CHECK(packed_numel >= (wnumel * bits + 7) / 8, "packed_weight is too small for requested conv weight shape");
  DIMQ_CHECK(variant >= DIMQ_VARIANT_AUTO && variant <= DIMQ_VARIANT_MFMA, "unknown kernel variant %d", variant);
  DIMQ_CHECK(residual == nullptr || is_float_dtype(residual_dtype), "residual must be floating point");
  DIMQ_CHECK(activation >= DIMQ_ACT_NONE && activation <= DIMQ_ACT_GELU, "unknown activation %d", activation);
  const Epi epi{residual, residual_dtype, activation, residual != nullptr && aligned(residual, 16)};
  if (s.B * s.OC * s.OH * s.OW == 0) return DIMQ_OK;
  const int64_t hw = prepared_w ? halo_part_words(s.OC, s.C, s.KH, s.KW, bits) : 0;
  const int64_t gw = prepared_w ? gemm_part_words(s.OC, s.C, s.KH, s.KW, bits) : 0;
  if (prepared_w != nullptr) DIMQ_CHECK(prepared_words >= hw + gw, "prepared weight buffer is too small");
  const int mode = epi_mode(epi);
  const bool gemm_ok = gw > 0 && variant != DIMQ_VARIANT_SMALL_M && s.groups == 1 && x_layout == DIMQ_NHWC &&
                       (mode == kEpiNone || mode == kEpiRelu || mode == kEpiRes || mode == kEpiResRelu) &&
                       y_layout == DIMQ_NHWC && (x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16) && aligned(x, 16) &&
                       aligned(y, 16) && aligned(prepared_w + hw, 16);
  const bool halo_ok = hw > 0 && variant != DIMQ_VARIANT_SMALL_M && aligned(x, 16) &&
                       halo_eligible(s.C, s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, s.groups, s.OH, s.OW, bits, x_dtype,
                                     epi_mode(epi), y_layout);
  // DIMQ_VARIANT_MFMA forces the implicit-GEMM tiles over the LDS-halo kernel
  // (A/B runs of the choice prefer_gemm_conv makes)
  if (gemm_ok && (!halo_ok || variant == DIMQ_VARIANT_MFMA || prefer_gemm_conv(s.C, s.KH, s.KW, s.sh))) {
    GemmArgs p = conv_args(s, x, x_layout, reinterpret_cast<const uint8_t*>(prepared_w + hw), codebook, cb_dtype,
                           cb_rows, cb_size, bias, bias_dtype, y, y_dtype, y_layout);
    p.ldy = s.OC;
    p.epi = epi;
    const int tile = gemm_conv_tile(p.M, p.N, p.K);
    switch (bits) {
      case 2: return launch_big_conv_b2(p, x_dtype, tile, as_stream(stream));
      case 3: return launch_big_conv_b3(p, x_dtype, tile, as_stream(stream));
      default: return launch_big_conv_b4(p, x_dtype, tile, as_stream(stream));
    }
  }
  if (halo_ok) {
    return launch_conv_halo(x, x_dtype, x_layout, s.B, s.C, s.H, s.W, prepared_w, bits, codebook, cb_dtype, cb_rows,
                            cb_size, bias, bias_dtype, s.OC, s.KH, s.KW, s.sh, s.ph, s.pw, s.OH, s.OW, y, y_dtype,
                            y_layout, epi, as_stream(stream));
  }
  if (variant != DIMQ_VARIANT_SMALL_M &&
      stem_eligible(s.C, s.OC, s.KH, s.KW, s.sh, s.sw, s.pw, s.dh, s.dw, s.groups, s.OH, s.OW, bits, x_dtype, y_dtype, x, y,
                    epi_mode(epi), packed_w, packed_numel, codebook, cb_dtype, cb_rows, cb_size)) {
    return launch_conv_stem(x, x_dtype, x_layout, s.B, s.C, s.H, s.W, packed_w, packed_numel, bits, codebook,
                            cb_dtype, cb_rows, cb_size, bias, bias_dtype, s.OC, s.KH, s.KW, s.ph, s.pw, s.OH, s.OW,
                            y, y_dtype, y_layout, epi, as_stream(stream));
  }
  GemmArgs p = conv_args(s, x, x_layout, packed_w, codebook, cb_dtype, cb_rows, cb_size, bias, bias_dtype, y,
                         y_dtype, y_layout);
  p.epi = epi;
  int tile = gemm_pick_tile(p.M, p.N, variant);
  if (tile == kTileGemv) tile = kTile16x16;  // the GEMV kernel has no im2col/group support
  return gemm_dispatch(p, bits, x_dtype, false, tile, as_stream(stream));
}
