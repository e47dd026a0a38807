// Host side of the codebook Conv2d ops: argument checks (reference messages
// from csrc/dimq_conv2d_lut.cu:105-134) and launch of the implicit-GEMM
// kernels (im2col gathered on the fly, never materialised).
#include "gemm_kernel.h"

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
}  // namespace dimq

using namespace dimq;

extern "C" int dimq_conv2d_lut(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                               const uint8_t* packed_w, int64_t packed_numel, const void* codebook, int cb_dtype,
                               int64_t cb_numel, double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                               int64_t bias_numel, int64_t out_channels, int64_t in_channels_per_group,
                               int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                               int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, float* y,
                               void* stream) {
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
  if (s.B * s.OC * s.OH * s.OW == 0) return DIMQ_OK;
  GemmArgs p = conv_args(s, x, DIMQ_NCHW, packed_w, codebook, cb_dtype, 1, 16, bias, bias_dtype, y, DIMQ_F32,
                         DIMQ_NCHW);
  p.act_scale = static_cast<float>(act_scale);
  p.act_zp = static_cast<int>(act_zp);
  return gemm_dispatch(p, 4, x_dtype, true, kTile64x32, as_stream(stream));
}

extern "C" int64_t dimq_conv2d_prepared_words(int64_t out_channels, int64_t in_channels, int64_t kernel_h,
                                              int64_t kernel_w, int bits) {
  if (!halo_weight_supported(in_channels, kernel_h, kernel_w, bits) || out_channels <= 0) return 0;
  return halo_prepared_words(out_channels, in_channels, kernel_h, kernel_w, bits);
}

extern "C" int dimq_conv2d_prepare_weight(const uint8_t* packed_w, int64_t packed_numel, int bits,
                                          int64_t out_channels, int64_t in_channels, int64_t kernel_h,
                                          int64_t kernel_w, uint32_t* prepared_w, int64_t prepared_words,
                                          void* stream) {
  if (!halo_weight_supported(in_channels, kernel_h, kernel_w, bits))
    return set_error(DIMQ_ERR_UNSUPPORTED, "no kernel layout for C=%lld KH=%lld KW=%lld bits=%d",
                     (long long)in_channels, (long long)kernel_h, (long long)kernel_w, bits);
  DIMQ_CHECK(out_channels > 0, "channel counts must be positive");
  const int64_t wnumel = out_channels * in_channels * kernel_h * kernel_w;
  DIMQ_CHECK(packed_numel >= (wnumel * bits + 7) / 8, "packed_weight is too small for requested conv weight shape");
  DIMQ_CHECK(prepared_words >= halo_prepared_words(out_channels, in_channels, kernel_h, kernel_w, bits),
             "prepared weight buffer is too small");
  return launch_prepare(packed_w, out_channels, in_channels, kernel_h, kernel_w, bits, prepared_w,
                        as_stream(stream));
}

extern "C" int dimq_conv2d_codebook(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H,
                                    int64_t W, const uint8_t* packed_w, int64_t packed_numel, int bits,
                                    const uint32_t* prepared_w, int64_t prepared_words, const void* codebook, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                                    const void* bias, int bias_dtype, int64_t out_channels, int64_t kernel_h,
                                    int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                                    int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, void* y,
                                    int y_dtype, int y_layout, int variant, void* stream) {
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
  if (s.B * s.OC * s.OH * s.OW == 0) return DIMQ_OK;
  if (prepared_w != nullptr && variant != DIMQ_VARIANT_SMALL_M && aligned(x, 16) &&
      halo_eligible(s.C, s.KH, s.KW, s.sh, s.sw, s.dh, s.dw, s.groups, s.OH, s.OW, bits, x_dtype)) {
    DIMQ_CHECK(prepared_words >= halo_prepared_words(s.OC, s.C, s.KH, s.KW, bits),
               "prepared weight buffer is too small");
    return launch_conv_halo(x, x_dtype, x_layout, s.B, s.C, s.H, s.W, prepared_w, bits, codebook, cb_dtype, cb_rows,
                            cb_size, bias, bias_dtype, s.OC, s.KH, s.KW, s.sh, s.ph, s.pw, s.OH, s.OW, y, y_dtype,
                            y_layout, as_stream(stream));
  }
  if (variant != DIMQ_VARIANT_SMALL_M &&
      stem_eligible(s.C, s.OC, s.KH, s.KW, s.sh, s.sw, s.pw, s.dh, s.dw, s.groups, s.OH, s.OW, bits, y_dtype, x, y)) {
    return launch_conv_stem(x, x_dtype, x_layout, s.B, s.C, s.H, s.W, packed_w, packed_numel, bits, codebook,
                            cb_dtype, cb_rows, cb_size, bias, bias_dtype, s.OC, s.KH, s.KW, s.ph, s.pw, s.OH, s.OW,
                            y, y_dtype, y_layout, as_stream(stream));
  }
  GemmArgs p = conv_args(s, x, x_layout, packed_w, codebook, cb_dtype, cb_rows, cb_size, bias, bias_dtype, y,
                         y_dtype, y_layout);
  int tile = gemm_pick_tile(p.M, p.N, variant);
  if (tile == kTileGemv) tile = kTile16x16;  // the GEMV kernel has no im2col/group support
  return gemm_dispatch(p, bits, x_dtype, false, tile, as_stream(stream));
}
