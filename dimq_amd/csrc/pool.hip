// 2-D max pooling over channels-last (NHWC) fp16/bf16 activations, for the
// ResNet-18 workload's stem pool (3x3, stride 2, padding 1 on
// [128, 112, 112, 64]): y[b, oh, ow, c] = max over the window's in-image taps
// of x[b, oh*sh - ph + kh, ow*sw - pw + kw, c], as torch.nn.functional.max_pool2d
// (padding never wins; a NaN in the window gives NaN).
//
// Thread = 8 consecutive channels of one output pixel: one 16-byte load per
// tap and one 16-byte store; consecutive threads take consecutive channel
// groups, then pixels, so every load and store instruction of a wave covers
// contiguous memory.  Neighbouring windows share input rows through L2, so
// HBM sees each input byte about once.  3x3 windows issue their nine loads
// back to back (ResNet-18 stem pool, bs128, same process: 67.0 -> 52.2 us);
// handing each XCD a contiguous run of output rows (so that the row two
// output rows share stays in one L2) measured no faster (52.3 us).
#include "common.h"

namespace dimq {
namespace {

template <int XT>
__device__ __forceinline__ float to_float16b(uint32_t h) {
  return XT == DIMQ_F16 ? f16_bits_to_float(h) : bf16_bits_to_float(h);
}

// m = max(m, the 8 values of v); a NaN, once in, stays
template <int XT>
__device__ __forceinline__ void max8(float (&m)[8], const uint4& v) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = to_float16b<XT>(u[j] & 0xffffu), hi = to_float16b<XT>(u[j] >> 16);
    m[2 * j] = (lo > m[2 * j] || lo != lo) ? lo : m[2 * j];
    m[2 * j + 1] = (hi > m[2 * j + 1] || hi != hi) ? hi : m[2 * j + 1];
  }
}

// K > 0: a K x K window (the ResNet stem pool: K = 3), all K * K loads issued
// before the first is used -- a tap outside the image loads the clamped
// in-image pixel and is left out of the maximum by a select, since a branch
// around each load made the compiler wait for every load before issuing the
// next.  K = 0: any window, taps in a loop.
template <int XT, int K>
__global__ __launch_bounds__(256) void max_pool_nhwc_kernel(const uint16_t* __restrict__ x, int H, int W, int C,
                                                            int OH, int OW, int KH, int KW, int sh, int sw, int ph,
                                                            int pw, int64_t total8, uint16_t* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= total8) return;
  const int c8 = C >> 3;
  const int cq = static_cast<int>(t % c8);
  int64_t pix = t / c8;
  const int ow = static_cast<int>(pix % OW);
  pix /= OW;
  const int oh = static_cast<int>(pix % OH);
  const int64_t b = pix / OH;
  float m[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) m[j] = -__builtin_inff();
  if constexpr (K > 0) {
    uint4 v[K][K];
    bool in[K][K];
#pragma unroll
    for (int kh = 0; kh < K; ++kh) {
      const int ih = oh * sh - ph + kh;
      const int ihc = min(max(ih, 0), H - 1);
#pragma unroll
      for (int kw = 0; kw < K; ++kw) {
        const int iw = ow * sw - pw + kw;
        const int iwc = min(max(iw, 0), W - 1);
        in[kh][kw] = ih == ihc && iw == iwc;
        v[kh][kw] = *reinterpret_cast<const uint4*>(x + ((b * H + ihc) * W + iwc) * C + 8 * cq);
      }
    }
#pragma unroll
    for (int kh = 0; kh < K; ++kh)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) {
        float mt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) mt[j] = m[j];
        max8<XT>(mt, v[kh][kw]);
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = in[kh][kw] ? mt[j] : m[j];
      }
  } else {
  for (int kh = 0; kh < KH; ++kh) {
    const int ih = oh * sh - ph + kh;
    if (ih < 0 || ih >= H) continue;
    for (int kw = 0; kw < KW; ++kw) {
      const int iw = ow * sw - pw + kw;
      if (iw < 0 || iw >= W) continue;
      max8<XT>(m, *reinterpret_cast<const uint4*>(x + ((b * H + ih) * W + iw) * C + 8 * cq));
    }
  }
  }
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // the maxima are input values, so the conversion back is exact
    o[j] = XT == DIMQ_F16 ? (float_to_f16_bits(m[2 * j]) | (float_to_f16_bits(m[2 * j + 1]) << 16))
                          : (float_to_bf16_bits(m[2 * j]) | (float_to_bf16_bits(m[2 * j + 1]) << 16));
  }
  *reinterpret_cast<uint4*>(y + (((b * OH + oh) * OW + ow) * C) + 8 * cq) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace
}  // namespace dimq

using namespace dimq;

extern "C" int dimq_max_pool2d_nhwc(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                                    int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                                    int64_t pad_h, int64_t pad_w, void* y, void* stream) {
  DIMQ_CHECK(x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16, "max_pool2d expects fp16 or bf16 input");
  DIMQ_CHECK(B >= 0 && C > 0 && H > 0 && W > 0, "max_pool2d input sizes must be positive");
  DIMQ_CHECK(C % 8 == 0, "max_pool2d needs a channel count that is a multiple of 8");
  DIMQ_CHECK(kernel_h > 0 && kernel_w > 0 && stride_h > 0 && stride_w > 0, "max_pool2d kernel and stride must be positive");
  DIMQ_CHECK(pad_h >= 0 && pad_w >= 0 && 2 * pad_h <= kernel_h && 2 * pad_w <= kernel_w,
             "pad should be at most half of effective kernel size");  // torch's check
  DIMQ_CHECK(aligned(x, 16) && aligned(y, 16), "max_pool2d needs 16-byte aligned input and output");
  const int64_t OH = (H + 2 * pad_h - kernel_h) / stride_h + 1;
  const int64_t OW = (W + 2 * pad_w - kernel_w) / stride_w + 1;
  DIMQ_CHECK(OH > 0 && OW > 0, "max_pool2d output size is too small");
  const int64_t total8 = B * OH * OW * (C / 8);
  if (total8 == 0) return DIMQ_OK;
  DIMQ_CHECK((total8 + 255) / 256 < (int64_t)1 << 31, "max_pool2d: too many outputs for one launch");
  const dim3 grid(static_cast<unsigned>((total8 + 255) / 256));
  const hipStream_t s = as_stream(stream);
  const bool k3 = kernel_h == 3 && kernel_w == 3;
  auto k = max_pool_nhwc_kernel<DIMQ_F16, 0>;
  if (x_dtype == DIMQ_F16) k = k3 ? max_pool_nhwc_kernel<DIMQ_F16, 3> : max_pool_nhwc_kernel<DIMQ_F16, 0>;
  else k = k3 ? max_pool_nhwc_kernel<DIMQ_BF16, 3> : max_pool_nhwc_kernel<DIMQ_BF16, 0>;
  hipLaunchKernelGGL(k, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x), (int)H, (int)W, (int)C, (int)OH,
                     (int)OW, (int)kernel_h, (int)kernel_w, (int)stride_h, (int)stride_w, (int)pad_h, (int)pad_w,
                     total8, static_cast<uint16_t*>(y));
  return check_launch("max_pool2d");
}
