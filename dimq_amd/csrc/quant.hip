// Element-wise quantization kernels:
//  * u4 activation quantization (dimq_backend/reference.py:11-21,
//    csrc/dimq_pack.cu:37-48) with an IEEE divide and round-half-to-even;
//  * activation x centroid product tables (dimq_backend/reference.py:32-44,
//    csrc/dimq_product_table.cu:11-25), per layer or per output channel;
//  * nearest-centre index assignment (quant/dimq.py:197-221,
//    dimq_backend/export.py:24-35), per layer or per output channel.
#include "common.h"

namespace dimq {
namespace {

constexpr int kThreads = 256;

// 8 activations per thread; the HIP divide is IEEE-correct (no fast-math).
__global__ __launch_bounds__(kThreads) void quantize_act_kernel(const void* __restrict__ x, int dt, int64_t n,
                                                                float s, int zp, uint8_t* __restrict__ out) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;
  if (base >= n) return;
  if (base + 8 <= n) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t q = (uint32_t)quantize_u4(load_as_float(x, dt, base + j), s, zp);
      if (j < 4) lo |= q << (8 * j); else hi |= q << (8 * (j - 4));
    }
    if (((reinterpret_cast<uintptr_t>(out) + base) & 7) == 0) {
      *reinterpret_cast<uint2*>(out + base) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[base + j] = (uint8_t)((j < 4 ? lo >> (8 * j) : hi >> (8 * (j - 4))) & 0xff);
    }
  } else {
    for (int64_t i = base; i < n; ++i) out[i] = (uint8_t)quantize_u4(load_as_float(x, dt, i), s, zp);
  }
}

// table[g][w][a] = C[g][w] * (s * (a - zp)), fp32, same operation order as
// the reference (product of the centroid and the dequantized level).
__global__ __launch_bounds__(kThreads) void product_table_kernel(const void* __restrict__ cb, int dt, int64_t total,
                                                                 float s, int zp, float* __restrict__ table) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const int a = static_cast<int>(i & 15);
  const float w = load_as_float(cb, dt, i >> 4);
  const float ahat = s * static_cast<float>(a - zp);
  table[i] = w * ahat;
}

// Nearest centre, exact argmin semantics of torch on fp32 distances:
// d = (w - c)^2 with one rounding per operation; strict '<' keeps the first
// minimum; a NaN distance wins and the first NaN is kept.
// Block = one row segment of 256*4 weights; the row's centres sit in LDS and
// are read as broadcasts.
__global__ __launch_bounds__(kThreads) void hard_quantize_kernel(const void* __restrict__ w, int dt, int64_t rows,
                                                                 int64_t row_len, const float* __restrict__ centers,
                                                                 int K, int per_channel, uint8_t* __restrict__ idx,
                                                                 void* __restrict__ values, int64_t seg_per_row) {
  __shared__ float c_s[256];
  const int64_t row = static_cast<int64_t>(blockIdx.x) / seg_per_row;
  const int64_t seg = static_cast<int64_t>(blockIdx.x) % seg_per_row;
  const float* c = centers + (per_channel ? row * K : 0);
  for (int j = threadIdx.x; j < K; j += kThreads) c_s[j] = c[j];
  __syncthreads();
  const int64_t start = seg * (kThreads * 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t k = start + r * kThreads + threadIdx.x;
    if (k >= row_len) break;
    const int64_t e = row * row_len + k;
    const float x = load_as_float(w, dt, e);
    int best = 0;
    float best_d = __builtin_inff();
    bool have = false;
    bool have_nan = false;
    for (int j = 0; j < K; ++j) {
      const float diff = x - c_s[j];
      const float d = __fmul_rn(diff, diff);
      if (d != d) {
        if (!have_nan) {
          best = j;
          have_nan = true;
        }
      } else if (!have_nan && (!have || d < best_d)) {
        best = j;
        best_d = d;
        have = true;
      }
    }
    idx[e] = (uint8_t)best;
    if (values) store_from_float(values, dt, e, c_s[best]);
  }
}

}  // namespace
}  // namespace dimq

using namespace dimq;

extern "C" int dimq_quantize_activation_u4(const void* x, int x_dtype, int64_t numel, double act_scale,
                                           int64_t act_zp, uint8_t* out, void* stream) {
  DIMQ_CHECK(is_float_dtype(x_dtype), "quantize_activation_u4 expects floating input");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  DIMQ_CHECK(act_zp >= 0 && act_zp <= 15, "act_zero_point must be in [0, 15]");
  DIMQ_CHECK(numel >= 0, "numel must be non-negative");
  if (numel == 0) return DIMQ_OK;
  const int64_t threads_needed = (numel + 7) / 8;
  const int64_t blocks = (threads_needed + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(quantize_act_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream), x, x_dtype,
                     numel, static_cast<float>(act_scale), static_cast<int>(act_zp), out);
  return check_launch("quantize_activation_u4");
}

extern "C" int dimq_build_product_table_grouped(const void* codebook, int cb_dtype, int64_t groups, int64_t kc,
                                                double act_scale, int64_t act_zp, float* table, void* stream) {
  DIMQ_CHECK(is_float_dtype(cb_dtype), "build_product_table expects floating codebook");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  DIMQ_CHECK(act_zp >= 0 && act_zp <= 15, "act_zero_point must be in [0, 15]");
  DIMQ_CHECK(groups >= 0 && kc > 0, "codebook shape must be positive");
  const int64_t total = groups * kc * 16;
  if (total == 0) return DIMQ_OK;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(product_table_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream), codebook,
                     cb_dtype, total, static_cast<float>(act_scale), static_cast<int>(act_zp), table);
  return check_launch("build_product_table");
}

extern "C" int dimq_build_product_table(const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale,
                                        int64_t act_zp, float* table, void* stream) {
  DIMQ_CHECK(is_float_dtype(cb_dtype), "build_product_table expects floating codebook");
  DIMQ_CHECK(cb_numel == 16, "build_product_table expects exactly 16 codebook entries");
  return dimq_build_product_table_grouped(codebook, cb_dtype, 1, 16, act_scale, act_zp, table, stream);
}

extern "C" int dimq_hard_quantize(const void* w, int w_dtype, int64_t rows, int64_t row_len, const float* centers,
                                  int64_t n_centers, int per_channel, uint8_t* indices, void* values, void* stream) {
  DIMQ_CHECK(w_dtype == DIMQ_F32 || w_dtype == DIMQ_F16 || w_dtype == DIMQ_BF16,
             "hard_quantize expects fp32/fp16/bf16 weights");
  DIMQ_CHECK(n_centers > 0, "centers must be non-empty");
  DIMQ_CHECK(n_centers <= 256, "at most 256 centers are supported (uint8 indices), got %lld",
             (long long)n_centers);
  DIMQ_CHECK(rows >= 0 && row_len >= 0, "weight shape must be non-negative");
  if (rows == 0 || row_len == 0) return DIMQ_OK;
  const int64_t seg = (row_len + kThreads * 4 - 1) / (kThreads * 4);
  const int64_t blocks = rows * seg;
  DIMQ_CHECK(blocks < (int64_t)1 << 31, "weight too large for one launch");
  hipLaunchKernelGGL(hard_quantize_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream), w, w_dtype,
                     rows, row_len, centers, static_cast<int>(n_centers), per_channel ? 1 : 0, indices, values, seg);
  return check_launch("hard_quantize");
}
