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

// W4A4 activations for the weight-only kernels: out = fp16(q - zp) with
// q = clamp(rint(x / s) + zp, 0, 15), the same code as quantize_act_kernel.
// q - zp is an integer in [-15, 15], exact in fp16, so a weight-only GEMM/conv
// over these values times s equals sum_k C[w] * (s * (a - zp)) up to fp32
// summation order.  8 activations per thread, one 16-byte store; VEC: x is
// 16-byte aligned (vector loads of the 8 inputs).
template <int XT, bool VEC>
__global__ __launch_bounds__(kThreads) void quantize_a4_f16_kernel(const void* __restrict__ x, int64_t n, float s,
                                                                   int zp, uint16_t* __restrict__ out) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;
  if (base >= n) return;
  if (base + 8 <= n) {
    float v[8];
    if constexpr (VEC && XT == DIMQ_F32) {
      const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base)[0];
      const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else if constexpr (VEC && (XT == DIMQ_F16 || XT == DIMQ_BF16)) {
      const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = XT == DIMQ_F16 ? f16_bits_to_float(w[j] & 0xffffu) : bf16_bits_to_float(w[j] & 0xffffu);
        v[2 * j + 1] = XT == DIMQ_F16 ? f16_bits_to_float(w[j] >> 16) : bf16_bits_to_float(w[j] >> 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = load_as_float(x, XT, base + j);
    }
    u4_codes<8>(v, s, zp);
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = f16x2_rne(v[2 * j], v[2 * j + 1]);
    *reinterpret_cast<uint4*>(out + base) = make_uint4(h[0], h[1], h[2], h[3]);
  } else {
    for (int64_t i = base; i < n; ++i) {
      const float v = load_as_float(x, XT, i);
      out[i] = (uint16_t)float_to_f16_bits((float)(quantize_u4(v, s, zp) - zp));
    }
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

// Activation codebook (the QAT wrapper's activation_centers,
// quant/dimq_wrapper.py:80-85 via hard_quantize_weight, quant/dimq.py:197-221):
// out = C_a[argmin_c (x - C_a[c])^2] in x's dtype, with hard_quantize_kernel's torch
// argmin semantics (first minimum; a NaN distance wins, the first NaN kept).
// 4 activations per thread, the K <= 256 centres in LDS.
__global__ __launch_bounds__(kThreads) void act_codebook_kernel(const void* __restrict__ x, int dt, int64_t n,
                                                                const float* __restrict__ centers, int K,
                                                                void* __restrict__ out) {
  __shared__ float c_s[256];
  for (int j = threadIdx.x; j < K; j += kThreads) c_s[j] = centers[j];
  __syncthreads();
  const int64_t start = static_cast<int64_t>(blockIdx.x) * (kThreads * 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t e = start + r * kThreads + threadIdx.x;
    if (e >= n) break;
    const float v = load_as_float(x, dt, e);
    int best = 0;
    float best_d = __builtin_inff();
    bool have = false;
    bool have_nan = false;
    for (int j = 0; j < K; ++j) {
      const float diff = v - c_s[j];
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
    store_from_float(out, dt, e, c_s[best]);  // centers[idx].to(x.dtype)
  }
}

}  // namespace

// Launches act_codebook_kernel (K in [1, 256]); out holds n elements of x_dtype.
int launch_act_codebook(const void* x, int x_dtype, int64_t n, const float* centers, int K, void* out,
                        hipStream_t st) {
  if (n == 0) return DIMQ_OK;
  const int64_t blocks = (n + kThreads * 4 - 1) / (kThreads * 4);
  DIMQ_CHECK(blocks < (int64_t)1 << 31, "activations too large for one launch");
  hipLaunchKernelGGL(act_codebook_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, x, x_dtype,
                     n, centers, K, out);
  return check_launch("activation codebook");
}

// Launches quantize_a4_f16_kernel; out must be 16-byte aligned.
int launch_quantize_a4_f16(const void* x, int x_dtype, int64_t n, float s, int zp, uint16_t* out, hipStream_t st) {
  if (n == 0) return DIMQ_OK;
  const int64_t blocks = ((n + 7) / 8 + kThreads - 1) / kThreads;
  const bool vec = aligned(x, 16);
  const dim3 grid(static_cast<unsigned>(blocks));
#define DIMQ_QA4(XT)                                                                                 \
  if (vec)                                                                                           \
    hipLaunchKernelGGL((quantize_a4_f16_kernel<XT, true>), grid, dim3(kThreads), 0, st, x, n, s, zp, out); \
  else                                                                                               \
    hipLaunchKernelGGL((quantize_a4_f16_kernel<XT, false>), grid, dim3(kThreads), 0, st, x, n, s, zp, out)
  switch (x_dtype) {
    case DIMQ_F32: DIMQ_QA4(DIMQ_F32); break;
    case DIMQ_F16: DIMQ_QA4(DIMQ_F16); break;
    case DIMQ_BF16: DIMQ_QA4(DIMQ_BF16); break;
    default: hipLaunchKernelGGL((quantize_a4_f16_kernel<DIMQ_F64, false>), grid, dim3(kThreads), 0, st, x, n, s, zp,
                                out); break;
  }
#undef DIMQ_QA4
  return check_launch("quantize activations (W4A4 fast path)");
}

}  // namespace dimq

using namespace dimq;

// The W4A4 input form of a tensor: out = fp16(q - zp), q the reference's u4
// code (reference.py:11-21).  Entry point of a chain of W4A4 layers whose
// later inputs come from the quantizing epilogue of the layer before.
extern "C" int dimq_quantize_activation_f16(const void* x, int x_dtype, int64_t numel, double act_scale,
                                            int64_t act_zp, uint16_t* out, void* stream) {
  DIMQ_CHECK(is_float_dtype(x_dtype), "quantize_activation expects floating input");
  DIMQ_CHECK(act_scale > 0.0, "act_scale must be positive");
  DIMQ_CHECK(act_zp >= 0 && act_zp <= 15, "act_zero_point must be in [0, 15]");
  DIMQ_CHECK(numel >= 0, "numel must be non-negative");
  DIMQ_CHECK(aligned(out, 16), "out must be 16-byte aligned");
  return launch_quantize_a4_f16(x, x_dtype, numel, static_cast<float>(act_scale), static_cast<int>(act_zp), out,
                                as_stream(stream));
}

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
