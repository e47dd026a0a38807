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
// summation order.  kQa4Groups groups of 8 activations per thread, group u of
// thread t of work-group b at (b * kQa4Groups + u) * kThreads + t (loads
// coalesced per u, all of a thread's loads in flight at once); VEC: x is
// 16-byte aligned (vector loads of the 8 inputs).
template <int XT, bool VEC>
__global__ __launch_bounds__(kThreads) void quantize_a4_f16_kernel(const void* __restrict__ x, int64_t n, float s,
                                                                   int zp, uint16_t* __restrict__ out) {
  quantize_a4_f16_groups<XT, VEC, kQa4Groups>(
      x, n, s, zp, out, static_cast<int64_t>(blockIdx.x) * kThreads * kQa4Groups + threadIdx.x, kThreads);
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

// Nearest centre with torch's argmin semantics on fp32 distances
// d(c) = RN(RN(x - c)^2) (quant/dimq.py:213-214): the first minimum wins, a
// NaN distance beats every number and the first NaN is kept.
//
// RN is monotone, so for a finite x, d(c) does not increase as c rises
// towards x and does not decrease as c rises beyond it: over the centres in
// ascending order the minimum sits at one of x's two neighbours, and the
// centres with that distance form one run around them.  The work-group sorts
// its row's centres in LDS once (rank sort on (value, index)), and each
// element costs a binary search, two distances and a scan of the tied run
// (usually one step), whatever the number of centres.  NaN distances come
// only from NaN centres, a NaN x, or an infinite x meeting the same
// infinity; those cases are answered from the first-index flags below.
struct CentreRow {
  float sv[256];  // centres in ascending order (ties by index)
  int si[256];    // their indices
  float raw[256];
  int first_nan, first_pinf, first_ninf;  // first NaN / +inf / -inf centre, K if none
};

__device__ __forceinline__ float centre_dist(float x, float c) {
#pragma clang fp contract(off)  // one rounding of the square, never fused into a later add
  const float diff = x - c;
  return diff * diff;
}

// Whole work-group: the row's K (1..256) centres into `r`.
__device__ void centre_row_setup(const float* __restrict__ c, int K, CentreRow& r) {
  if (threadIdx.x == 0) {
    r.first_nan = K;
    r.first_pinf = K;
    r.first_ninf = K;
  }
  for (int j = threadIdx.x; j < K; j += blockDim.x) r.raw[j] = c[j];
  __syncthreads();
  for (int j = threadIdx.x; j < K; j += blockDim.x) {
    const float v = r.raw[j];
    if (v != v) atomicMin(&r.first_nan, j);
    if (v == __builtin_inff()) atomicMin(&r.first_pinf, j);
    if (v == -__builtin_inff()) atomicMin(&r.first_ninf, j);
    int rank = 0;
#pragma unroll 8
    for (int i = 0; i < K; ++i) {
      const float u = r.raw[i];
      rank += (u < v) || (u == v && i < j);
    }
    // with a NaN centre ranks can collide; the sorted view is then unused
    r.sv[rank] = v;
    r.si[rank] = j;
  }
  __syncthreads();
}

__device__ __forceinline__ int nearest_centre(float x, const CentreRow& r, int K) {
  if (x != x) return 0;  // every distance NaN
  if (x == __builtin_inff() || x == -__builtin_inff()) {
    // NaN distances: the NaN centres and the centres equal to x; else all inf
    const int f = min(r.first_nan, x > 0.0f ? r.first_pinf : r.first_ninf);
    return f < K ? f : 0;
  }
  if (r.first_nan < K) return r.first_nan;
  int pos = 0;  // number of centres <= x
#pragma unroll
  for (int step = 256; step > 0; step >>= 1)
    if (pos + step <= K && r.sv[pos + step - 1] <= x) pos += step;
  const int L = pos - 1, R = pos;
  const float dl = L >= 0 ? centre_dist(x, r.sv[L]) : 0.0f;
  const float dr = R < K ? centre_dist(x, r.sv[R]) : 0.0f;
  const float ds = L < 0 ? dr : (R >= K ? dl : fminf(dl, dr));
  int best = K;
  if (L >= 0 && dl == ds)
    for (int i = L; i >= 0 && centre_dist(x, r.sv[i]) == ds; --i) best = min(best, r.si[i]);
  if (R < K && dr == ds)
    for (int i = R; i < K && centre_dist(x, r.sv[i]) == ds; ++i) best = min(best, r.si[i]);
  return best;
}

// Nearest-centre assignment of a [rows, row_len] tensor (per_channel: row r
// uses centres[r * K ..]; else one set for all).  One work-group per segment
// of seg_len = 256 * ept elements of a row; writes the index (idx, nullable)
// and / or centres[idx].to(dtype) (values, nullable).  hard_quantize_weight,
// quant/dimq.py:197-221.
__global__ __launch_bounds__(kThreads) void nearest_centre_kernel(const void* __restrict__ w, int dt, int64_t row_len,
                                                                  const float* __restrict__ centers, int K,
                                                                  int per_channel, uint8_t* __restrict__ idx,
                                                                  void* __restrict__ values, int64_t seg_per_row,
                                                                  int ept) {
  __shared__ CentreRow r;
  const int64_t row = static_cast<int64_t>(blockIdx.x) / seg_per_row;
  const int64_t seg = static_cast<int64_t>(blockIdx.x) % seg_per_row;
  const int64_t start = seg * (static_cast<int64_t>(kThreads) * ept);
  // the first element is requested before the centres are sorted
  const float x0 = start + threadIdx.x < row_len ? load_as_float(w, dt, row * row_len + start + threadIdx.x) : 0.0f;
  centre_row_setup(centers + (per_channel ? row * K : 0), K, r);
  for (int q = 0; q < ept; ++q) {
    const int64_t k = start + q * kThreads + threadIdx.x;
    if (k >= row_len) break;
    const int64_t e = row * row_len + k;
    const int best = nearest_centre(q == 0 ? x0 : load_as_float(w, dt, e), r, K);
    if (idx) idx[e] = static_cast<uint8_t>(best);
    if (values) store_from_float(values, dt, e, r.raw[best]);  // centers[idx].to(dtype)
  }
}

// Elements per thread: 1 while that leaves fewer than 2048 work-groups, up to
// 16 for large tensors (the centre sort is paid once per work-group).
inline int nearest_ept(int64_t rows, int64_t row_len) {
  int ept = 1;
  while (ept < 16 && rows * ((row_len + kThreads * ept - 1) / (kThreads * ept)) >= 4096) ept *= 2;
  return ept;
}

int launch_nearest_centre(const void* w, int dt, int64_t rows, int64_t row_len, const float* centers, int K,
                          int per_channel, uint8_t* idx, void* values, hipStream_t st) {
  if (rows == 0 || row_len == 0) return DIMQ_OK;
  const int ept = nearest_ept(rows, row_len);
  const int64_t seg = (row_len + kThreads * ept - 1) / (kThreads * ept);
  const int64_t blocks = rows * seg;
  DIMQ_CHECK(blocks < (int64_t)1 << 31, "tensor too large for one launch");
  hipLaunchKernelGGL(nearest_centre_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, w, dt,
                     row_len, centers, K, per_channel ? 1 : 0, idx, values, seg, ept);
  return check_launch("nearest centre");
}

}  // namespace

// Activation codebook (the QAT wrapper's activation_centers,
// quant/dimq_wrapper.py:80-85 via hard_quantize_weight, quant/dimq.py:197-221):
// out = C_a[argmin_c (x - C_a[c])^2] in x's dtype (K in [1, 256]).
int launch_act_codebook(const void* x, int x_dtype, int64_t n, const float* centers, int K, void* out,
                        hipStream_t st) {
  return launch_nearest_centre(x, x_dtype, 1, n, centers, K, 0, nullptr, out, st);
}

// Launches quantize_a4_f16_kernel; out must be 16-byte aligned.
int launch_quantize_a4_f16(const void* x, int x_dtype, int64_t n, float s, int zp, uint16_t* out, hipStream_t st) {
  if (n == 0) return DIMQ_OK;
  const int64_t blocks = ((n + 7) / 8 + kThreads * kQa4Groups - 1) / (kThreads * kQa4Groups);
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
  return launch_nearest_centre(w, w_dtype, rows, row_len, centers, static_cast<int>(n_centers), per_channel,
                               indices, values, as_stream(stream));
}
