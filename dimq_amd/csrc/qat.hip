// Training-side DIMQ kernels (the QAT step before the packed path):
//  * the Gibbs softmin distortion  L = sum_i -tau (logsumexp_j(-d_ij / tau) - log K),
//    d_ij = (w_i - c_j)^2  (dimq_softmin_loss, quant/dimq.py:244-273), forward and
//    backward;
//  * soft dequantization  out_i = sum_j p_ij c_j,  p_ij = softmax_j(-d_ij / tau)
//    (soft_dequantize_weight, quant/dimq.py:224-241), forward and backward;
//  * the hinge separation loss over centre pairs with margin
//    delta = eta * 6 * std(w) / K  (separation_loss, quant/dimq.py:276-296) and
//    its gradient in the centres.
// Everything is computed in fp32 from w.float() and centres.float(), as the
// reference does.  The centres (K <= 256) sit in LDS.  Exponents are formed as
// -(d_ij - dmin_i) / tau with dmin_i = min_j d_ij (exact 0 at the nearest
// centre, no cancellation of two large terms at small tau), so
//   logsumexp_j(-d_ij / tau) = -dmin_i / tau + log s_i,
//   s_i = sum_j exp(-(d_ij - dmin_i) / tau),   p_ij = exp(-(d_ij - dmin_i) / tau) / s_i,
// and the softmin term is dmin_i - tau log(s_i / K).  For s_i > K / 2
// (near-uniform p: large tau) log(s_i / K) is formed as
// log1p(sum_j expm1(-(d_ij - dmin_i) / tau) / K), since log s_i - log K would
// cancel to a few digits there; otherwise as log s_i - log K.  The forward kernels store
// (dmin_i, log s_i) per element, so a backward pass gets p_ij without a second
// pass over the centres.  Sums over elements (the loss, the centre gradients)
// go through per-work-group partials and a final pass in a fixed order:
// results do not depend on scheduling.
#include "common.h"

namespace dimq {
namespace {

constexpr int kQatThreads = 256;
constexpr int kQatEpt = 4;                         // elements per thread per work-group
constexpr int kQatChunk = kQatThreads * kQatEpt;  // elements per work-group
constexpr int kQatTile = 16;                       // centres per gradient tile

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ void stage_centres(const float* __restrict__ c, int K, float* cs) {
  for (int j = threadIdx.x; j < K; j += kQatThreads) cs[j] = c[j];
}

// (w - c)^2 rounded to fp32 once, as the reference's (w - c).pow(2): never
// contracted into a later subtraction (hipcc contracts a * b - c into an fma
// by default; an exact square there differs from dmin's rounded one, and at
// small tau that difference times 1/tau moves the exponent by O(1))
__device__ __forceinline__ float sqd(float w, float c) {
#pragma clang fp contract(off)
  const float d = w - c;
  return d * d;
}

// Exponent arguments are clamped at -100: exp(-100) is below fp32's smallest
// normal, so no clamped term can change a sum that holds exp(0) = 1, and the
// device exp / expm1 never see arguments of order -(d_ij - dmin_i) / tau at
// tiny tau (-1e7 and beyond), where they are not relied on.
__device__ __forceinline__ float xarg(float d2, float dmin, float inv_tau) {
#pragma clang fp contract(off)
  return fmaxf(-(d2 - dmin) * inv_tau, -100.0f);
}

// (dmin, log(s / K), log s) of element w: its nearest squared distance and
// the logs of its shifted sum of exponentials (log s exactly 0 for a single
// nearest centre, so its p is exactly 1 and out exactly that centre)
__device__ __forceinline__ float3 lse_of(float w, const float* cs, int K, float inv_tau) {
  float dmin = __builtin_inff();
  for (int j = 0; j < K; ++j) dmin = fminf(dmin, sqd(w, cs[j]));
  float s = 0.0f;  // sum_j exp(x_j), x_j = -(d_j - dmin) / tau <= 0: in [1, K]
  for (int j = 0; j < K; ++j) s += expf(xarg(sqd(w, cs[j]), dmin, inv_tau));
  const float fK = static_cast<float>(K);
  const float logK = logf(fK);
  if (s <= 0.5f * fK) {  // |log(s / K)| >= log 2: no cancellation
    const float ls = logf(s);
    return make_float3(dmin, ls - logK, ls);
  }
  float q = 0.0f;  // near-uniform p: sum_j (exp(x_j) - 1), small terms kept exactly
  for (int j = 0; j < K; ++j) q += expm1f(xarg(sqd(w, cs[j]), dmin, inv_tau));
  const float lq = log1pf(q / fK);
  return make_float3(dmin, lq, logK + lq);
}

// p_ij from the element's stored (dmin, log s)
__device__ __forceinline__ float p_of(float d2, float2 a, float inv_tau) {
  return expf(xarg(d2, a.x, inv_tau) - a.y);
}

// MODE 0: softmin loss partials (+ aux);  MODE 1: soft dequantization (+ aux).
template <int MODE>
__global__ __launch_bounds__(kQatThreads) void qat_forward_kernel(const void* __restrict__ w, int wdt, int64_t n,
                                                                  const float* __restrict__ c, int K, float inv_tau,
                                                                  float tau, float2* __restrict__ aux,
                                                                  float* __restrict__ partial, void* __restrict__ out) {
  __shared__ float cs[256];
  __shared__ float red[4];
  stage_centres(c, K, cs);
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kQatChunk;
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < kQatEpt; ++e) {
    const int64_t i = base + e * kQatThreads + threadIdx.x;
    if (i >= n) break;
    const float wi = load_as_float(w, wdt, i);
    const float3 l = lse_of(wi, cs, K, inv_tau);
    const float2 a = make_float2(l.x, l.z);  // (dmin, log s)
    if (aux) aux[i] = a;
    if (MODE == 0) {
      acc += l.x - tau * l.y;
    } else {
      float v = 0.0f;
      for (int j = 0; j < K; ++j) v += p_of(sqd(wi, cs[j]), a, inv_tau) * cs[j];
      store_from_float(out, wdt, i, v);
    }
  }
  if (MODE == 0) {
    const float s = block_sum(acc, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = s;
  }
}

// Backward of both forwards, tile by tile over the centres (16 gradient
// accumulators per thread, reduced over the work-group per tile):
//   MODE 0 (softmin, upstream scalar g):
//     dL/dw_i = g sum_j p_ij 2 (w_i - c_j),   dL/dc_j = -2 g sum_i p_ij (w_i - c_j)
//   MODE 1 (soft dequantization, upstream g_i, out_i = sum_j p_ij c_j):
//     dL/dw_i = g_i sum_j p_ij (c_j - out_i) (-2 (w_i - c_j) / tau)
//     dL/dc_j = sum_i g_i p_ij (1 + (c_j - out_i) 2 (w_i - c_j) / tau)
template <int MODE>
__global__ __launch_bounds__(kQatThreads) void qat_backward_kernel(const void* __restrict__ w, int wdt, int64_t n,
                                                                   const float* __restrict__ c, int K, float inv_tau,
                                                                   const float2* __restrict__ aux,
                                                                   const float* __restrict__ gscalar,
                                                                   const void* __restrict__ gout, int gdt,
                                                                   void* __restrict__ grad_w, int gwdt,
                                                                   float* __restrict__ partial) {
  __shared__ float cs[256];
  __shared__ float red[4][kQatTile];
  stage_centres(c, K, cs);
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kQatChunk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float wv[kQatEpt], gv[kQatEpt], ov[kQatEpt], gw[kQatEpt];
  float2 lv[kQatEpt];
  const float g0 = MODE == 0 ? *gscalar : 0.0f;
#pragma unroll
  for (int e = 0; e < kQatEpt; ++e) {
    const int64_t i = base + e * kQatThreads + threadIdx.x;
    const bool ok = i < n;
    wv[e] = ok ? load_as_float(w, wdt, i) : 0.0f;
    lv[e] = ok ? aux[i] : make_float2(0.0f, __builtin_inff());  // p = 0 for elements past the end
    gv[e] = MODE == 0 ? g0 : (ok ? load_as_float(gout, gdt, i) : 0.0f);
    gw[e] = 0.0f;
    ov[e] = 0.0f;
  }
  if (MODE == 1) {  // out_i again (the forward's value before its rounding to w's dtype)
    for (int j = 0; j < K; ++j)
#pragma unroll
      for (int e = 0; e < kQatEpt; ++e) ov[e] += p_of(sqd(wv[e], cs[j]), lv[e], inv_tau) * cs[j];
  }
  const float two_tau = 2.0f * inv_tau;
  for (int t0 = 0; t0 < K; t0 += kQatTile) {
    float gc[kQatTile];
#pragma unroll
    for (int u = 0; u < kQatTile; ++u) gc[u] = 0.0f;
#pragma unroll
    for (int u = 0; u < kQatTile; ++u) {
      const int j = t0 + u;
      if (j >= K) break;
      const float cj = cs[j];
#pragma unroll
      for (int e = 0; e < kQatEpt; ++e) {
        const float d = wv[e] - cj;
        const float pij = p_of(sqd(wv[e], cj), lv[e], inv_tau);
        if (MODE == 0) {
          gw[e] += pij * (2.0f * d);
          gc[u] += pij * d;
        } else {
          const float q = gv[e] * pij;
          gw[e] += q * (cj - ov[e]) * (-two_tau * d);
          gc[u] += q * (1.0f + (cj - ov[e]) * (two_tau * d));
        }
      }
    }
    // the tile's 16 sums over the work-group's elements
#pragma unroll
    for (int u = 0; u < kQatTile; ++u) {
      float v = gc[u];
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
      gc[u] = v;
    }
    if (lane == 0)
#pragma unroll
      for (int u = 0; u < kQatTile; ++u) red[wave][u] = gc[u];
    __syncthreads();
    if (threadIdx.x < kQatTile && t0 + threadIdx.x < K) {
      const int u = threadIdx.x;
      const float s = (red[0][u] + red[1][u]) + (red[2][u] + red[3][u]);
      partial[static_cast<int64_t>(blockIdx.x) * K + t0 + u] = MODE == 0 ? -2.0f * g0 * s : s;
    }
    __syncthreads();
  }
#pragma unroll
  for (int e = 0; e < kQatEpt; ++e) {
    const int64_t i = base + e * kQatThreads + threadIdx.x;
    if (i < n && grad_w) store_from_float(grad_w, gwdt, i, MODE == 0 ? g0 * gw[e] : gw[e]);
  }
}

// out[j] = scale * sum over the `rows` partial rows of column j, in row order
// (one thread per column; rows of a column are summed pairwise in blocks of
// 64 for accuracy, then the block sums in order).
__global__ __launch_bounds__(256) void qat_reduce_kernel(const float* __restrict__ partial, int64_t rows, int cols,
                                                         float scale, float* __restrict__ out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= cols) return;
  float total = 0.0f;
  for (int64_t r0 = 0; r0 < rows; r0 += 64) {
    float s = 0.0f;
    const int64_t r1 = r0 + 64 < rows ? r0 + 64 : rows;
    for (int64_t r = r0; r < r1; ++r) s += partial[r * cols + j];
    total += s;
  }
  out[j] = total * scale;
}

// sum(w) and sum((w - mean)^2) partials: the population std of w
// (std(unbiased=False)) in two passes.
__global__ __launch_bounds__(kQatThreads) void moments_kernel(const void* __restrict__ w, int wdt, int64_t n,
                                                              const float* __restrict__ mean, float* __restrict__ partial) {
  __shared__ float red[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kQatChunk;
  const float mu = mean ? *mean : 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < kQatEpt; ++e) {
    const int64_t i = base + e * kQatThreads + threadIdx.x;
    if (i >= n) break;
    const float v = load_as_float(w, wdt, i);
    acc += mean ? (v - mu) * (v - mu) : v;
  }
  const float s = block_sum(acc, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

// Separation loss and its gradient in the centres (one work-group):
//   delta = eta * 6 * max(sqrt(var), 1e-12) / K,
//   L = sum_{a<b} relu(delta - sqrt((c_a - c_b)^2 + eps))^2,
//   dL/dc_a = sum_{b != a} -2 relu(delta - r_ab) (c_a - c_b) / r_ab.
__global__ __launch_bounds__(kQatThreads) void separation_kernel(const float* __restrict__ c, int K,
                                                                 const float* __restrict__ var, float eta, float eps,
                                                                 float* __restrict__ loss, float* __restrict__ grad_c) {
  __shared__ float cs[256];
  __shared__ float red[4];
  stage_centres(c, K, cs);
  __syncthreads();
  const float sigma = fmaxf(sqrtf(*var), 1e-12f);
  const float delta = eta * 6.0f * sigma / static_cast<float>(K);
  float acc = 0.0f;
  for (int a = threadIdx.x; a < K; a += kQatThreads) {
    float g = 0.0f;
    for (int b = 0; b < K; ++b) {
      if (b == a) continue;
      const float diff = cs[a] - cs[b];
      const float r = sqrtf(diff * diff + eps);
      const float h = fmaxf(delta - r, 0.0f);
      if (b > a) acc += h * h;
      g += -2.0f * h * diff / r;
    }
    if (grad_c) grad_c[a] = g;
  }
  const float s = block_sum(acc, red);
  if (threadIdx.x == 0) *loss = s;
}

inline int64_t qat_blocks(int64_t n) { return (n + kQatChunk - 1) / kQatChunk; }

}  // namespace
}  // namespace dimq

using namespace dimq;

extern "C" int64_t dimq_qat_workspace_bytes(int64_t n, int64_t n_centers) {
  if (n < 0 || n_centers < 1) return -1;
  const int64_t blocks = qat_blocks(n > 0 ? n : 1);
  return blocks * (n_centers > 1 ? n_centers : 1) * static_cast<int64_t>(sizeof(float)) + 256;
}

static int qat_check(const void* w, int w_dtype, int64_t n, const float* centers, int64_t K, double tau) {
  DIMQ_CHECK(w_dtype == DIMQ_F32 || w_dtype == DIMQ_F16 || w_dtype == DIMQ_BF16 || w_dtype == DIMQ_F64,
             "weights must be fp32, fp16, bf16 or fp64");
  DIMQ_CHECK(n >= 0, "the weight size must be non-negative");
  DIMQ_CHECK(n == 0 || w != nullptr, "weights are required");
  DIMQ_CHECK(centers != nullptr && K >= 1 && K <= 256, "centers must hold between 1 and 256 values");
  DIMQ_CHECK(tau > 0.0, "tau must be positive (the reference clamps it to at least 1e-12)");
  DIMQ_CHECK(qat_blocks(n) < (int64_t)1 << 31, "weights too large for one launch");
  return DIMQ_OK;
}

extern "C" int dimq_softmin_loss_forward(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                                         double tau, int mean_reduction, float* aux, float* loss, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  int rc = qat_check(w, w_dtype, n, centers, n_centers, tau);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(loss != nullptr, "loss output is required");
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= dimq_qat_workspace_bytes(n, n_centers),
             "workspace must hold dimq_qat_workspace_bytes bytes");
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  const int64_t blocks = qat_blocks(n);
  if (n == 0) {
    hipLaunchKernelGGL(qat_reduce_kernel, dim3(1), dim3(256), 0, s, partial, (int64_t)0, 1, 0.0f, loss);
    return check_launch("softmin loss");
  }
  const float t = static_cast<float>(tau);
  hipLaunchKernelGGL(qat_forward_kernel<0>, dim3(static_cast<unsigned>(blocks)), dim3(kQatThreads), 0, s, w, w_dtype,
                     n, centers, static_cast<int>(n_centers), 1.0f / t, t, reinterpret_cast<float2*>(aux), partial,
                     nullptr);
  rc = check_launch("softmin loss");
  if (rc != DIMQ_OK) return rc;
  hipLaunchKernelGGL(qat_reduce_kernel, dim3(1), dim3(256), 0, s, partial, blocks, 1,
                     mean_reduction ? 1.0f / static_cast<float>(n) : 1.0f, loss);
  return check_launch("softmin loss (sum)");
}

extern "C" int dimq_softmin_loss_backward(const void* w, int w_dtype, int64_t n, const float* centers,
                                          int64_t n_centers, double tau, int mean_reduction, const float* aux,
                                          const float* grad_loss, void* grad_w, int grad_w_dtype, float* grad_centers,
                                          void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = qat_check(w, w_dtype, n, centers, n_centers, tau);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(aux != nullptr && grad_loss != nullptr, "the forward's aux and the loss gradient are required");
  DIMQ_CHECK(grad_w == nullptr || is_float_dtype(grad_w_dtype), "grad_w must be floating point");
  DIMQ_CHECK(grad_centers != nullptr, "grad_centers is required");
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= dimq_qat_workspace_bytes(n, n_centers),
             "workspace must hold dimq_qat_workspace_bytes bytes");
  DIMQ_CHECK(!mean_reduction, "the mean reduction's backward is the sum's scaled by 1/n: pass the scaled gradient");
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  const int64_t blocks = n > 0 ? qat_blocks(n) : 0;
  const int K = static_cast<int>(n_centers);
  if (blocks > 0) {
    hipLaunchKernelGGL(qat_backward_kernel<0>, dim3(static_cast<unsigned>(blocks)), dim3(kQatThreads), 0, s, w,
                       w_dtype, n, centers, K, static_cast<float>(1.0 / tau), reinterpret_cast<const float2*>(aux),
                       grad_loss, nullptr, 0, grad_w,
                       grad_w_dtype, partial);
    rc = check_launch("softmin loss backward");
    if (rc != DIMQ_OK) return rc;
  }
  hipLaunchKernelGGL(qat_reduce_kernel, dim3((K + 255) / 256), dim3(256), 0, s, partial, blocks, K, 1.0f, grad_centers);
  return check_launch("softmin loss backward (centres)");
}

extern "C" int dimq_soft_dequantize_forward(const void* w, int w_dtype, int64_t n, const float* centers,
                                            int64_t n_centers, double tau, void* out, float* aux, void* stream) {
  int rc = qat_check(w, w_dtype, n, centers, n_centers, tau);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(n == 0 || (out != nullptr && aux != nullptr), "out and aux are required");
  if (n == 0) return DIMQ_OK;
  const float t = static_cast<float>(tau);
  hipLaunchKernelGGL(qat_forward_kernel<1>, dim3(static_cast<unsigned>(qat_blocks(n))), dim3(kQatThreads), 0,
                     as_stream(stream), w, w_dtype, n, centers, static_cast<int>(n_centers), 1.0f / t, t,
                     reinterpret_cast<float2*>(aux), nullptr, out);
  return check_launch("soft dequantize");
}

extern "C" int dimq_soft_dequantize_backward(const void* w, int w_dtype, int64_t n, const float* centers,
                                             int64_t n_centers, double tau, const float* aux, const void* grad_out,
                                             int grad_out_dtype, void* grad_w, int grad_w_dtype, float* grad_centers,
                                             void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = qat_check(w, w_dtype, n, centers, n_centers, tau);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(n == 0 || (aux != nullptr && grad_out != nullptr), "the forward's aux and grad_out are required");
  DIMQ_CHECK(is_float_dtype(grad_out_dtype), "grad_out must be floating point");
  DIMQ_CHECK(grad_w == nullptr || is_float_dtype(grad_w_dtype), "grad_w must be floating point");
  DIMQ_CHECK(grad_centers != nullptr, "grad_centers is required");
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= dimq_qat_workspace_bytes(n, n_centers),
             "workspace must hold dimq_qat_workspace_bytes bytes");
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  const int64_t blocks = n > 0 ? qat_blocks(n) : 0;
  const int K = static_cast<int>(n_centers);
  if (blocks > 0) {
    hipLaunchKernelGGL(qat_backward_kernel<1>, dim3(static_cast<unsigned>(blocks)), dim3(kQatThreads), 0, s, w,
                       w_dtype, n, centers, K, static_cast<float>(1.0 / tau), reinterpret_cast<const float2*>(aux),
                       nullptr, grad_out, grad_out_dtype,
                       grad_w, grad_w_dtype, partial);
    rc = check_launch("soft dequantize backward");
    if (rc != DIMQ_OK) return rc;
  }
  hipLaunchKernelGGL(qat_reduce_kernel, dim3((K + 255) / 256), dim3(256), 0, s, partial, blocks, K, 1.0f, grad_centers);
  return check_launch("soft dequantize backward (centres)");
}

extern "C" int dimq_separation_loss(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                                    double eta, double eps, float* loss, float* grad_centers, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  int rc = qat_check(w, w_dtype, n, centers, n_centers, 1.0);
  if (rc != DIMQ_OK) return rc;
  DIMQ_CHECK(n >= 1, "separation_loss needs a non-empty weight (its margin is a multiple of std(w))");
  DIMQ_CHECK(loss != nullptr, "loss output is required");
  DIMQ_CHECK(workspace != nullptr && workspace_bytes >= dimq_qat_workspace_bytes(n, n_centers),
             "workspace must hold dimq_qat_workspace_bytes bytes");
  DIMQ_CHECK(eps >= 0.0, "eps must be non-negative");
  const hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  float* stats = reinterpret_cast<float*>(static_cast<char*>(workspace) + workspace_bytes - 64);  // mean, var
  stats = reinterpret_cast<float*>(reinterpret_cast<uintptr_t>(stats) & ~uintptr_t(15));
  const int64_t blocks = n > 0 ? qat_blocks(n) : 0;
  // mean, then the mean of squared deviations (torch's std(unbiased=False) of w.float())
  if (blocks > 0) {
    hipLaunchKernelGGL(moments_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kQatThreads), 0, s, w, w_dtype, n,
                       nullptr, partial);
    rc = check_launch("separation loss (mean)");
    if (rc != DIMQ_OK) return rc;
  }
  const float inv_n = n > 0 ? 1.0f / static_cast<float>(n) : 0.0f;
  hipLaunchKernelGGL(qat_reduce_kernel, dim3(1), dim3(256), 0, s, partial, blocks, 1, inv_n, stats);
  if (blocks > 0) {
    hipLaunchKernelGGL(moments_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kQatThreads), 0, s, w, w_dtype, n,
                       stats, partial);
    rc = check_launch("separation loss (variance)");
    if (rc != DIMQ_OK) return rc;
  }
  hipLaunchKernelGGL(qat_reduce_kernel, dim3(1), dim3(256), 0, s, partial, blocks, 1, inv_n, stats + 1);
  hipLaunchKernelGGL(separation_kernel, dim3(1), dim3(kQatThreads), 0, s, centers, static_cast<int>(n_centers),
                     stats + 1, static_cast<float>(eta), static_cast<float>(eps), loss, grad_centers);
  return check_launch("separation loss");
}
