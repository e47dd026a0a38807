// LayerNorm over the last dimension for the ViT-B/16 workload (its 25
// LayerNorms, eps 1e-6, bf16 activations): y = (x - mean) * rstd * w + b with
// mean and variance in fp32 over each row (biased variance, as
// torch.nn.functional.layer_norm), one rounding to the output dtype (the
// input's, or fp16 / bf16 for a consumer that wants the other format: the
// ViT workload's LayerNorms feed fp16 to the codebook GEMMs).
//
// One wave per row at a time: lane l holds 16-byte chunks l, l + 64, ... of
// the row in registers, so the row is read from HBM once; the mean and then
// the sum of squared deviations are two wave reductions over those registers
// (two-pass, no cancellation), and the normalised row leaves as 16-byte
// stores.  Weight and bias chunks are loaded once per wave (vector loads)
// and kept in registers while the wave walks its rows.
#include "common.h"

namespace dimq {
namespace {

constexpr int kRowsPerBlock = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ uint32_t to_bits16(float v, int dt) {
  return dt == DIMQ_F16 ? float_to_f16_bits(v) : float_to_bf16_bits(v);
}

// 8 consecutive values of a [D] parameter vector as floats (k0 % 8 == 0).
template <int WT>
__device__ __forceinline__ void load8_param(const void* p, int k0, float out[8]) {
  if (p == nullptr) {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = 0.0f;
  } else if constexpr (WT == DIMQ_F32) {
    const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(p) + k0)[0];
    const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(p) + k0)[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + k0);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = WT == DIMQ_F16 ? f16_bits_to_float(u[j] & 0xffffu) : bf16_bits_to_float(u[j] & 0xffffu);
      out[2 * j + 1] = WT == DIMQ_F16 ? f16_bits_to_float(u[j] >> 16) : bf16_bits_to_float(u[j] >> 16);
    }
  }
}

// NCH: 16-byte chunks (8 elements) per lane; D <= 512 * NCH.  Each wave
// keeps its lanes' weight and bias chunks in registers and walks rows
// row0, row0 + stride, ...; the next row's loads are issued before the
// current row's reductions.
template <int XT, int WT, int YT, int NCH>
__global__ __launch_bounds__(256) void layer_norm_kernel(const void* __restrict__ x, int64_t ldx, int64_t rows, int D,
                                                         const void* __restrict__ w, const void* __restrict__ b,
                                                         float eps, void* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform per wave
  const int nchunk = D >> 3;
  float wv[NCH][8], bv[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int q = lane + 64 * c < nchunk ? lane + 64 * c : 0;
    load8_param<WT>(w, 8 * q, wv[c]);
    if (w == nullptr) {
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[c][j] = 1.0f;
    }
    load8_param<WT>(b, 8 * q, bv[c]);
  }
  // Row r's chunks, loaded without a branch: chunks past the row re-read its
  // last chunk and are zeroed by a select, and the prefetch past the last row
  // re-reads the last row.  With a branch around the loads the compiler waited
  // for every load in flight, the prefetched row's included, before the
  // current row's reductions (ViT shape, same process: 12.2 -> 11.4 us).  Two
  // rows per wave at a time (32 lanes per row, no idle lanes at D = 768) was
  // slower: 12.4 us.
  auto load_row = [&](int64_t r, uint4 v[NCH]) {
    const uint16_t* xr = static_cast<const uint16_t*>(x) + r * ldx;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int q = lane + 64 * c;
      const uint4 t = *reinterpret_cast<const uint4*>(xr + 8 * (q < nchunk ? q : nchunk - 1));
      const uint32_t m = q < nchunk ? 0xffffffffu : 0u;
      v[c] = make_uint4(t.x & m, t.y & m, t.z & m, t.w & m);
    }
  };
  const float inv_d = 1.0f / static_cast<float>(D);
  uint4 cur[NCH];
  load_row(row, cur);
  for (; row < rows; row += stride) {
    uint4 nxt[NCH];
    load_row(row + stride < rows ? row + stride : rows - 1, nxt);
    float f[NCH][8];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint32_t u[4] = {cur[c].x, cur[c].y, cur[c].z, cur[c].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[c][2 * j] = XT == DIMQ_F16 ? f16_bits_to_float(u[j] & 0xffffu) : bf16_bits_to_float(u[j] & 0xffffu);
        f[c][2 * j + 1] = XT == DIMQ_F16 ? f16_bits_to_float(u[j] >> 16) : bf16_bits_to_float(u[j] >> 16);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += f[c][j];  // chunks past the row hold zeros
    }
    const float mean = wave_sum(s) * inv_d;
    float sq = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (lane + 64 * c < nchunk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float d = f[c][j] - mean;
          sq += d * d;
        }
      }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(sq) * inv_d + eps);
    uint16_t* yr = static_cast<uint16_t*>(y) + row * static_cast<int64_t>(D);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int q = lane + 64 * c;
      if (q >= nchunk) continue;
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[j] = to_bits16((f[c][2 * j] - mean) * rstd * wv[c][2 * j] + bv[c][2 * j], YT) |
               (to_bits16((f[c][2 * j + 1] - mean) * rstd * wv[c][2 * j + 1] + bv[c][2 * j + 1], YT) << 16);
      }
      *reinterpret_cast<uint4*>(yr + 8 * q) = make_uint4(o[0], o[1], o[2], o[3]);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) cur[c] = nxt[c];
  }
}

template <int XT, int WT, int YT>
void launch_ln(const void* x, int64_t ldx, int64_t rows, int D, const void* w, const void* b, float eps, void* y,
               hipStream_t s) {
  // about 3 rows per wave at the ViT shape (12,608 rows): 1024 work-groups of 4 waves
  const int64_t want = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const dim3 grid(static_cast<unsigned>(want < 1024 ? want : 1024));
  if (D <= 512)
    hipLaunchKernelGGL((layer_norm_kernel<XT, WT, YT, 1>), grid, dim3(256), 0, s, x, ldx, rows, D, w, b, eps, y);
  else if (D <= 1024)
    hipLaunchKernelGGL((layer_norm_kernel<XT, WT, YT, 2>), grid, dim3(256), 0, s, x, ldx, rows, D, w, b, eps, y);
  else
    hipLaunchKernelGGL((layer_norm_kernel<XT, WT, YT, 4>), grid, dim3(256), 0, s, x, ldx, rows, D, w, b, eps, y);
}

template <int XT, int YT>
void launch_ln_w(const void* x, int64_t ldx, int64_t rows, int D, const void* w, const void* b, int wdt, float eps,
                 void* y, hipStream_t s) {
  switch (wdt) {
    case DIMQ_F32: launch_ln<XT, DIMQ_F32, YT>(x, ldx, rows, D, w, b, eps, y, s); break;
    case DIMQ_F16: launch_ln<XT, DIMQ_F16, YT>(x, ldx, rows, D, w, b, eps, y, s); break;
    default: launch_ln<XT, DIMQ_BF16, YT>(x, ldx, rows, D, w, b, eps, y, s); break;
  }
}

}  // namespace
}  // namespace dimq

using namespace dimq;

extern "C" int dimq_layer_norm_ex(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx,
                                  const void* weight, const void* bias, int wb_dtype, double eps, void* y, int y_dtype,
                                  void* stream) {
  DIMQ_CHECK(x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16, "layer_norm expects fp16 or bf16 input");
  DIMQ_CHECK(y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16, "layer_norm writes fp16 or bf16 output");
  DIMQ_CHECK(rows >= 0 && dim > 0, "layer_norm dimensions must be positive");
  DIMQ_CHECK(dim % 8 == 0 && dim <= 2048, "layer_norm supports a normalized size that is a multiple of 8, at most 2048");
  DIMQ_CHECK(ldx >= dim && ldx % 8 == 0, "layer_norm row stride must be a multiple of 8 and at least dim");
  DIMQ_CHECK(aligned(x, 16) && aligned(y, 16), "layer_norm needs 16-byte aligned input and output");
  DIMQ_CHECK((weight == nullptr && bias == nullptr) ||
                 wb_dtype == DIMQ_F32 || wb_dtype == DIMQ_F16 || wb_dtype == DIMQ_BF16,
             "layer_norm weight and bias must be fp32, fp16 or bf16");
  DIMQ_CHECK(aligned(weight, 16) && aligned(bias, 16), "layer_norm needs 16-byte aligned weight and bias");
  DIMQ_CHECK(eps >= 0.0, "layer_norm eps must be non-negative");
  DIMQ_CHECK(rows / kRowsPerBlock < (int64_t)1 << 31, "layer_norm: too many rows for one launch");
  if (rows == 0) return DIMQ_OK;
  const hipStream_t s = as_stream(stream);
  const float e = static_cast<float>(eps);
  const int D = static_cast<int>(dim);
  if (x_dtype == DIMQ_F16 && y_dtype == DIMQ_F16)
    launch_ln_w<DIMQ_F16, DIMQ_F16>(x, ldx, rows, D, weight, bias, wb_dtype, e, y, s);
  else if (x_dtype == DIMQ_F16)
    launch_ln_w<DIMQ_F16, DIMQ_BF16>(x, ldx, rows, D, weight, bias, wb_dtype, e, y, s);
  else if (y_dtype == DIMQ_F16)
    launch_ln_w<DIMQ_BF16, DIMQ_F16>(x, ldx, rows, D, weight, bias, wb_dtype, e, y, s);
  else
    launch_ln_w<DIMQ_BF16, DIMQ_BF16>(x, ldx, rows, D, weight, bias, wb_dtype, e, y, s);
  return check_launch("layer_norm");
}

extern "C" int dimq_layer_norm(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx,
                               const void* weight, const void* bias, int wb_dtype, double eps, void* y,
                               void* stream) {
  return dimq_layer_norm_ex(x, x_dtype, rows, dim, ldx, weight, bias, wb_dtype, eps, y, x_dtype, stream);
}
