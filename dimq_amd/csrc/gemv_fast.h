// Decode-shape codebook GEMV (M <= 16): y[M,N] = x[M,K] W_hat^T + b, the
// HBM-bound case of BASELINE cfg5 (W 4096x4096 3-bit: 6.3 MB of indices).
//
// Work-group = 16 waves on 16 output columns; wave w owns k-range
// [w*K/16, (w+1)*K/16) and lane group g = lane / 16 a contiguous quarter of
// it, so each lane's weight indices and activations are contiguous in memory.
// Every load of the wave (the lane's K/64 packed indices: 24 bytes at 3 bits;
// its activation row slice: 128 bytes at bf16) is issued before any compute,
// so the whole weight stream is in flight at once.  Loads retire in order,
// so the codebook values and the activations are loaded *before* the weight
// stream: the waits for them (codebook planes, activation conversion) do not
// wait for the weights, and that VALU work runs while the weights stream in
// (measured at cfg5 M = 1: the codebook and activations issued after the
// weights left every VALU phase serial behind the last weight byte).  The 16x16x32 MFMA's k
// dimension takes 8 consecutive k from each lane group (any k order works as
// long as the activation and weight lanes agree); rows m >= M are zero.  The
// 16 partial sums are reduced through LDS.
#pragma once

#include "gemm_big.h"

namespace dimq {
namespace {

template <int BITS, int XT>
__global__ __launch_bounds__(1024) void gemv_fast_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int WAVES = 16;
  constexpr int KL = 64;  // k per lane and round; a round covers 16 waves x 4 lane groups x 64 = 4096 k
  constexpr int E = 1 << BITS;
  __shared__ floatx4 red[WAVES][64];
  __shared__ float cbs[16 * E];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t n = n0 + col < p.N ? n0 + col : p.N - 1;
  const int rounds = static_cast<int>(p.K / (KL * WAVES * 4));  // k-ranges of KL per lane

  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const bool arow = col < p.M;
  CodebookRegs<BITS> cb;
  float colscale = 1.0f;
  // codebook value tid of the 16 rows (as stage_codebook: 0 past cb_size or N)
  const int cb_total = ((p.cb_rows == 1) ? 1 : 16) * E;
  float cbv = 0.0f;
  if (tid < cb_total) {
    const int rr = tid / E, j = tid - (tid / E) * E;
    const int64_t row = (p.cb_rows == 1) ? 0 : n0 + rr;
    if (j < p.cb_size && (p.cb_rows == 1 || row < p.N)) cbv = load_as_float(p.cb, p.cb_dt, row * p.cb_size + j);
  }
  for (int r = 0; r < rounds; ++r) {
    const int64_t k0 = ((int64_t)(r * WAVES + wave) * 4 + g) * KL;
    // ---- all loads of the round first: activations, then the weight stream
    RawA<XT> ra[KL / 16];
    {
#pragma unroll
      for (int h = 0; h < KL / 16; ++h) {
        if (arow) {
          issue_a16<XT>(p.x, (int64_t)col * p.ldx + k0 + 16 * h, ra[h]);
        } else {
#pragma unroll
          for (int w = 0; w < RawA<XT>::kWords; ++w) ra[h].w[w] = 0u;
        }
      }
    }
    uint32_t bw[KL * BITS / 32];
    {
      const uint8_t* src = p.w + (((n * p.K + k0) * BITS) >> 3);
      if constexpr (BITS == 3) {
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const uint2 t = reinterpret_cast<const uint2*>(src)[q];
          bw[2 * q] = t.x;
          bw[2 * q + 1] = t.y;
        }
      } else {
#pragma unroll
        for (int q = 0; q < BITS / 2; ++q) {
          const uint4 t = reinterpret_cast<const uint4*>(src)[q];
          bw[4 * q] = t.x;
          bw[4 * q + 1] = t.y;
          bw[4 * q + 2] = t.z;
          bw[4 * q + 3] = t.w;
        }
      }
    }
    if (r == 0) {
      if (tid < cb_total) cbs[tid] = cbv;
      __syncthreads();  // codebook staged
      const int e = planes_from_lds<BITS, false>(cbs + ((p.cb_rows == 1) ? 0 : col * E), cb, cb);
      colscale = ldexpf(p.acc_scale, -e);
    }
    // ---- activations to fp16 (their loads went out before the weights')
    uint32_t a8s[KL / 16][8];
#pragma unroll
    for (int h = 0; h < KL / 16; ++h) convert_a16_big<BITS, XT>(ra[h], a8s[h]);
    // ---- decode + MFMA, 8 k per step
#pragma unroll
    for (int h = 0; h < KL / 16; ++h) {
      const uint32_t* a8 = a8s[h];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int s = 2 * h + t;  // step: indices 8s .. 8s+7 of the lane's range
        uint32_t chunk[BITS];
#pragma unroll
        for (int w = 0; w < BITS; ++w) chunk[w] = bw[(s >> 2) * BITS + w];
        const half8 bf = decode_sub<BITS>(chunk, s & 3, cb);
        const u32x4 a4 = {a8[4 * t], a8[4 * t + 1], a8[4 * t + 2], a8[4 * t + 3]};
        acc = mfma16x16x32(__builtin_bit_cast(half8, a4), bf, acc);
      }
    }
  }
  if (rounds == 0) __syncthreads();
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    floatx4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[w][lane];
    if (n0 + col < p.N) {
      const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n0 + col) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = 4 * g + i;
        if (m < p.M) store_from_float(p.y, p.y_dt, m * p.ldy + n0 + col, epi1(p.epi, m * p.ldy + n0 + col, t[i] * colscale + b));
      }
    }
  }
}

// Split-K decode GEMV for 4 < M <= 16 (cfg5 M = 16), same tiling as
// gemv_cb_kernel: work-group = 16 waves on 16 output columns, wave w takes
// the 128-wide k steps w, w + 16, ... and lane group g the 32 k at 32g of a
// step (32 activations of row m = col: 64 bytes, against 4*BITS bytes of
// weights, so the 16 rows' activations are most of what a lane loads).  A
// round holds NS steps per wave in registers and issues every load of the
// round before any wait: the codebook value (first round), the activations,
// then the packed weights, so the codebook planes and the activation
// conversion wait only for the small loads issued ahead of the weights.
template <int BITS, int XT>
__global__ __launch_bounds__(1024) void gemv_split_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int WAVES = 16;
  constexpr int NS = 2;  // k steps per wave and round: a round covers 16 waves x 2 x 128 = 4096 k
  constexpr int E = 1 << BITS;
  __shared__ floatx4 red[WAVES][64];
  __shared__ float cbs[16 * E];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t n = n0 + col < p.N ? n0 + col : p.N - 1;
  const int rounds = static_cast<int>(p.K / (kKM * WAVES * NS));

  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const bool arow = col < p.M;
  CodebookRegs<BITS> cb;
  float colscale = 1.0f;
  const int cb_total = ((p.cb_rows == 1) ? 1 : 16) * E;
  float cbv = 0.0f;
  if (tid < cb_total) {
    const int rr = tid / E, j = tid - (tid / E) * E;
    const int64_t row = (p.cb_rows == 1) ? 0 : n0 + rr;
    if (j < p.cb_size && (p.cb_rows == 1 || row < p.N)) cbv = load_as_float(p.cb, p.cb_dt, row * p.cb_size + j);
  }
  for (int r = 0; r < rounds; ++r) {
    RawA<XT> ra[NS][2];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int64_t k0 = ((int64_t)(r * NS + j) * WAVES + wave) * kKM + 32 * g;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (arow) {
          issue_a16<XT>(p.x, (int64_t)col * p.ldx + k0 + 16 * h, ra[j][h]);
        } else {
#pragma unroll
          for (int w = 0; w < RawA<XT>::kWords; ++w) ra[j][h].w[w] = 0u;
        }
      }
    }
    uint32_t bw[NS][BITS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int64_t k0 = ((int64_t)(r * NS + j) * WAVES + wave) * kKM + 32 * g;
      const uint8_t* src = p.w + (((n * p.K + k0) * BITS) >> 3);  // 32 indices: 4*BITS bytes
      if constexpr (BITS == 2) {
        const uint2 t = *reinterpret_cast<const uint2*>(src);
        bw[j][0] = t.x;
        bw[j][1] = t.y;
      } else if constexpr (BITS == 4) {
        const uint4 t = *reinterpret_cast<const uint4*>(src);
        bw[j][0] = t.x;
        bw[j][1] = t.y;
        bw[j][2] = t.z;
        bw[j][3] = t.w;
      } else {
#pragma unroll
        for (int w = 0; w < 3; ++w) bw[j][w] = reinterpret_cast<const uint32_t*>(src)[w];
      }
    }
    if (r == 0) {
      if (tid < cb_total) cbs[tid] = cbv;
      __syncthreads();  // codebook staged
      const int e = planes_from_lds<BITS, false>(cbs + ((p.cb_rows == 1) ? 0 : col * E), cb, cb);
      colscale = ldexpf(p.acc_scale, -e);
    }
    uint32_t a[NS][16];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      convert_a16_big<BITS, XT>(ra[j][0], &a[j][0]);
      convert_a16_big<BITS, XT>(ra[j][1], &a[j][8]);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4 a4 = {a[j][4 * st], a[j][4 * st + 1], a[j][4 * st + 2], a[j][4 * st + 3]};
        const half8 bf = decode_sub<BITS>(bw[j], st, cb);
        acc = mfma16x16x32(__builtin_bit_cast(half8, a4), bf, acc);
      }
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    floatx4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[w][lane];
    if (n0 + col < p.N) {
      const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n0 + col) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = 4 * g + i;
        if (m < p.M) store_from_float(p.y, p.y_dt, m * p.ldy + n0 + col, epi1(p.epi, m * p.ldy + n0 + col, t[i] * colscale + b));
      }
    }
  }
}

}  // namespace

// Shapes the split-K kernel runs: 4 < M <= 16 (measured: at M = 16 it and the
// gemv_fast_kernel trade places by activation volume), K a multiple of 4096,
// 16-byte aligned rows/streams.
inline bool gemv_split_supported(const GemmArgs& p, int bits) {
  return p.M >= 1 && p.M <= 16 && !p.conv && (bits == 2 || bits == 3 || bits == 4) && p.K % 4096 == 0 &&
         p.fast_b && p.vec_a;
}

template <int BITS>
int launch_gemv_split(const GemmArgs& p, int xt, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.N + 15) / 16));
  switch (xt) {
    case DIMQ_F32: hipLaunchKernelGGL((gemv_split_kernel<BITS, DIMQ_F32>), grid, dim3(1024), 0, s, p); break;
    case DIMQ_F16: hipLaunchKernelGGL((gemv_split_kernel<BITS, DIMQ_F16>), grid, dim3(1024), 0, s, p); break;
    default: hipLaunchKernelGGL((gemv_split_kernel<BITS, DIMQ_BF16>), grid, dim3(1024), 0, s, p); break;
  }
  return check_launch("linear_codebook (split-K gemv)");
}

// Shapes it runs: M <= 4 (measured: at M = 16 the split-K kernel is faster,
// the activation conversion of 16 rows per lane costing more than the
// up-front loads save), K a multiple of 4096, 16-byte aligned rows/streams.
inline bool gemv_fast_supported(const GemmArgs& p, int bits) {
  return p.M >= 1 && p.M <= 4 && !p.conv && (bits == 2 || bits == 3 || bits == 4) && p.K % 4096 == 0 &&
         p.fast_b && p.vec_a;
}

template <int BITS>
int launch_gemv_fast(const GemmArgs& p, int xt, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.N + 15) / 16));
  switch (xt) {
    case DIMQ_F32: hipLaunchKernelGGL((gemv_fast_kernel<BITS, DIMQ_F32>), grid, dim3(1024), 0, s, p); break;
    case DIMQ_F16: hipLaunchKernelGGL((gemv_fast_kernel<BITS, DIMQ_F16>), grid, dim3(1024), 0, s, p); break;
    default: hipLaunchKernelGGL((gemv_fast_kernel<BITS, DIMQ_BF16>), grid, dim3(1024), 0, s, p); break;
  }
  return check_launch("linear_codebook (gemv)");
}

}  // namespace dimq
