// Decode-shape codebook GEMV (M <= 16): y[M,N] = x[M,K] W_hat^T + b, the
// HBM-bound case of BASELINE cfg5 (W 4096x4096 3-bit: 6.3 MB of indices).
//
// Work-group = 4 waves on 16 x NCB output columns and a k range of K / KS.
// The work-group first stages its activation rows x[0:M, k range] once in LDS
// as fp16, in the slot order of the weight decoder (rows >= M read a zero
// row), then each lane streams one contiguous run of R packed indices of its
// column (R / 32 chunks of 32 indices): every load of the run is issued
// before the first is used, and the run is consumed 8 indices at a time in
// issue order, so the decode of the first chunks runs while the rest of the
// stream is still arriving.  One v_mfma_f32_16x16x32_f16 per 8 indices and
// lane group: A = 8 activations of row m = lane % 16 from LDS, B = the 8
// decoded weights of column lane % 16.
//   NCB = 1: the 4 waves take the four quarters of the work-group's k range
//            and their partial sums are reduced through LDS (M <= 4, or no
//            workspace for the split-K form).
//   NCB = 4: each wave takes one 16-column block over the whole k range, so
//            a staged activation is read by 64 columns instead of 16 (for
//            4 < M <= 16 the activations outweigh the 3-bit weights 5:1 per
//            16 columns).  With KS > 1 the work-groups of one column block
//            write fp32 partial sums into the caller's workspace and
//            gemv_reduce_kernel adds them (bias and epilogue there).
#pragma once

#include "gemm_big.h"

namespace dimq {
namespace {

constexpr int kGemvThreads = 256;

constexpr int kGemvRun = 256;  // indices per lane run (8 chunks of 32)

// Position of activation k (work-group-local) in a staged row: runs of
// kGemvRun padded by 8 halves, so the four lane groups' runs start 16 bytes
// apart in the LDS banks.
__device__ __forceinline__ int gemv_pos(int k) { return (k / kGemvRun) * (kGemvRun + 8) + k % kGemvRun; }

template <int BITS, int XT, int NCB>
__global__ __launch_bounds__(kGemvThreads) void gemv_stream_kernel(const GemmArgs p, int KS, float* __restrict__ partial) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int E = 1 << BITS;
  constexpr int R = kGemvRun;
  constexpr int NW = R / 32 * BITS;  // packed words of a run
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ floatx4 red[NCB == 1 ? 4 : 1][64];
  __shared__ uint32_t wbig[4];  // range guard: a wave staged an activation >= 2^-7

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  constexpr int krange = (NCB == 1 ? 16 : 4) * kGemvRun;  // k range of the work-group (K = KS * krange)
  const int64_t kw0 = (int64_t)blockIdx.y * krange;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * NCB + (NCB == 1 ? 0 : 16 * wave);
  const int64_t n = n0 + col < p.N ? n0 + col : p.N - 1;
  const int run = (NCB == 1 ? 4 * wave : 0) + g;   // this lane's run within the work-group's range
  constexpr int pitch = (krange / R) * (R + 8) + 8;  // fp16 row pitch of the staged activations
  const int rows = p.M < 16 ? (int)p.M : 16;
  constexpr int gpr = krange / 16;                   // 16-element groups per row
  const int groups = rows * gpr;

  uint32_t trk = 0;  // range guard (common.h)
  // codebook row of the lane's column (issued first: its wait does not wait for the streams)
  float cbv[E];
  load_cb_row<E>(p.cb, p.cb_dt, p.cb_rows == 1 ? 0 : n, p.cb_size, cbv);
  // groups past the staged rows issue no load (at M = 1 seven of the eight
  // would re-read group 0 and hold up the address path ahead of the weights)
  auto issue_x = [&](int base, RawA<XT> (&ra)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int gi = base + u * kGemvThreads + tid;
      if (gi >= groups) break;
      const int m = gi / gpr;
      issue_a16<XT>(p.x, (int64_t)m * p.ldx + kw0 + (int64_t)(gi - m * gpr) * 16, ra[u]);
    }
  };
  auto commit_x = [&](int base, const RawA<XT> (&ra)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int gi = base + u * kGemvThreads + tid;
      if (gi >= groups) continue;
      const int m = gi / gpr;
      uint32_t o[8];
      convert_a16_big<BITS, XT>(ra[u], o);
      if constexpr (range_guarded<XT>()) trk = range_track(trk, o);
      uint4* dst = reinterpret_cast<uint4*>(xs + m * pitch + gemv_pos((gi - m * gpr) * 16));
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };
  // activations of the first batch, then the whole weight run: loads retire
  // in order, so the activation conversion waits only for the activations
  RawA<XT> ra[8];
  issue_x(0, ra);
  __builtin_amdgcn_sched_barrier(0);  // keep every activation load ahead of the weight run
  uint32_t bw[NW];
  {
    const uint4* src = reinterpret_cast<const uint4*>(p.w + (((n * p.K + kw0 + (int64_t)run * R) * BITS) >> 3));
#pragma unroll
    for (int q = 0; q < NW / 4; ++q) {
      const uint4 t = src[q];
      bw[4 * q] = t.x; bw[4 * q + 1] = t.y; bw[4 * q + 2] = t.z; bw[4 * q + 3] = t.w;
    }
  }
  commit_x(0, ra);
  for (int base = 8 * kGemvThreads; base < groups; base += 8 * kGemvThreads) {  // M = 16 over 4096 k only
    issue_x(base, ra);
    commit_x(base, ra);
  }
  for (int i = tid; i < pitch / 8; i += kGemvThreads)  // row `rows`: zeros for the MFMA rows m >= M
    *reinterpret_cast<uint4*>(xs + rows * pitch + 8 * i) = make_uint4(0, 0, 0, 0);
  CodebookRegs<BITS> cb;
  const int e = planes_from_lds<BITS, false>(cbv, cb, cb);
  const float colscale = ldexpf(p.acc_scale, -e);
  constexpr bool kGuard = range_guarded<XT>();
  if constexpr (kGuard) {
    const bool any = wave_any((trk & kRangeBigBits) != 0u);
    if (lane == 0) wbig[wave] = any;
  }
  lds_barrier();  // the weight runs stay in flight

  // the run, 8 indices per MFMA, consumed in issue order
  const uint16_t* arow = xs + (col < rows ? col : rows) * pitch + run * (R + 8);
  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < R / 32; ++c) {
    uint32_t chunk[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) chunk[w] = bw[c * BITS + w];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const half8 bf = decode_sub<BITS>(chunk, sub, cb);
      const half8 af = *reinterpret_cast<const half8*>(arow + 32 * c + 8 * sub);
      acc = mfma16x16x32(af, bf, acc);
    }
  }

  // range guard, per wave (its outputs: NCB = 4 its 16 columns; NCB = 1 the
  // partial sums of its k quarter): recomputed in fp32 when the work-group
  // staged no activation >= 2^-7 or an accumulator of the wave is not finite
  bool exact = false;
  if constexpr (kGuard) {
    exact = !(wbig[0] | wbig[1] | wbig[2] | wbig[3]) || wave_any(!finite_acc<4>(&acc, 1, 1));
    if (exact && NCB == 4) {
      const int64_t c0 = n0, c1 = n0 + 16;
      if (KS > 1) {
        exact_tile(p, XT, BITS, 0, 16, c0, c1, kw0, kw0 + krange, 0, false, lane, 64,
                   [&](int64_t m, int64_t nn, float v) {
                     partial[(static_cast<int64_t>(blockIdx.y) * p.M + m) * p.N + nn] = v * p.acc_scale;
                   });
      } else {
        exact_tile_out(p, XT, BITS, 0, 16, c0, c1, 0, false, lane, 64);
      }
      return;
    }
  }

  // acc[i] = partial y[4g + i][n0 + col]
  if constexpr (NCB == 1) {
    if (exact) {  // this wave's k quarter in fp32, in the accumulator layout, times 2^e (colscale follows)
      const int64_t kq = kw0 + static_cast<int64_t>(4 * wave) * R;
      exact_tile(p, XT, BITS, 0, 16, n0, n0 + 16, kq, kq + 4 * R, 0, false, lane, 64,
                 [&](int64_t m, int64_t nn, float v) { red[wave][(m >> 2) * 16 + (nn - n0)][m & 3] = ldexpf(v, e); });
    } else {
      red[wave][lane] = acc;
    }
    __syncthreads();
    if (wave != 0) return;
    acc = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
  }
  if (n0 + col >= p.N) return;
  if (KS > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = 4 * g + i;
      if (m < p.M) partial[((int64_t)blockIdx.y * p.M + m) * p.N + n0 + col] = acc[i] * colscale;
    }
    return;
  }
  const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n0 + col) : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = 4 * g + i;
    if (m < p.M) {
      const int64_t off = m * p.ldy + n0 + col;
      store_from_float(p.y, p.y_dt, off, epi1(p.epi, off, acc[i] * colscale + b));
    }
  }
}

// y[m, n] = epilogue(sum over the KS partial sums + bias).
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const GemmArgs p, int KS, const float* __restrict__ partial) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.M * p.N) return;
  const int64_t m = i / p.N, n = i - m * p.N;
  float v = p.bias ? load_as_float(p.bias, p.bias_dt, n) : 0.0f;
  for (int k = 0; k < KS; ++k) v += partial[(int64_t)k * p.M * p.N + i];
  const int64_t off = m * p.ldy + n;
  store_from_float(p.y, p.y_dt, off, epi1(p.epi, off, v));
}

// Split of a GEMV call: column blocks per work-group (NCB) and k splits (KS);
// every lane streams one run of kGemvRun indices.  False when the shape does
// not fit the kernel (other M <= 16 shapes take gemv_cb_kernel).
struct GemvPlan {
  int ncb, ks;
  size_t lds;
};

inline bool gemv_plan(const GemmArgs& p, int bits, bool have_ws, GemvPlan& pl) {
  if (!(p.M >= 1 && p.M <= 16) || p.conv || !(bits == 2 || bits == 3 || bits == 4) || !p.fast_b || !p.vec_a)
    return false;
  constexpr int64_t kWg1 = 16 * kGemvRun;  // k range of an NCB = 1 work-group (4 waves x 4 runs)
  constexpr int64_t kWg4 = 4 * kGemvRun;   // k range of an NCB = 4 work-group (4 runs)
  if (p.M > 4 && have_ws && p.N % 64 == 0 && p.K % kWg4 == 0) {
    pl.ncb = 4;
    pl.ks = (int)(p.K / kWg4);
  } else if (p.K == kWg1 || (have_ws && p.K % kWg1 == 0)) {
    pl.ncb = 1;
    pl.ks = (int)(p.K / kWg1);
  } else {
    return false;
  }
  const int rows = p.M < 16 ? (int)p.M : 16;
  const int64_t krange = p.K / pl.ks;
  pl.lds = (size_t)(rows + 1) * ((krange / kGemvRun) * (kGemvRun + 8) + 8) * sizeof(uint16_t);
  return pl.lds <= 150 * 1024;
}

inline int64_t gemv_partial_bytes(const GemmArgs& p, const GemvPlan& pl) {
  return pl.ks > 1 ? (int64_t)pl.ks * p.M * p.N * 4 : 0;
}

template <int BITS, int XT, int NCB>
int launch_gemv_stream_k(const GemmArgs& p, const GemvPlan& pl, float* partial, hipStream_t s) {
  auto k = gemv_stream_kernel<BITS, XT, NCB>;
  if (pl.lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds);
    if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "linear_codebook (gemv): %s", hipGetErrorString(e));
  }
  const dim3 grid(static_cast<unsigned>((p.N + 16 * NCB - 1) / (16 * NCB)), static_cast<unsigned>(pl.ks));
  hipLaunchKernelGGL(k, grid, dim3(kGemvThreads), pl.lds, s, p, pl.ks, partial);
  return check_launch("linear_codebook (gemv)");
}

}  // namespace

// Runs a planned GEMV; `partial` holds gemv_partial_bytes when pl.ks > 1.
template <int BITS>
int launch_gemv_stream(const GemmArgs& p, int xt, const GemvPlan& pl, float* partial, hipStream_t s) {
  int rc;
#define DIMQ_GEMV_XT(XT)                                                                               \
  rc = pl.ncb == 1 ? launch_gemv_stream_k<BITS, XT, 1>(p, pl, partial, s)                             \
                   : launch_gemv_stream_k<BITS, XT, 4>(p, pl, partial, s);
  switch (xt) {
    case DIMQ_F32: DIMQ_GEMV_XT(DIMQ_F32) break;
    case DIMQ_F16: DIMQ_GEMV_XT(DIMQ_F16) break;
    default: DIMQ_GEMV_XT(DIMQ_BF16) break;
  }
#undef DIMQ_GEMV_XT
  if (rc != DIMQ_OK || pl.ks == 1) return rc;
  const int64_t total = p.M * p.N;
  hipLaunchKernelGGL(gemv_reduce_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s, p, pl.ks,
                     partial);
  return check_launch("linear_codebook (gemv reduce)");
}

}  // namespace dimq
