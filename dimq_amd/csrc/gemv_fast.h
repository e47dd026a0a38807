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
// bf16 activations with 4 < M <= 16 take gemv_direct_kernel (below) instead.
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
  // codebook row of the lane's column, converted before the activation and
  // weight loads are issued (measured against converting it after them, same
  // process, cfg5: 5.90 against 5.96 us at M = 1, 7.06 against 7.20 at M = 4)
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

// ---- bf16 activations, 4 < M <= 16: direct A operand, bf16 hi + lo weights --
//
// For bf16 activations the MFMA can take x as it is (v_mfma_f32_16x16x32_bf16),
// with each weight split into two bf16 parts, hi = bf16(c) and lo = bf16(c -
// hi), whose sum carries 16 significant bits (two MFMAs per 8 indices).  The
// activations then need no conversion, no LDS staging and no range guard
// (bf16 has fp32's exponent range), so a work-group can own 16 columns over
// the whole k range without the 128 KB of staged fp16 rows per work-group
// that M = 16 costs the staged kernel, and the split-k partial sums and their
// second launch go away: each lane loads its A fragments (8 consecutive x of
// row lane % 16) straight from global memory, two 32-index chunks ahead.
// Work-group = 4 waves on 16 columns; wave w takes the k quarter w, lane
// (col, g) the run of R = K / 16 indices 4w + g of its column; the four waves'
// 16 x 16 partial tiles are added through LDS.  Measured at cfg5 M = 16 (X
// bf16 [16, 4096], 3-bit): 9.4 against 10.1 us for the staged split-k kernel
// and its reduction; at M <= 4 the staged kernel stays faster (5.9 against
// 6.5 us at M = 1), whose rows past M cost nothing.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// 8-index field word of sub-step s of a 32-index chunk (slot order of decode_sub).
template <int BITS>
__device__ __forceinline__ uint32_t chunk_word(const uint32_t (&c)[BITS], int s) {
  if constexpr (BITS == 4) {
    return c[s];
  } else if constexpr (BITS == 2) {
    return c[s >> 1] >> (4 * (s & 1));
  } else {
    if (s == 0) return c[0];
    if (s == 1) return __builtin_amdgcn_alignbit(c[1], c[0], 24);
    if (s == 2) return __builtin_amdgcn_alignbit(c[2], c[1], 16);
    return c[2] >> 8;
  }
}

// Eight indices -> their hi and lo bf16 weights (slot order), one selector pass for both.
template <int BITS>
__device__ __forceinline__ void decode_hilo(uint32_t G, const CodebookRegs<BITS>& ch, const CodebookRegs<BITS>& cl,
                                            bf16x8& wh, bf16x8& wl) {
  uint32_t D0, D1;
  if constexpr (BITS == 4) {
    D0 = G & 0x0f0f0f0fu;
    D1 = (G >> 4) & 0x0f0f0f0fu;
  } else if constexpr (BITS == 2) {
    D0 = G & 0x03030303u;
    D1 = (G >> 2) & 0x03030303u;
  } else {
    D0 = spread3x4(G & 0xfffu);
    D1 = spread3x4((G >> 12) & 0xfffu);
  }
  uint32_t h[4], l[4];
  lookup4<BITS>(ch, D0, h[0], h[1]);
  lookup4<BITS>(ch, D1, h[2], h[3]);
  lookup4<BITS>(cl, D0, l[0], l[1]);
  lookup4<BITS>(cl, D1, l[2], l[3]);
  const u32x4 hv = {h[0], h[1], h[2], h[3]}, lv = {l[0], l[1], l[2], l[3]};
  wh = __builtin_bit_cast(bf16x8, hv);
  wl = __builtin_bit_cast(bf16x8, lv);
}

// A fragment of sub-step s of a 32-index chunk in the weight decoder's slot
// order (kperm16), from the chunk's 32 activations in natural order (x[4]
// holds k 8j .. 8j + 7 in x[j]): 3-bit slots are natural; 4-bit slots hold the
// even k of a group of 8, then the odd k; 2-bit sub-steps 2h, 2h + 1 take k
// {0,4,8,12,1,5,9,13} and {2,6,10,14,3,7,11,15} of the chunk's 16-group h.
template <int BITS>
__device__ __forceinline__ uint4 a_slots(const uint4 (&x)[4], int s) {
  constexpr uint32_t LO = 0x05040100u, HI = 0x07060302u;  // low / high halves of two dwords
  if constexpr (BITS == 3) {
    return x[s];
  } else if constexpr (BITS == 4) {
    const uint4 v = x[s];
    return make_uint4(perm(v.y, v.x, LO), perm(v.w, v.z, LO), perm(v.y, v.x, HI), perm(v.w, v.z, HI));
  } else {
    const uint4 a = x[2 * (s >> 1)], b = x[2 * (s >> 1) + 1];  // dwords d0..d3, d4..d7 of the 16-group
    if ((s & 1) == 0)
      return make_uint4(perm(a.z, a.x, LO), perm(b.z, b.x, LO), perm(a.z, a.x, HI), perm(b.z, b.x, HI));
    return make_uint4(perm(a.w, a.y, LO), perm(b.w, b.y, LO), perm(a.w, a.y, HI), perm(b.w, b.y, HI));
  }
}

template <int BITS, int R>
__global__ __launch_bounds__(256) void gemv_direct_kernel(const GemmArgs p) {
  constexpr int E = 1 << BITS;
  constexpr int NW = R / 32 * BITS;  // packed words of a run
  constexpr int CH = R / 32;         // 32-index chunks of a run
  __shared__ floatx4 red[4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t n = n0 + col < p.N ? n0 + col : p.N - 1;
  const int64_t k0 = (int64_t)(4 * wave + g) * R;
  // the codebook row's raw loads first, converted once the weight run and the
  // first chunk's activations are requested too (cfg5 M = 16, same process:
  // 8.93 -> 8.53 us against converting it before them)
  CbRaw<E> cbraw;
  cb_row_issue<E>(p.cb, p.cb_dt, p.cb_rows == 1 ? 0 : n, p.cb_size, cbraw);
  uint32_t bw[NW];
  if constexpr (NW % 4 == 0) {
    const uint4* src = reinterpret_cast<const uint4*>(p.w + (((n * p.K + k0) * BITS) >> 3));
#pragma unroll
    for (int q = 0; q < NW / 4; ++q) {
      const uint4 t = src[q];
      bw[4 * q] = t.x; bw[4 * q + 1] = t.y; bw[4 * q + 2] = t.z; bw[4 * q + 3] = t.w;
    }
  } else {
    // 3-bit runs of 64 indices: 24 bytes, 8-byte aligned
    static_assert(NW % 2 == 0, "a run is a whole number of 8-byte pieces");
    const uint2* src = reinterpret_cast<const uint2*>(p.w + (((n * p.K + k0) * BITS) >> 3));
#pragma unroll
    for (int q = 0; q < NW / 2; ++q) {
      const uint2 t = src[q];
      bw[2 * q] = t.x; bw[2 * q + 1] = t.y;
    }
  }
  const bool live = col < p.M;  // A row col; rows >= M are zero (and load row 0)
  const uint4* xa =
      reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.x) + (live ? col : 0) * p.ldx + k0);
  // Activation chunks held: the chunk computed and the next two in flight
  // (cfg5 M = 16, same process: 8.51 us one ahead, 8.35 two, 8.42 three,
  // 8.69 four; a chunk's ~550 cycles of decode and MFMAs are shorter than its
  // activations' load latency).
  constexpr int XD = 3;
  uint4 xr[XD][4];
  // the first chunks' activations, before the codebook's wait
#pragma unroll
  for (int j = 0; j < XD - 1 && j < CH; ++j)
#pragma unroll
    for (int s = 0; s < 4; ++s) xr[j][s] = xa[4 * j + s];
  float cbv[E];
  cb_row_finish<E>(cbraw, p.cb_dt, p.cb_size, cbv);
  CodebookRegs<BITS> ch, cl;
  {
    uint32_t hb[E], lb[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
      hb[j] = float_to_bf16_bits(cbv[j]);
      lb[j] = float_to_bf16_bits(cbv[j] - bf16_bits_to_float(hb[j]));
    }
    set_planes<BITS>(ch, hb);
    set_planes<BITS>(cl, lb);
  }
  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f}, acc2 = acc;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (c + XD - 1 < CH) {
#pragma unroll
      for (int s = 0; s < 4; ++s) xr[(c + XD - 1) % XD][s] = xa[4 * (c + XD - 1) + s];
    }
    uint32_t chunk[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) chunk[w] = bw[c * BITS + w];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 wh, wl;
      decode_hilo<BITS>(chunk_word<BITS>(chunk, s), ch, cl, wh, wl);
      const uint4 xv = live ? a_slots<BITS>(xr[c % XD], s) : make_uint4(0, 0, 0, 0);
      const bf16x8 a = __builtin_bit_cast(bf16x8, xv);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, wh, acc, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, wl, acc2, 0, 0, 0);
    }
  }
  red[wave][lane] = acc + acc2;
  __syncthreads();
  if (wave != 0) return;
  acc = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];  // acc[i] = y[4g + i][n0 + col]
  if (n0 + col >= p.N) return;
  const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n0 + col) : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = 4 * g + i;
    if (m < p.M) {
      const int64_t off = m * p.ldy + n0 + col;
      store_from_float(p.y, p.y_dt, off, epi1(p.epi, off, acc[i] * p.acc_scale + b));
    }
  }
}

// The direct kernel's shapes: bf16 x, 4 < M <= 16, K = 16 R with R in {64, 128, 256}.
inline bool gemv_direct_ok(const GemmArgs& p, int bits, int xt) {
  return xt == DIMQ_BF16 && p.M > 4 && p.M <= 16 && !p.conv && (bits == 2 || bits == 3 || bits == 4) && p.fast_b &&
         p.vec_a && (p.K == 1024 || p.K == 2048 || p.K == 4096);
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

template <int BITS>
int launch_gemv_direct(const GemmArgs& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.N + 15) / 16));
  switch (p.K) {
    case 1024: hipLaunchKernelGGL((gemv_direct_kernel<BITS, 64>), grid, dim3(256), 0, s, p); break;
    case 2048: hipLaunchKernelGGL((gemv_direct_kernel<BITS, 128>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((gemv_direct_kernel<BITS, 256>), grid, dim3(256), 0, s, p); break;
  }
  return check_launch("linear_codebook (gemv, bf16)");
}

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
