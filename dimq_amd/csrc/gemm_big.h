// Large-tile codebook GEMM for the MFMA-bound Linear shapes (ViT-B/16
// qkv/proj/fc1/fc2 at M = 12,608, BASELINE cfg1): y[M,N] = x[M,K] W_hat^T + b.
//
// Work-group = WGM x WGN waves; wave (wm, wn) owns a (MBLK*32) x (NBLK*32)
// block of the (WGM*MBLK*32) x (WGN*NBLK*32) tile.  With WGM = 1 every weight
// column is decoded by exactly one wave.  The MFMA
// is v_mfma_f32_32x32x16_f16 with the *weights* as the A operand (rows =
// output columns n) and the activations as the B operand (columns = rows m),
// so each lane's accumulator holds 4 consecutive n of one m: 16-byte stores
// into row-major y.
//
// Per 64-wide k stage:
//   * activations: raw 16-byte global loads issued one stage ahead into
//     registers, converted to fp16 in the k-slot order of the weight decoder
//     (fp16: byte selects; bf16 and fp32: round to nearest, under the
//     range guard of common.h) and written to a
//     double-buffered LDS tile (row pitch 72 halves: the 16-byte reads of 16
//     consecutive rows hit distinct bank groups);
//   * weights: each lane loads its row's 64 packed indices (8*BITS bytes,
//     one stage ahead) and decodes one 8-index word per k16 step with v_perm
//     lookups into the row's codebook byte planes held in VGPRs; one decoded
//     fragment feeds MBLK MFMAs.
// Codebook rows are scaled by a power of two before rounding to fp16; the
// epilogue multiplies by 2^-e and adds the bias.
#pragma once

#include "gemm_kernel.h"

#include <utility>

namespace dimq {
namespace {

typedef float floatx16g __attribute__((ext_vector_type(16)));

constexpr int kBigKS = 64;           // k per pipeline stage
constexpr int kBigLDA = kBigKS + 8;  // LDS row pitch (halves)

__device__ __forceinline__ floatx16g mfma32(half8 a, half8 b, floatx16g c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>): a loop body
// instantiated per index, for bodies too large for the unroller whose register
// arrays must stay statically indexed.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// 64 indices of row n from column k0 (K % 64 == 0): 8*BITS bytes, 16-byte
// aligned for BITS 2 and 4, 8-byte aligned for BITS 3.
template <int BITS>
__device__ __forceinline__ void issue_b_stage(const uint8_t* w, int64_t n, int64_t K, int64_t k0,
                                              uint32_t (&c)[2 * BITS]) {
  const uint8_t* src = w + (((n * K + k0) * BITS) >> 3);
  if constexpr (BITS == 3) {
    const uint2* s2 = reinterpret_cast<const uint2*>(src);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const uint2 t = s2[q];
      c[2 * q] = t.x;
      c[2 * q + 1] = t.y;
    }
  } else {
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
#pragma unroll
    for (int q = 0; q < BITS / 2; ++q) {
      const uint4 t = s4[q];
      c[4 * q] = t.x;
      c[4 * q + 1] = t.y;
      c[4 * q + 2] = t.z;
      c[4 * q + 3] = t.w;
    }
  }
}

// Field word of k16 step s of the stage for lane group g: sub-step u = 2s + g
// of the stage's two 32-index chunks (slot order of decode_sub).
template <int BITS>
__device__ __forceinline__ uint32_t stage_word(const uint32_t (&c)[2 * BITS], int s, int g) {
  const int t = s & 1;                     // sub-steps 2t + g of chunk s >> 1
  const uint32_t* ch = c + (s >> 1) * BITS;
  if constexpr (BITS == 4) {
    return g ? ch[2 * t + 1] : ch[2 * t];
  } else if constexpr (BITS == 2) {
    return ch[t] >> (4 * g);
  } else {
    if (t == 0) return g ? __builtin_amdgcn_alignbit(ch[1], ch[0], 24) : ch[0];
    return g ? (ch[2] >> 8) : __builtin_amdgcn_alignbit(ch[2], ch[1], 16);
  }
}

// 16 raw activations -> 8 dwords of fp16 pairs in the slot order of BITS
// (fp32, bf16: one round-to-nearest v_cvt_pk_f16_f32 per pair).
template <int BITS, int XT>
__device__ __forceinline__ void convert_a16_big(const RawA<XT>& r, uint32_t out[8]) {
  if constexpr (XT == DIMQ_F32) {
#pragma unroll
    for (int d = 0; d < 8; ++d)
      out[d] = f16x2_rne(__uint_as_float(r.w[kperm16(BITS, 2 * d)]), __uint_as_float(r.w[kperm16(BITS, 2 * d + 1)]));
  } else {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (XT == DIMQ_F16) {
        w[i] = r.w[i];
      } else {
        w[i] = f16x2_rne(__uint_as_float(r.w[i] << 16), __uint_as_float(r.w[i] & 0xffff0000u));
      }
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int a = kperm16(BITS, 2 * d), b = kperm16(BITS, 2 * d + 1);
      if ((a >> 1) == (b >> 1) && (a & 1) == 0 && (b & 1) == 1) {
        out[d] = w[a >> 1];
      } else {
        // low half <- half (a & 1) of word a/2, high half <- half (b & 1) of word b/2
        const uint32_t sel = ((a & 1) ? 0x0302u : 0x0100u) | ((b & 1) ? 0x07060000u : 0x05040000u);
        out[d] = perm(w[b >> 1], w[a >> 1], sel);
      }
    }
  }
}

// CONV: implicit-GEMM convolution on NHWC activations with a tap-major
// weight stream (k = (kh*KW + kw)*C + c, C % 64 == 0): row m is output pixel
// (b, oh, ow), and a 64-wide k stage is 64 consecutive channels of one input
// pixel (one tap), or zeros where the tap falls into the padding.  y is the
// NHWC output, row-major [M, OC].
// Occupancy hint: the 2-bit implicit-GEMM conv with 64x64 wave tiles fits
// three waves per SIMD without spilling (measured faster than two); the other
// instantiations keep the compiler's choice.
constexpr int big_min_waves(int bits, int mblk, int nblk, bool conv) {
  return (conv && bits == 2 && mblk * nblk <= 4) ? 3 : 1;
}

template <int BITS, int XT, int WGM, int WGN, int MBLK, int NBLK, bool CONV = false, int MODE = kEpiNone>
__global__ __launch_bounds__(64 * WGM * WGN, big_min_waves(BITS, MBLK, NBLK, CONV)) void gemm_big_kernel(
    const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int NT = 64 * WGM * WGN;
  constexpr int BM = WGM * MBLK * 32;
  constexpr int BN = WGN * NBLK * 32;
  constexpr int E = 1 << BITS;
  constexpr int A_TASKS = BM * (kBigKS / 16) / NT;  // 16-element groups per thread
  static_assert(A_TASKS * NT == BM * (kBigKS / 16), "tile rows must split evenly over the threads");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kBigLDA];
  __shared__ float cbs[BN * E];
  __shared__ float ebias[BN];  // the tile's bias, staged once (the epilogue's loads would serialise)
  __shared__ float escale[BN];  // the tile's column factors acc_scale 2^-e (parked epilogue)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  const int wm = wave / WGN;
  const int wn = wave - wm * WGN;
  int64_t mt, nt;
  tile_coords((p.N + BN - 1) / BN, mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t n0 = nt * BN;

  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, n0, BN, p.N, cbs, tid, NT);
  for (int c = tid; c < BN; c += NT) ebias[c] = (p.bias && n0 + c < p.N) ? load_as_float(p.bias, p.bias_dt, n0 + c) : 0.0f;
  __syncthreads();
  CodebookRegs<BITS> cb[NBLK];
  float rscale[NBLK];
  int64_t brow[NBLK];
#pragma unroll
  for (int nb = 0; nb < NBLK; ++nb) {
    // column block nb of wave column wn: tile columns (nb WGN + wn) 32 ..,
    // so that the epilogue's pass nb covers WGN * 32 contiguous columns
    const int nl = (nb * WGN + wn) * 32 + col;
    brow[nb] = n0 + nl < p.N ? n0 + nl : p.N - 1;
    const int rl = (p.cb_rows == 1) ? 0 : nl;
    const int e = planes_from_lds<BITS, false>(cbs + rl * E, cb[nb], cb[nb]);
    rscale[nb] = ldexpf(p.acc_scale, -e);
    if (g == 0) escale[nl] = rscale[nb];
  }

  // activation tasks: (row m, 16-wide group kg) per thread, 4 groups per row
  int64_t aoff[A_TASKS];
  int alds[A_TASKS];
  int aih[A_TASKS], aiw[A_TASKS];  // CONV: input row/column of tap (0, 0)
#pragma unroll
  for (int i = 0; i < A_TASKS; ++i) {
    const int task = tid + NT * i;
    const int m = task >> 2, kg = task & 3;
    alds[i] = m * kBigLDA + 16 * kg;
    if constexpr (CONV) {
      const int64_t mg = m0 + m;
      const int64_t hw = p.cOH * p.cOW;
      aoff[i] = 16 * kg;
      aih[i] = -(1 << 30);  // rows past M read zeros
      aiw[i] = 0;
      if (mg < p.M) {
        const int64_t b = mg / hw;
        const int r = static_cast<int>(mg - b * hw);
        const int oh = r / static_cast<int>(p.cOW);
        const int ow = r - oh * static_cast<int>(p.cOW);
        aoff[i] += b * p.cH * p.cW * p.cC;
        aih[i] = oh * p.csh - p.cph;
        aiw[i] = ow * p.csw - p.cpw;
      }
    } else {
      const int64_t row = (m0 + m < p.M) ? m0 + m : p.M - 1;
      aoff[i] = row * p.ldx + 16 * kg;
    }
  }

  floatx16g acc[MBLK][NBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][nb][i] = 0.0f;

  const int64_t nk = p.K / kBigKS;
  RawA<XT> ra[A_TASKS];
  bool avalid[A_TASKS];  // CONV: the task's tap lies inside the image (else its group reads as zeros)
  uint32_t b0[NBLK][2 * BITS], b1[NBLK][2 * BITS];
  uint32_t trk = 0;

  // CONV taps in the padding still issue their load (pixel (0, 0) of the
  // row's image) and are zeroed at commit: with a branch around the load the
  // compiler cannot count the loads in flight, and its wait for the stage
  // being computed then also waited for part of the next stage's loads,
  // issued just before (a full memory latency per 64-k stage).
  auto issue_a = [&](int64_t kt) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kBigKS;
    if constexpr (CONV) {
      const int tap = static_cast<int>(k / p.cC);
      const int64_t c0 = k - tap * p.cC;
      const int kh = tap / p.cKW;
      const int kw = tap - kh * p.cKW;
#pragma unroll
      for (int i = 0; i < A_TASKS; ++i) {
        const int ih = aih[i] + kh * p.cdh;
        const int iw = aiw[i] + kw * p.cdw;
        avalid[i] = static_cast<unsigned>(ih) < static_cast<unsigned>(p.cH) &&
                    static_cast<unsigned>(iw) < static_cast<unsigned>(p.cW);
        const int64_t pix = avalid[i] ? static_cast<int64_t>(ih) * p.cW + iw : 0;
        issue_a16<XT>(p.x, aoff[i] + pix * p.cC + c0, ra[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_TASKS; ++i) issue_a16<XT>(p.x, aoff[i] + k, ra[i]);
    }
  };
  auto commit_a = [&](int buf, bool track = false) {
#pragma unroll
    for (int i = 0; i < A_TASKS; ++i) {
      uint32_t o[8];
      convert_a16_big<BITS, XT>(ra[i], o);
      if constexpr (CONV) {
        const uint32_t m = avalid[i] ? 0xffffffffu : 0u;
#pragma unroll
        for (int w = 0; w < 8; ++w) o[w] &= m;
      }
      if (range_guarded<XT>() && track) trk = range_track(trk, o);
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][alds[i]]);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };
  auto issue_b = [&](int64_t kt, uint32_t (&dst)[NBLK][2 * BITS]) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kBigKS;
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) issue_b_stage<BITS>(p.w, brow[nb], p.K, k, dst[nb]);
  };
  const uint16_t* arow = nullptr;  // this lane's activation row in a stage tile
  // activation fragments: double-buffered across the four k16 steps (the
  // reads of step s+1 go out under the MFMAs of step s) for small wave tiles;
  // large ones (>= 12 MFMAs per step) read each step's fragments at its start
  // and let the first MFMAs cover the later reads
  constexpr bool XDB = MBLK * NBLK < 12;
  auto compute = [&](int buf, const uint32_t (&bq)[NBLK][2 * BITS]) {
    arow = &As[buf][(wm * MBLK * 32 + col) * kBigLDA + 8 * g];
    half8 xf[XDB ? 2 : 1][MBLK];
    if constexpr (XDB) {
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) xf[0][mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA);
    }
#pragma unroll
    for (int s = 0; s < kBigKS / 16; ++s) {
      const int cur = XDB ? (s & 1) : 0;
      if constexpr (XDB) {
        if (s + 1 < kBigKS / 16) {
#pragma unroll
          for (int mb = 0; mb < MBLK; ++mb)
            xf[(s + 1) & 1][mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA + 16 * (s + 1));
        }
      } else {
#pragma unroll
        for (int mb = 0; mb < MBLK; ++mb)
          xf[0][mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA + 16 * s);
      }
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) {
        const half8 wf = decode_word<BITS>(stage_word<BITS>(bq[nb], s, g), cb[nb]);
#pragma unroll
        for (int mb = 0; mb < MBLK; ++mb) acc[mb][nb] = mfma32(wf, xf[cur][mb], acc[mb][nb]);
      }
    }
    if constexpr (XDB) {
      // order: first reads; then per step its decode, and its MFMAs paired
      // with the next step's reads
      __builtin_amdgcn_sched_group_barrier(0x100, MBLK, 0);
#pragma unroll
      for (int s = 0; s < kBigKS / 16; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x002, 12 * NBLK, 0);
#pragma unroll
        for (int i = 0; i < MBLK * NBLK; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (s + 1 < kBigKS / 16 && i < MBLK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    }
  };

  // Pipeline (two stages per loop trip so the weight register sets alternate
  // without copies): loads for stage kt+1 are in flight while stage kt
  // computes; sched_barriers keep those loads ahead of the MFMAs and the
  // commit, which waits for them, after the MFMAs.
  issue_a(0);
  issue_b(0, b0);
  commit_a(0, true);  // the range guard looks at the first k stage
  __syncthreads();
  int64_t kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    issue_a(kt + 1);
    issue_b(kt + 1, b1);
    __builtin_amdgcn_sched_barrier(0);  // loads go out before the MFMAs, not after
    compute(0, b0);
    __builtin_amdgcn_sched_barrier(0);
    commit_a(1);
    __syncthreads();
    issue_a(kt + 2);
    issue_b(kt + 2, b0);
    __builtin_amdgcn_sched_barrier(0);
    compute(1, b1);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 2 < nk) commit_a(0);
    __syncthreads();
  }
  if (kt < nk) compute(0, b0);

  if constexpr (range_guarded<XT>()) {
    if (tile_needs_exact(p, XT, m0, m0 + BM, trk, finite_acc<1>(&acc[0][0], MBLK, NBLK))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, n0, n0 + BN, 0, CONV);
      return;
    }
  }

  // Parked epilogue where a pass of WGN * 32 columns fits in the activation
  // buffers; otherwise (64 x 128 tiles) stores straight from the accumulators.
  constexpr bool kParked = BM * (WGN * 32 + 4) * 4 <= 2 * BM * kBigLDA * 2;
  if constexpr (kParked) {
    // Epilogue through LDS, in NBLK passes: pass nb parks every wave's column
    // block nb (acc[mb][nb][4j + i] = tile row wm*MBLK*32 + mb*32 + col, tile
    // column (nb WGN + wn) 32 + 8j + 4g + i) as fp32 in the activation
    // buffers, then the work-group stores the pass's WGN * 32 contiguous
    // columns as 8-column chunks: 8 consecutive lanes write a row's whole run
    // (128 bytes of fp16 at WGN 2).  Stored straight from the accumulators,
    // each instruction wrote 32-byte pieces of 32 rows.  One conv timed alone
    // over rotated buffers (ResNet-18 3x3 at bs128, same process), stored
    // non-temporally: layer2 57.8 -> 54.9 us, with the residual 64.2 -> 58.4;
    // layer3 53.2 -> 50.3, 55.1 -> 52.4 (ordinary stores took about half of
    // that).  In the bs128 forward, where the next layer reads the output
    // back, ordinary stores were as fast or faster, so they are kept.
    // 16-bit residuals: pass 0's requested before the first park, pass nb + 1's
    // before pass nb's stores.
    constexpr int PW = WGN * 32;          // columns per pass
    constexpr int OTP = PW + 4;           // fp32 row pitch of the parked pass
    static_assert(BM * OTP * 4 <= 2 * BM * kBigLDA * 2, "a parked pass fits in the activation buffers");
    constexpr int CH = BM * PW / 8;       // 8-column chunks per pass
    constexpr int CPT = (CH + NT - 1) / NT;  // chunks per thread
    static_assert(NT % (PW / 8) == 0, "a thread's chunks share one column group");
    float* ot = reinterpret_cast<float*>(&As[0][0]);
    const bool vec8 = p.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && p.y_dt != DIMQ_F64;
    const int qg = tid % (PW / 8);  // this thread's 8-column group of every pass
    const bool rpair = (MODE & kEpiRes) && res_pairs(p.epi, vec8);
    auto res_load = [&](int nb, ResPairs<8> (&rr)[CPT]) {
#pragma unroll
      for (int u = 0; u < CPT; ++u) {
        const int c = tid + u * NT;
        const int64_t m = m0 + c / (PW / 8);
        const int64_t n = n0 + nb * PW + 8 * qg;
        if (c < CH && m < p.M && n + 8 <= p.N) res_issue<8>(p.epi, m * p.ldy + n, rr[u]);
      }
    };
    ResPairs<8> rr[CPT], rn[CPT];
    if constexpr ((MODE & kEpiRes) != 0) {
      if (rpair) res_load(0, rr);
    }
    __syncthreads();  // every wave is done reading the activation buffers
    static_for<NBLK>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<float4*>(ot + (wm * MBLK * 32 + mb * 32 + col) * OTP + wn * 32 + 8 * j + 4 * g) =
              make_float4(acc[mb][nb][4 * j], acc[mb][nb][4 * j + 1], acc[mb][nb][4 * j + 2], acc[mb][nb][4 * j + 3]);
      __syncthreads();
      if constexpr ((MODE & kEpiRes) != 0) {
        if (rpair && nb + 1 < NBLK) res_load(nb + 1, rn);
      }
      const int nlg = nb * PW + 8 * qg;  // tile column of this thread's chunks
      const float4 s0 = reinterpret_cast<const float4*>(escale)[nlg / 4];
      const float4 s1 = reinterpret_cast<const float4*>(escale)[nlg / 4 + 1];
      const float4 b0 = reinterpret_cast<const float4*>(ebias)[nlg / 4];
      const float4 b1 = reinterpret_cast<const float4*>(ebias)[nlg / 4 + 1];
      float v[CPT][8];
#pragma unroll
      for (int u = 0; u < CPT; ++u) {
        const int r = (tid + u * NT < CH ? tid + u * NT : CH - 1) / (PW / 8);
        const float4* a4 = reinterpret_cast<const float4*>(ot + r * OTP) + 2 * qg;
        const float4 a0 = a4[0], a1 = a4[1];
        v[u][0] = a0.x * s0.x + b0.x; v[u][1] = a0.y * s0.y + b0.y;
        v[u][2] = a0.z * s0.z + b0.z; v[u][3] = a0.w * s0.w + b0.w;
        v[u][4] = a1.x * s1.x + b1.x; v[u][5] = a1.y * s1.y + b1.y;
        v[u][6] = a1.z * s1.z + b1.z; v[u][7] = a1.w * s1.w + b1.w;
      }
      typedef float f4v __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int u = 0; u < CPT; ++u) {
        const int c = tid + u * NT;
        if (CH % NT != 0 && c >= CH) break;
        const int64_t m = m0 + c / (PW / 8);
        const int64_t n = n0 + nlg;
        if (m >= p.M) continue;
        const int64_t off = m * p.ldy + n;
        if (vec8 && n + 8 <= p.N) {
          epi_m<MODE, 8>(p.epi, &rr[u], off, true, v[u]);
          if (p.y_dt == DIMQ_F32) {
            f4v* yp = reinterpret_cast<f4v*>(reinterpret_cast<float*>(p.y) + off);
            const f4v lo = {v[u][0], v[u][1], v[u][2], v[u][3]}, hi = {v[u][4], v[u][5], v[u][6], v[u][7]};
            yp[0] = lo;
            yp[1] = hi;
          } else {
            u32x4 h;
            if (p.y_dt == DIMQ_F16) {
#pragma unroll
              for (int i = 0; i < 4; ++i) h[i] = f16x2_rne(v[u][2 * i], v[u][2 * i + 1]);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) h[i] = bf16x2_rne(v[u][2 * i], v[u][2 * i + 1]);
            }
            u32x4* yp = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.y) + off);
            *yp = h;
          }
        } else {
          for (int i = 0; i < 8; ++i)
            if (n + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[u][i]));
        }
      }
      __syncthreads();  // the next pass overwrites the parked values
      if constexpr ((MODE & kEpiRes) != 0) {
#pragma unroll
        for (int u = 0; u < CPT; ++u) rr[u] = rn[u];
      }
    });
  } else {
    // epilogue: acc[mb][nb][4j + i] = y[m][n], m = block row m0 + wm*MBLK*32 +
    // mb*32 + col, n = n0 + (nb*WGN + wn)*32 + 8j + 4g + i.  For j = 2 jp and
    // 2 jp + 1 the lanes l and l + 32 (g 0 and 1, same row) swap four finished
    // values, so lane g holds the 8 columns 16 jp + 8 g .. + 7 of its row and
    // writes them as one 16-byte store (two 8-byte stores per lane before).
    const bool vec = p.ldy % 4 == 0 && p.y_dt != DIMQ_F64;
    const bool vec8 = p.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && p.y_dt != DIMQ_F64;
    // 16-bit residuals of row group gi = 2 nb + jp, requested one group ahead
    // of its stores (two register sets; a whole-tile prefetch would cost this
    // kernel an occupancy step), so each group's loads land during the
    // previous group's stores: requested right before their own stores, their
    // latency added to every group (ResNet-18 bs128, the residual layers)
    const bool rpair = (MODE & kEpiRes) && res_pairs(p.epi, vec8);
    ResPairs<8> rbuf[2][MBLK];
    auto res_group = [&](int gi, ResPairs<8> (&rr)[MBLK]) {
      const int64_t n8 = n0 + ((gi >> 1) * WGN + wn) * 32 + 16 * (gi & 1) + 8 * g;
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) {
        const int64_t m = m0 + wm * MBLK * 32 + mb * 32 + col;
        if (m < p.M && n8 + 8 <= p.N) res_issue<8>(p.epi, m * p.ldy + n8, rr[mb]);
      }
    };
    if constexpr ((MODE & kEpiRes) != 0) {
      if (rpair) res_group(0, rbuf[0]);
    }
    static_for<NBLK>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        const int gi = 2 * nb + jp;
        if constexpr ((MODE & kEpiRes) != 0) {
          if (rpair && gi + 1 < 2 * NBLK) res_group(gi + 1, rbuf[(gi + 1) & 1]);
        }
        float sc[2][4], bv[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int nl = 8 * (2 * jp + h) + 4 * g;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sc[h][i] = __shfl(rscale[nb], nl + i, 32);
            bv[h][i] = ebias[(nb * WGN + wn) * 32 + nl + i];
          }
        }
        const int64_t n8 = n0 + (nb * WGN + wn) * 32 + 16 * jp + 8 * g;  // this lane's 8 columns
        ResPairs<8>(&rr)[MBLK] = rbuf[gi & 1];
#pragma unroll
        for (int mb = 0; mb < MBLK; ++mb) {
          const int64_t m = m0 + wm * MBLK * 32 + mb * 32 + col;
          float va[4], vb[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            va[i] = acc[mb][nb][4 * (2 * jp) + i] * sc[0][i] + bv[0][i];
            vb[i] = acc[mb][nb][4 * (2 * jp + 1) + i] * sc[1][i] + bv[1][i];
          }
          if (vec8) {
            // g 0 keeps va (columns +0..3) and takes the partner's va (+4..7);
            // g 1 takes the partner's vb (+8..11) and keeps vb (+12..15)
            float v[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float r = __shfl_xor(g ? va[i] : vb[i], 32);
              v[i] = g ? r : va[i];
              v[4 + i] = g ? vb[i] : r;
            }
            if (m >= p.M) continue;
            const int64_t off = m * p.ldy + n8;
            if (n8 + 8 <= p.N) {
              epi_m<MODE, 8>(p.epi, &rr[mb], off, true, v);
              if (p.y_dt == DIMQ_F32) {
                float* yp = reinterpret_cast<float*>(p.y) + off;
                *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
                *reinterpret_cast<float4*>(yp + 4) = make_float4(v[4], v[5], v[6], v[7]);
              } else {
                uint32_t h[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                  h[i] = p.y_dt == DIMQ_F16 ? f16x2_rne(v[2 * i], v[2 * i + 1]) : bf16x2_rne(v[2 * i], v[2 * i + 1]);
                *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.y) + off) = make_uint4(h[0], h[1], h[2], h[3]);
              }
            } else {
              for (int i = 0; i < 8; ++i)
                if (n8 + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[i]));
            }
          } else {
            if (m >= p.M) continue;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float* vv = h ? vb : va;
              const int64_t n = n0 + (nb * WGN + wn) * 32 + 8 * (2 * jp + h) + 4 * g;
              const int64_t off = m * p.ldy + n;
              float v[4] = {vv[0], vv[1], vv[2], vv[3]};
              if (vec && n + 4 <= p.N) {
                epi_m<MODE, 4>(p.epi, nullptr, off, true, v);
                if (p.y_dt == DIMQ_F32) {
                  *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.y) + off) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
                  const uint32_t h0 = p.y_dt == DIMQ_F16 ? f16x2_rne(v[0], v[1]) : bf16x2_rne(v[0], v[1]);
                  const uint32_t h1 = p.y_dt == DIMQ_F16 ? f16x2_rne(v[2], v[3]) : bf16x2_rne(v[2], v[3]);
                  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + off) = make_uint2(h0, h1);
                }
              } else {
                for (int i = 0; i < 4; ++i)
                  if (n + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[i]));
              }
            }
          }
        }
      }
    });
  }
}

// Shared-decode variant: the work-group decodes each 64-wide k stage of its
// BN weight rows once, cooperatively, into LDS as fp16 (row pitch 72 halves,
// the layout the activations use), and every wave reads its weight fragments
// from there.  With per-lane decoding (gemm_big_kernel) every wave row of the
// tile decodes the same columns again; here a weight is decoded once per
// work-group, so the tile can be tall (BM = 256) and the decode and
// activation-conversion work per MFMA drops.  Thread t decodes B_TASKS of the
// 8 words (k16 step s, lane group g) of weight row t / (8 / B_TASKS).
template <int BITS, int XT, int WGM, int WGN, int MBLK, int NBLK, int MODE = kEpiNone, int INTERLEAVE = 0>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_lds_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int NT = 64 * WGM * WGN;
  constexpr int BM = WGM * MBLK * 32;
  constexpr int BN = WGN * NBLK * 32;
  constexpr int E = 1 << BITS;
  constexpr int A_TASKS = BM * (kBigKS / 16) / NT;
  constexpr int B_TASKS = BN * 8 / NT;  // decode words per thread and stage
  static_assert(A_TASKS * NT == BM * (kBigKS / 16), "activation groups split evenly over the threads");
  static_assert(B_TASKS * NT == BN * 8 && 8 % B_TASKS == 0, "weight words split evenly over the threads");
  constexpr int TPR = 8 / B_TASKS;  // threads per weight row
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kBigLDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kBigLDA];
  __shared__ __attribute__((aligned(16))) float escale[BN];  // per tile column: 2^-e
  __shared__ __attribute__((aligned(16))) float ebias[BN];   // and the bias
  // the codebook rows are staged in the second weight buffer, which is first
  // written after the barrier that follows the codebook planes' setup
  static_assert(BN * E * 4 <= BN * kBigLDA * 2, "codebook staging fits in one weight stage buffer");
  float* cbs = reinterpret_cast<float*>(&Bs[1][0]);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  const int wm = wave / WGN;
  const int wn = wave - wm * WGN;
  int64_t mt, nt;
  tile_coords((p.N + BN - 1) / BN, mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t n0 = nt * BN;

  // this thread's weight row and words
  const int brl = tid / TPR;
  const int bw0 = (tid - brl * TPR) * B_TASKS;
  const int64_t brow = n0 + brl < p.N ? n0 + brl : p.N - 1;
  CodebookRegs<BITS> cb;  // set in the prologue, after the first stages' loads are out

  int64_t aoff[A_TASKS];
  int alds[A_TASKS];
#pragma unroll
  for (int i = 0; i < A_TASKS; ++i) {
    const int task = tid + NT * i;
    const int m = task >> 2, kg = task & 3;
    alds[i] = m * kBigLDA + 16 * kg;
    const int64_t row = (m0 + m < p.M) ? m0 + m : p.M - 1;
    aoff[i] = row * p.ldx + 16 * kg;
  }

  floatx16g acc[MBLK][NBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][nb][i] = 0.0f;

  const int64_t nk = p.K / kBigKS;
  RawA<XT> ra0[A_TASKS], ra1[A_TASKS];
  uint32_t bq0[2 * BITS], bq1[2 * BITS];
  uint32_t trk = 0;
  auto issue = [&](int64_t kt, RawA<XT> (&ra)[A_TASKS], uint32_t (&bq)[2 * BITS]) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kBigKS;
#pragma unroll
    for (int i = 0; i < A_TASKS; ++i) issue_a16<XT>(p.x, aoff[i] + k, ra[i]);
    issue_b_stage<BITS>(p.w, brow, p.K, k, bq);
  };
  auto commit = [&](int buf, const RawA<XT> (&ra)[A_TASKS], const uint32_t (&bq)[2 * BITS], bool track = false) {
#pragma unroll
    for (int i = 0; i < A_TASKS; ++i) {
      uint32_t o[8];
      convert_a16_big<BITS, XT>(ra[i], o);
      if (range_guarded<XT>() && track) trk = range_track(trk, o);
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][alds[i]]);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
#pragma unroll
    for (int j = 0; j < B_TASKS; ++j) {
      const int w = bw0 + j;  // word w: k16 step w >> 1, lane group w & 1
      const half8 h = decode_word<BITS>(stage_word<BITS>(bq, w >> 1, w & 1), cb);
      *reinterpret_cast<half8*>(&Bs[buf][brl * kBigLDA + 8 * w]) = h;
    }
  };
  auto compute = [&](int buf) {
    const uint16_t* arow = &As[buf][(wm * MBLK * 32 + col) * kBigLDA + 8 * g];
    const uint16_t* bro = &Bs[buf][(wn * NBLK * 32 + col) * kBigLDA + 8 * g];
#pragma unroll
    for (int s = 0; s < kBigKS / 16; ++s) {
      half8 xf[MBLK], wf[NBLK];
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) xf[mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA + 16 * s);
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) wf[nb] = *reinterpret_cast<const half8*>(bro + nb * 32 * kBigLDA + 16 * s);
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
        for (int mb = 0; mb < MBLK; ++mb) acc[mb][nb] = mfma32(wf[nb], xf[mb], acc[mb][nb]);
    }
  };
  // One stage's MFMAs with the next stage's conversion and decode woven in
  // between them (its loads were issued a full stage earlier), so the matrix
  // cores and the VALU work at the same time within each wave; the weave
  // writes the other LDS buffer, which every wave finished reading before the
  // previous barrier.
  auto step = [&](int buf, bool next, const RawA<XT> (&ra)[A_TASKS], const uint32_t (&bq)[2 * BITS]) {
    compute(buf);
    if (next) commit(buf ^ 1, ra, bq);
    if constexpr (INTERLEAVE) {
      constexpr int NMFMA = MBLK * NBLK * (kBigKS / 16);
#pragma unroll
      for (int i = 0; i < NMFMA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, INTERLEAVE, 0);  // then VALU
      }
    }
  };

  // prologue: stages 0 and 1 loading while the codebook rows are staged (the
  // two latencies overlap), stage 0 committed, stage 2 loading
  issue(0, ra0, bq0);
  issue(1, ra1, bq1);
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, n0, BN, p.N, cbs, tid, NT);
  __syncthreads();
  {
    const int e = planes_from_lds<BITS, false>(cbs + ((p.cb_rows == 1) ? 0 : brl * E), cb, cb);
    if (bw0 == 0) {
      escale[brl] = ldexpf(p.acc_scale, -e);
      ebias[brl] = (p.bias && n0 + brl < p.N) ? load_as_float(p.bias, p.bias_dt, n0 + brl) : 0.0f;
    }
  }
  commit(0, ra0, bq0, true);  // the range guard looks at the first k stage
  __syncthreads();
  issue(2, ra0, bq0);
  int64_t kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    step(0, true, ra1, bq1);  // compute stage kt, commit stage kt+1 (set 1)
    __syncthreads();
    issue(kt + 3, ra1, bq1);
    step(1, kt + 2 < nk, ra0, bq0);  // compute stage kt+1, commit stage kt+2 (set 0)
    __syncthreads();
    issue(kt + 4, ra0, bq0);
  }
  if (kt < nk) compute(0);

  if constexpr (range_guarded<XT>()) {
    if (tile_needs_exact(p, XT, m0, m0 + BM, trk, finite_acc<1>(&acc[0][0], MBLK, NBLK))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, n0, n0 + BN, 0);
      return;
    }
  }

  // Epilogue through LDS, in NBLK passes: pass nb parks every wave's column
  // block nb (acc[mb][nb][4j + i] = tile row wm*MBLK*32 + mb*32 + col, column
  // wn*32 + 8j + 4g + i of the pass) as fp32 in the activation buffers, then
  // the work-group stores the pass as 8-column chunks of rows: 16-byte stores
  // of contiguous rows, residuals loaded before the stores, and one compact
  // loop instead of an unrolled store per accumulator (the unrolled form made
  // the kernel's once-per-tile tail the size of its instruction cache).
  constexpr int PW = WGN * 32;          // columns per pass
  constexpr int OTP = PW + 4;           // fp32 row pitch of the parked pass
  static_assert(BM * OTP * 4 <= 2 * BM * kBigLDA * 2, "a parked pass fits in the activation buffers");
  constexpr int CH = BM * PW / 8;       // 8-column chunks per pass
  constexpr int CPT = (CH + NT - 1) / NT;  // chunks per thread
  float* ot = reinterpret_cast<float*>(&As[0][0]);
  __syncthreads();  // an odd-stage tail may still be reading the activation buffers
  const bool vec8 = p.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && p.y_dt != DIMQ_F64;
  for (int nb = 0; nb < NBLK; ++nb) {
    static_for<NBLK>([&](auto nbc) {
      constexpr int NB = decltype(nbc)::value;
      if (NB != nb) return;
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<float4*>(ot + (wm * MBLK * 32 + mb * 32 + col) * OTP + wn * 32 + 8 * j + 4 * g) =
              make_float4(acc[mb][NB][4 * j], acc[mb][NB][4 * j + 1], acc[mb][NB][4 * j + 2], acc[mb][NB][4 * j + 3]);
    });
    __syncthreads();
    // chunk c: tile row c / (PW/8), pass columns 8*(c % (PW/8)) .. +8, i.e. wave
    // column block q / 4 (wn), its 8-column group q % 4
    ResPairs<8> rr[CPT];
    if ((MODE & kEpiRes) && res_pairs(p.epi, vec8)) {
#pragma unroll
      for (int u = 0; u < CPT; ++u) {
        const int c = tid + u * NT;
        const int r = c / (PW / 8), q = c - r * (PW / 8);
        const int64_t m = m0 + r;
        const int64_t n = n0 + (q >> 2) * NBLK * 32 + nb * 32 + 8 * (q & 3);
        if (c < CH && m < p.M && n + 8 <= p.N) res_issue<8>(p.epi, m * p.ldy + n, rr[u]);
      }
    }
    // A thread's chunks share column group q = tid % (PW / 8) (NT is a
    // multiple of PW / 8): its 8 column factors are read once per pass as
    // aligned 16-byte loads, and every chunk's parked values before any is
    // used, so the LDS latencies overlap; per-chunk branches only guard stores.
    static_assert(NT % (PW / 8) == 0, "a thread's chunks share one column group");
    const int qg = tid % (PW / 8);
    const int nlg = (qg >> 2) * NBLK * 32 + nb * 32 + 8 * (qg & 3);  // a multiple of 8, nlg + 7 < BN
    const float4 s0 = reinterpret_cast<const float4*>(escale)[nlg / 4];
    const float4 s1 = reinterpret_cast<const float4*>(escale)[nlg / 4 + 1];
    const float4 b0 = reinterpret_cast<const float4*>(ebias)[nlg / 4];
    const float4 b1 = reinterpret_cast<const float4*>(ebias)[nlg / 4 + 1];
    float v[CPT][8];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int r = (tid + u * NT < CH ? tid + u * NT : CH - 1) / (PW / 8);
      const float4* a4 = reinterpret_cast<const float4*>(ot + r * OTP) + 2 * qg;
      const float4 a0 = a4[0], a1 = a4[1];
      v[u][0] = a0.x * s0.x + b0.x; v[u][1] = a0.y * s0.y + b0.y;
      v[u][2] = a0.z * s0.z + b0.z; v[u][3] = a0.w * s0.w + b0.w;
      v[u][4] = a1.x * s1.x + b1.x; v[u][5] = a1.y * s1.y + b1.y;
      v[u][6] = a1.z * s1.z + b1.z; v[u][7] = a1.w * s1.w + b1.w;
    }
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * NT;
      if (CH % NT != 0 && c >= CH) break;
      const int r = c / (PW / 8);
      const int64_t m = m0 + r;
      const int64_t n = n0 + (qg >> 2) * NBLK * 32 + nb * 32 + 8 * (qg & 3);
      if (m >= p.M) continue;
      const int64_t off = m * p.ldy + n;
      if (vec8 && n + 8 <= p.N) {
        epi_m<MODE, 8>(p.epi, &rr[u], off, true, v[u]);
        if (p.y_dt == DIMQ_F32) {
          float* yp = reinterpret_cast<float*>(p.y) + off;
          *reinterpret_cast<float4*>(yp) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
          *reinterpret_cast<float4*>(yp + 4) = make_float4(v[u][4], v[u][5], v[u][6], v[u][7]);
        } else {
          uint32_t h[4];
          if (p.y_dt == DIMQ_F16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = f16x2_rne(v[u][2 * i], v[u][2 * i + 1]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = bf16x2_rne(v[u][2 * i], v[u][2 * i + 1]);
          }
          *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.y) + off) = make_uint4(h[0], h[1], h[2], h[3]);
        }
      } else {
        for (int i = 0; i < 8; ++i)
          if (n + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[u][i]));
      }
    }
    __syncthreads();  // the next pass overwrites the parked values
  }
}

typedef __attribute__((address_space(3))) void lds_void_g;

// Row blocks (32 rows each) of the deep-pipeline tile: 64 x 128 tiles.  At the
// cfg1 shape (M 1576, N 3072, K 768, fp32 x) 64-row tiles (624 of them)
// measured 25.9 us against 28.1 us for 128-row tiles (312, two rounds on 256
// CUs, the second a fifth full) and 31.0 us for 192-row tiles (216).
constexpr int kDeepMblk = 2;

// Deep-pipeline variant: 4 waves side by side in n
// (wave tile (MBLK*32) x 32), activations two stages ahead in registers,
// packed weights through a 3-stage LDS ring filled with global_load_lds
// (no registers held by the weight loads).
template <int BITS, int XT, int MBLK, int MODE = kEpiNone>
__global__ __launch_bounds__(256) void gemm_deep_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int BM = MBLK * 32;
  constexpr int BN = 128;
  constexpr int E = 1 << BITS;
  constexpr int A_TASKS = BM * (kBigKS / 16) / 256;
  constexpr int RB = 8 * BITS;                  // packed bytes of one row per stage
  constexpr int BSTAGE = BN * RB;               // bytes of one weight stage
  constexpr int DSZ = BITS == 4 ? 16 : 4;       // global_load_lds size
  constexpr int DPT = BSTAGE / DSZ / 256;       // loads per thread per stage
  static_assert(DPT * DSZ * 256 == BSTAGE, "weight stage splits evenly over the threads");
  constexpr int RING = 3;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kBigLDA];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[RING][BSTAGE];
  __shared__ float cbs[BN * E];
  __shared__ float ebias[BN];  // the tile's bias, staged once (the epilogue's loads would serialise)
  __shared__ float escale[BN];  // the tile's column factors acc_scale * 2^-e (parked epilogue)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  int64_t mt, nt;
  tile_coords((p.N + BN - 1) / BN, mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t n0 = nt * BN;

  const int nl = wave * 32 + col;  // this lane's weight row within the tile
  CodebookRegs<BITS> cb;           // set in the prologue, once the first stages' loads are out
  float rscale = 1.0f;

  int64_t aoff[A_TASKS];
  int alds[A_TASKS];
#pragma unroll
  for (int i = 0; i < A_TASKS; ++i) {
    const int task = tid + 256 * i;
    const int m = task >> 2, kg = task & 3;
    const int64_t row = (m0 + m < p.M) ? m0 + m : p.M - 1;
    aoff[i] = row * p.ldx + 16 * kg;
    alds[i] = m * kBigLDA + 16 * kg;
  }
  // weight loads: chunk c = tid + 256 * d of the stage -> row c / (RB / DSZ)
  const uint8_t* bsrc[DPT];
#pragma unroll
  for (int d = 0; d < DPT; ++d) {
    const int c = tid + 256 * d;
    const int r = c / (RB / DSZ);
    const int64_t n = n0 + r < p.N ? n0 + r : p.N - 1;
    bsrc[d] = p.w + ((n * p.K * BITS) >> 3) + (c - r * (RB / DSZ)) * DSZ;
  }

  floatx16g acc[MBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;

  const int64_t nk = p.K / kBigKS;
  RawA<XT> ra0[A_TASKS], ra1[A_TASKS];
  uint32_t trk = 0;

  auto issue_a = [&](int64_t kt, RawA<XT> (&dst)[A_TASKS]) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kBigKS;
#pragma unroll
    for (int i = 0; i < A_TASKS; ++i) issue_a16<XT>(p.x, aoff[i] + k, dst[i]);
  };
  auto commit_a = [&](int buf, const RawA<XT> (&src)[A_TASKS], bool track = false) {
#pragma unroll
    for (int i = 0; i < A_TASKS; ++i) {
      uint32_t o[8];
      convert_a16_big<BITS, XT>(src[i], o);
      if (range_guarded<XT>() && track) trk = range_track(trk, o);
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][alds[i]]);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };
  auto dma_b = [&](int64_t kt, int slot) {
    const int64_t kb = (((kt < nk ? kt : nk - 1) * kBigKS) * BITS) >> 3;
#pragma unroll
    for (int d = 0; d < DPT; ++d) {
      const void* src = reinterpret_cast<const void*>(bsrc[d] + kb);
      // Inline assembly rather than the builtin: the compiler cannot tell the
      // ring's slots apart, so with the builtin it put s_waitcnt vmcnt(0) in
      // front of every stage's weight reads, waiting for all loads in flight
      // (measured at the cfg1 shape: 32.1 -> 28.4 us).  The wait is the
      // activations' own: stage s's DMA is issued before stage s's activation
      // loads, so the commit's wait for those (vmcnt retires in issue order)
      // covers it, and the barrier after the commit publishes both.
      const uint32_t la =
          static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_g*)(&Bs[slot][(wave * 64 + 256 * d) * DSZ])));
      if constexpr (DSZ == 16)
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(la)) : "memory");
      else
        asm volatile("global_load_lds_dword %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(la)) : "memory");
    }
  };
  // 4-bit: k16 step s pairs 8-k chunk s (lane group 0) with chunk s + 4
  // (lane group 1) instead of chunks 2s and 2s + 1, so a lane's four packed
  // words of the stage are consecutive (one 16-byte LDS read, no per-lane
  // select) and its activation fragments are the 16-byte chunks s + 4g of
  // the row (the MFMA sums the 16 slots of both lane groups, so any pairing
  // of the stage's eight chunks gives the same products).
  constexpr bool kChunkPairs = BITS == 4;
  auto compute = [&](int buf, int slot) {
    uint32_t bq[2 * BITS];
    const uint32_t* brow = reinterpret_cast<const uint32_t*>(&Bs[slot][nl * RB]);
    if constexpr (kChunkPairs) {
      const uint4 q = *reinterpret_cast<const uint4*>(brow + 4 * g);
      bq[0] = q.x; bq[1] = q.y; bq[2] = q.z; bq[3] = q.w;
    } else {
#pragma unroll
      for (int w = 0; w < 2 * BITS; ++w) bq[w] = brow[w];
    }
    constexpr int AS = kChunkPairs ? 8 : 16;  // halves between the fragments of consecutive steps
    const uint16_t* arow = &As[buf][col * kBigLDA + (kChunkPairs ? 32 : 8) * g];
    half8 xf[2][MBLK];
#pragma unroll
    for (int mb = 0; mb < MBLK; ++mb) xf[0][mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA);
#pragma unroll
    for (int s = 0; s < kBigKS / 16; ++s) {
      if (s + 1 < kBigKS / 16) {
#pragma unroll
        for (int mb = 0; mb < MBLK; ++mb)
          xf[(s + 1) & 1][mb] = *reinterpret_cast<const half8*>(arow + mb * 32 * kBigLDA + AS * (s + 1));
      }
      const half8 wf = decode_word<BITS>(kChunkPairs ? bq[s] : stage_word<BITS>(bq, s, g), cb);
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) acc[mb] = mfma32(wf, xf[s & 1][mb], acc[mb]);
    }
  };

  // prologue: weight stages 0..2 and activation stages 0, 1 in flight, then
  // the codebook rows and bias (their latency overlaps the stages')
  dma_b(0, 0);
  dma_b(1, 1);
  dma_b(2, 2);
  issue_a(0, ra0);
  issue_a(1, ra1);
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, n0, BN, p.N, cbs, tid, 256);
  if (tid < BN) ebias[tid] = (p.bias && n0 + tid < p.N) ? load_as_float(p.bias, p.bias_dt, n0 + tid) : 0.0f;
  __syncthreads();
  {
    const int rl = (p.cb_rows == 1) ? 0 : nl;
    const int e = planes_from_lds<BITS, false>(cbs + rl * E, cb, cb);
    rscale = ldexpf(p.acc_scale, -e);
    if (g == 0) escale[nl] = rscale;
  }
  commit_a(0, ra0, true);  // waits for stage 0 (and the weight stages before it); range guard
  issue_a(2, ra0);
  __syncthreads();
  // steady state, two stages per trip (register sets alternate):
  //   compute kt | commit kt+1 (loaded two phases ago) | barrier |
  //   weight stage kt+3 into the freed ring slot, activations of kt+3
  int64_t kt = 0;
  int slot = 0;
  for (; kt + 2 <= nk; kt += 2) {
    compute(0, slot);
    __builtin_amdgcn_sched_barrier(0);
    commit_a(1, ra1);
    __syncthreads();
    dma_b(kt + 3, slot);
    issue_a(kt + 3, ra1);
    __builtin_amdgcn_sched_barrier(0);
    slot = slot == RING - 1 ? 0 : slot + 1;
    compute(1, slot);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 2 < nk) commit_a(0, ra0);
    __syncthreads();
    dma_b(kt + 4, slot);
    issue_a(kt + 4, ra0);
    __builtin_amdgcn_sched_barrier(0);
    slot = slot == RING - 1 ? 0 : slot + 1;
  }
  if (kt < nk) compute(0, slot);

  if constexpr (range_guarded<XT>()) {
    if (tile_needs_exact(p, XT, m0, m0 + BM, trk, finite_acc<1>(acc, MBLK, 1))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, n0, n0 + BN, 0);
      return;
    }
  }

  // Parked epilogue (fp32 y, epilogues without a residual or quantization):
  // two passes of MBLK/2 row blocks through LDS (the activation buffers are
  // free now), then each store instruction writes two whole 512-byte row runs
  // of the tile.  Stored straight from the accumulators, each instruction
  // covered 32 bytes of 32 rows, and the partly written lines doubled the HBM
  // write traffic (cfg1: 37.8 MB written for a 19.4 MB output; the kernel
  // measured 33.3 -> 32.1 us with the parked stores).  The stores are
  // non-temporal: the output streaming through the L2 evicted the activation
  // rows and packed weights that the other column and row tiles still read
  // (cfg1, same process: 26.0 -> 22.2 us with the output rotated over 22
  // buffers, 26.6 -> 25.0 us through bench.py, whose op reuses one output
  // allocation).
  constexpr bool kPark = (MODE & (kEpiRes | kEpiQuant)) == 0 && MBLK % 2 == 0;
  if (kPark && p.y_dt == DIMQ_F32 && p.ldy % 4 == 0) {
    constexpr int PR = MBLK / 2 * 32;  // rows per pass
    constexpr int PP = BN + 4;         // park pitch (floats)
    static_assert(!kPark || PR * PP * 4 <= (int)sizeof(As), "a pass fits in the activation buffers");
    float* park = reinterpret_cast<float*>(&As[0][0]);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      __syncthreads();  // the last stage's (pass 1: the previous pass's) readers are done
#pragma unroll
      for (int mbl = 0; mbl < MBLK / 2; ++mbl) {
        const int mb = pass * (MBLK / 2) + mbl;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<float4*>(park + (mbl * 32 + col) * PP + wave * 32 + 8 * j + 4 * g) =
              make_float4(acc[mb][4 * j], acc[mb][4 * j + 1], acc[mb][4 * j + 2], acc[mb][4 * j + 3]);
      }
      __syncthreads();
      constexpr int CH = PR * BN / 4;  // 16-byte chunks of a pass
#pragma unroll
      for (int u = 0; u < CH / 256; ++u) {
        const int c = tid + 256 * u;
        const int r = c / (BN / 4), c4 = c % (BN / 4);
        const int64_t m = m0 + pass * PR + r;
        const int64_t n = n0 + 4 * c4;
        if (m >= p.M) continue;
        const float4 a = *reinterpret_cast<const float4*>(park + r * PP + 4 * c4);
        const float4 sc = *reinterpret_cast<const float4*>(escale + 4 * c4);
        const float4 bb = *reinterpret_cast<const float4*>(ebias + 4 * c4);
        float v[4] = {a.x * sc.x + bb.x, a.y * sc.y + bb.y, a.z * sc.z + bb.z, a.w * sc.w + bb.w};
        const int64_t off = m * p.ldy + n;
        if (n + 4 <= p.N) {
          epi_m<MODE, 4>(p.epi, nullptr, off, true, v);
          typedef float f4v __attribute__((ext_vector_type(4)));
          const f4v vv = {v[0], v[1], v[2], v[3]};
          __builtin_nontemporal_store(vv, reinterpret_cast<f4v*>(reinterpret_cast<float*>(p.y) + off));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[i]));
        }
      }
    }
    return;
  }

  // epilogue: acc[mb][4j + i] = y[m][n], m = m0 + mb*32 + col, n = n0 + 32*wave + 8j + 4g + i
  const bool vec = p.ldy % 4 == 0;
  constexpr bool RES = (MODE & kEpiRes) != 0;
  ResPairs<4> rr[RES ? 4 : 1][RES ? MBLK : 1];  // 16-bit residuals: all loads out before the first store
  if constexpr ((MODE & kEpiRes) != 0) {
    if (res_pairs(p.epi, vec)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + wave * 32 + 8 * j + 4 * g;
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) {
        const int64_t m = m0 + mb * 32 + col;
        if (m < p.M && n + 4 <= p.N) res_issue<4>(p.epi, m * p.ldy + n, rr[j][mb]);
      }
    }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int nlo = 8 * j + 4 * g;
    const int64_t n = n0 + wave * 32 + nlo;
    float sc[4], bv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = __shfl(rscale, nlo + i, 32);
      bv[i] = ebias[wave * 32 + nlo + i];
    }
#pragma unroll
    for (int mb = 0; mb < MBLK; ++mb) {
      const int64_t m = m0 + mb * 32 + col;
      if (m >= p.M) continue;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[mb][4 * j + i] * sc[i] + bv[i];
      const int64_t off = m * p.ldy + n;
      if (vec && n + 4 <= p.N) {
        const ResPairs<4>* rp = nullptr;
        if constexpr (RES) rp = &rr[j][mb];
        epi_m<MODE, 4>(p.epi, rp, off, true, v);
        if (p.y_dt == DIMQ_F32) {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.y) + off) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          uint32_t h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) h[i] = p.y_dt == DIMQ_F16 ? float_to_f16_bits(v[i]) : float_to_bf16_bits(v[i]);
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + off) =
              make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < p.N) store_from_float(p.y, p.y_dt, off + i, epi1_m<MODE>(p.epi, off + i, v[i]));
      }
    }
  }
}

template <int BITS, int XT, int WGM, int WGN, int MBLK, int NBLK, int MODE = kEpiNone, int INTERLEAVE = 0>
int launch_lds(const GemmArgs& p, hipStream_t s) {
  constexpr int BM = WGM * MBLK * 32, BN = WGN * NBLK * 32;
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_lds_kernel<BITS, XT, WGM, WGN, MBLK, NBLK, MODE, INTERLEAVE>),
                     dim3(static_cast<unsigned>(tiles)), dim3(64 * WGM * WGN), 0, s, p);
  return check_launch("linear_codebook (shared-decode tiles)");
}

template <int BITS, int XT, int MBLK, int MODE = kEpiNone>
int launch_deep(const GemmArgs& p, hipStream_t s) {
  constexpr int BM = MBLK * 32, BN = 128;
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_deep_kernel<BITS, XT, MBLK, MODE>), dim3(static_cast<unsigned>(tiles)), dim3(256), 0, s,
                     p);
  return check_launch("linear_codebook (large tiles, deep pipeline)");
}

template <int BITS, int XT, int WGM, int WGN, int MBLK, int NBLK, bool CONV = false, int MODE = kEpiNone>
int launch_big(const GemmArgs& p, hipStream_t s) {
  constexpr int BM = WGM * MBLK * 32, BN = WGN * NBLK * 32;
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_big_kernel<BITS, XT, WGM, WGN, MBLK, NBLK, CONV, MODE>),
                     dim3(static_cast<unsigned>(tiles)), dim3(64 * WGM * WGN), 0, s, p);
  return check_launch(CONV ? "conv2d_codebook (implicit GEMM, large tiles)" : "linear_codebook (large tiles)");
}

// Implicit-GEMM conv tiles: 0 = 128x128 (2x2 waves of 64x64), 1 = 64x128
// (1x4 waves of 64x32), 2 = 256x128 (2x2 waves of 128x64).
// Epilogue modes: none / relu / residual / residual + relu on tiles 0 and 1
// (tile 2, an A/B option, only none; callers check gemm_conv_mode_ok).
template <int BITS, int XT, int WGM, int WGN, int MBLK, int NBLK>
int launch_big_conv_modes(const GemmArgs& p, int mode, hipStream_t s) {
  switch (mode) {
    case kEpiRelu: return launch_big<BITS, XT, WGM, WGN, MBLK, NBLK, true, kEpiRelu>(p, s);
    case kEpiRes: return launch_big<BITS, XT, WGM, WGN, MBLK, NBLK, true, kEpiRes>(p, s);
    case kEpiResRelu: return launch_big<BITS, XT, WGM, WGN, MBLK, NBLK, true, kEpiResRelu>(p, s);
    default: return launch_big<BITS, XT, WGM, WGN, MBLK, NBLK, true, kEpiNone>(p, s);
  }
}

// Implicit-GEMM conv tiles: 0 = 128x128 (2x2 waves of 64x64), 1 = 64x128
// (1x4 waves of 64x32) when the 128x128 grid would leave CUs idle.
template <int BITS>
int launch_big_conv_bits(const GemmArgs& p, int xt, int tile, hipStream_t s) {
  const int mode = epi_mode(p.epi);
#define DIMQ_CONV_TILES(XT)                                                 \
  switch (tile) {                                                           \
    case 1: return launch_big_conv_modes<BITS, XT, 1, 4, 2, 1>(p, mode, s); \
    default: return launch_big_conv_modes<BITS, XT, 2, 2, 2, 2>(p, mode, s); \
  }
  if (xt == DIMQ_F16) {
    DIMQ_CONV_TILES(DIMQ_F16)
  }
  DIMQ_CONV_TILES(DIMQ_BF16)
#undef DIMQ_CONV_TILES
}

// Linear tile ids (WGM x WGN waves of (MBLK*32) x (NBLK*32)):
//   2: 128x128 (2x2, 64x64)   7: 64x128 deep pipeline (kDeepMblk)
//  10: 256x256 shared decode (4x2, 64x128), next stage's decode woven between the MFMAs
// Epilogue modes: none / relu / gelu / residual on each; for fp16 inputs (the
// W4A4 activation codes) also none / relu / gelu with the next layer's
// activation quantization.
template <int BITS, int XT>
int launch_big_linear_modes(const GemmArgs& p, int tile, int mode, hipStream_t s) {
  if constexpr (XT == DIMQ_F16) {
    if ((mode & kEpiQuant) != 0) {
      switch (mode) {
#define DIMQ_QMODE(M)                                                                \
  case M:                                                                            \
    if (tile == 10) return launch_lds<BITS, XT, 4, 2, 2, 4, M, 8>(p, s);             \
    if (tile == 7) return launch_deep<BITS, XT, kDeepMblk, M>(p, s);                         \
    return launch_big<BITS, XT, 2, 2, 2, 2, false, M>(p, s);
        DIMQ_QMODE(kEpiQuant)
        DIMQ_QMODE(kEpiRelu | kEpiQuant)
        DIMQ_QMODE(kEpiGelu | kEpiQuant)
#undef DIMQ_QMODE
      }
    }
  }
  if (tile == 10) {
    switch (mode) {
      case kEpiRelu: return launch_lds<BITS, XT, 4, 2, 2, 4, kEpiRelu, 8>(p, s);
      case kEpiGelu: return launch_lds<BITS, XT, 4, 2, 2, 4, kEpiGelu, 8>(p, s);
      case kEpiRes: return launch_lds<BITS, XT, 4, 2, 2, 4, kEpiRes, 8>(p, s);
      default: return launch_lds<BITS, XT, 4, 2, 2, 4, kEpiNone, 8>(p, s);
    }
  }
  if (tile == 7) {
    switch (mode) {
      case kEpiRelu: return launch_deep<BITS, XT, kDeepMblk, kEpiRelu>(p, s);
      case kEpiGelu: return launch_deep<BITS, XT, kDeepMblk, kEpiGelu>(p, s);
      case kEpiRes: return launch_deep<BITS, XT, kDeepMblk, kEpiRes>(p, s);
      default: return launch_deep<BITS, XT, kDeepMblk, kEpiNone>(p, s);
    }
  }
  switch (mode) {
    case kEpiRelu: return launch_big<BITS, XT, 2, 2, 2, 2, false, kEpiRelu>(p, s);
    case kEpiGelu: return launch_big<BITS, XT, 2, 2, 2, 2, false, kEpiGelu>(p, s);
    case kEpiRes: return launch_big<BITS, XT, 2, 2, 2, 2, false, kEpiRes>(p, s);
    default: return launch_big<BITS, XT, 2, 2, 2, 2, false, kEpiNone>(p, s);
  }
}

template <int BITS>
int launch_big_bits(const GemmArgs& p, int xt, int tile, hipStream_t s) {
  const int mode = epi_mode(p.epi);
  switch (xt) {
    case DIMQ_F32: return launch_big_linear_modes<BITS, DIMQ_F32>(p, tile, mode, s);
    case DIMQ_F16: return launch_big_linear_modes<BITS, DIMQ_F16>(p, tile, mode, s);
    default: return launch_big_linear_modes<BITS, DIMQ_BF16>(p, tile, mode, s);
  }
}

}  // namespace

int launch_big_b2(const GemmArgs& p, int xt, int tile, hipStream_t s);
int launch_big_b3(const GemmArgs& p, int xt, int tile, hipStream_t s);
int launch_big_b4(const GemmArgs& p, int xt, int tile, hipStream_t s);
int launch_big_conv_b2(const GemmArgs& p, int xt, int tile, hipStream_t s);
int launch_big_conv_b3(const GemmArgs& p, int xt, int tile, hipStream_t s);
int launch_big_conv_b4(const GemmArgs& p, int xt, int tile, hipStream_t s);

}  // namespace dimq
