// Pre-decoded-weight GEMM for the large-M Linear shapes (ViT-B/16 at
// M = 12,608): y[M,N] = epilogue(x[M,K] W_hat^T), in two launches.
//
//   1. prep_kernel: the packed b-bit indices (dimq_packed_lut layout,
//      LSB-first, row-major [N, K]) and the codebook rows -> W_hat as fp16
//      [N, K] in natural k order, each row scaled by the power of two 2^e of
//      the register-codebook kernels (max|c| 2^e in [2^14, 2^15), decode.h),
//      plus the per-row factor acc_scale 2^-e, in the caller's workspace.
//      Every weight is decoded once per call.  The fused kernels decode it
//      once per 256-row activation tile (50 times at M 12,608), which rocprof
//      counters put at about two thirds of their VALU instructions, the VALU
//      being busy as long as the matrix cores.
//   2. gemm_pd_kernel: an fp16 x fp16 GEMM whose operands reach LDS through
//      global_load_lds (16 bytes per lane, no registers held, no VALU in the
//      main loop), in a ring of S stages of 32 or 64 k.  A stage row's 16-byte
//      chunks are XOR-swizzled (pd_swz) so the 16-byte fragment reads of
//      sixteen consecutive rows cover all 64 banks.  Tile shapes are listed
//      at PdTile; e.g. 8 waves (4 along m x 2 along n) on a 256 x 256 tile,
//      wave tile 64 x 128, v_mfma_f32_32x32x16_f16 with the weights as the A
//      operand (rows = output columns n) and the activations as the B operand,
//      so a lane's accumulator holds 4 consecutive n of one m.  The epilogue
//      parks each column pass in LDS and stores 8-column runs of rows.
//
// fp16 activations (the model's LayerNorm and fc1 outputs) are read as they
// are; bf16 and fp32 activations are converted to fp16 in the first launch,
// with the range guard of common.h applied per tile from per-row flags.
#include "gemm_big.h"

namespace dimq {
namespace {

constexpr int kPdK = 32;  // k granularity of the path (halves): the shorter stage

// Below this many activation rows the fused kernels' per-tile decode costs
// no more than the extra launch and the fp16 copies (cfg1, M 1576 fp32: 29.5
// us either way, same box).
constexpr int64_t kPredecodeMinM = 2048;

// A stage row holds CH 16-byte chunks (CH 4: 32 k, CH 8: 64 k); chunk c of
// row r lives at r * 16 CH + ((c ^ pd_swz<CH>(r)) << 4).  A 16-byte LDS read
// serves 16 lanes (256 bytes, gfx950's 64 banks) per clock, i.e. 256 / (16 CH)
// rows per bank window; the swizzle gives the 16 rows of one read 16
// distinct 16-byte slots.
template <int CH>
__device__ __forceinline__ int pd_swz(int r) {
  return (r / (16 / CH)) & (CH - 1);
}

// s_waitcnt vmcnt(n), leaving the other counters alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// One global_load_lds of 16 bytes per lane into LDS at byte address lds + 16 * lane.
// Issued as inline assembly so that the compiler's wait insertion, which
// would otherwise make every later LDS read wait for all such loads still in
// flight (it cannot tell the ring's slots apart), leaves the waits to the
// kernel: wait_vmcnt before the barrier that publishes a stage.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

constexpr int kPdRows = 4;     // weight rows per predecode work-group (2: 10.1 us, 4: 9.3, 8: slower, per ViT-B/16 block)
constexpr int kPdGroups = 16;  // 8-index groups per thread held in registers (K <= 4096 in one pass)

// Weight rows kPdRows b .. kPdRows b + kPdRows - 1 -> fp16 in wd, their factors acc_scale 2^-e in rs.
template <int BITS>
__device__ __forceinline__ void predecode_rows(const uint8_t* __restrict__ w, const void* cb, int cb_dt,
                                               int64_t cb_rows, int cb_size, int64_t N, int64_t K, float acc_scale,
                                               uint16_t* __restrict__ wd, float* __restrict__ rs, int64_t b) {
  constexpr int E = 1 << BITS;
  __shared__ float cbs[kPdRows * E];
  __shared__ uint32_t tab[kPdRows * E];  // fp16 bits of the scaled entries
  const int tid = threadIdx.x;
  const int64_t r0 = b * kPdRows;
  const int gpr = static_cast<int>(K >> 3);  // 8-index groups per row (K % 32 == 0)
  const int nr = N - r0 < kPdRows ? static_cast<int>(N - r0) : kPdRows;
  const int total = nr * gpr;
  // group gi = tid + 256 u: row gi / gpr, indices 8 (gi % gpr) .. + 7 = BITS whole bytes
  auto load_group = [&](int gi) -> uint32_t {
    const int r = gi / gpr;
    const uint8_t* src = w + ((((r0 + r) * K) + 8 * (gi - r * gpr)) * BITS >> 3);
    if constexpr (BITS == 2) return *reinterpret_cast<const uint16_t*>(src);
    if constexpr (BITS == 4) return *reinterpret_cast<const uint32_t*>(src);
    return static_cast<uint32_t>(src[0]) | (static_cast<uint32_t>(src[1]) << 8) | (static_cast<uint32_t>(src[2]) << 16);
  };
  // the packed words first: their latency overlaps the codebook loads
  uint32_t v[kPdGroups];
#pragma unroll
  for (int u = 0; u < kPdGroups; ++u) {
    const int gi = tid + 256 * u;
    v[u] = gi < total ? load_group(gi) : 0u;
  }
  if (tid < kPdRows * E) {
    const int r = tid / E, j = tid - r * E;
    const int64_t row = cb_rows == 1 ? 0 : (r0 + r < N ? r0 + r : N - 1);
    cbs[tid] = j < cb_size ? load_as_float(cb, cb_dt, row * cb_size + j) : 0.0f;
  }
  __syncthreads();
  // the scaled fp16 entries (one thread per entry, the row's exponent from the staged row)
  if (tid < kPdRows * E) {
    const int r = tid / E;
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) mx = fmaxf(mx, fabsf(cbs[r * E + j]));
    const int e = cb_exponent(mx);
    tab[tid] = float_to_f16_bits(ldexpf(cbs[tid], e));
    if (tid - r * E == 0 && r < nr) rs[r0 + r] = ldexpf(acc_scale, -e);
  }
  __syncthreads();
  auto store_group = [&](int gi, uint32_t x) {
    const int r = gi / gpr;
    const uint32_t* t = tab + r * E;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      h[i] = t[(x >> (2 * i * BITS)) & (E - 1)] | (t[(x >> ((2 * i + 1) * BITS)) & (E - 1)] << 16);
    *reinterpret_cast<uint4*>(wd + (r0 + r) * K + 8 * (gi - r * gpr)) = make_uint4(h[0], h[1], h[2], h[3]);
  };
#pragma unroll
  for (int u = 0; u < kPdGroups; ++u) {
    const int gi = tid + 256 * u;
    if (gi < total) store_group(gi, v[u]);
  }
  for (int gi = tid + 256 * kPdGroups; gi < total; gi += 256) store_group(gi, load_group(gi));
}

constexpr int kPxRows = 8;  // activation rows per conversion work-group

// Activation rows 8 b .. 8 b + 7 (bf16 or fp32) -> fp16 in xh (row pitch K),
// rounded to nearest; flags[m] != 0 when row m holds a value of magnitude
// >= 2^-7 after the rounding (the range guard's test, common.h).
template <int XT>
__device__ __forceinline__ void convert_rows(const void* __restrict__ x, int64_t M, int64_t K, int64_t ldx,
                                             uint16_t* __restrict__ xh, uint32_t* __restrict__ flags, int64_t b) {
  __shared__ uint32_t fl[kPxRows];
  const int tid = threadIdx.x;
  const int64_t r0 = b * kPxRows;
  const int gpr = static_cast<int>(K >> 3);
  const int nr = M - r0 < kPxRows ? static_cast<int>(M - r0) : kPxRows;
  if (tid < kPxRows) fl[tid] = 0u;
  __syncthreads();
  for (int gi = tid; gi < nr * gpr; gi += 256) {
    const int r = gi / gpr;
    const int64_t m = r0 + r, k = 8 * static_cast<int64_t>(gi - r * gpr);
    float v[8];
    if constexpr (XT == DIMQ_F32) {
      const float4* s4 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + m * ldx + k);
      const float4 a = s4[0], c = s4[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
      const uint4 t = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + m * ldx + k);
      const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    }
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = f16x2_rne(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4*>(xh + m * K + k) = make_uint4(h[0], h[1], h[2], h[3]);
    const uint32_t big = ((h[0] | h[1]) | (h[2] | h[3])) & kRangeBigBits;
    if (big) atomicOr(&fl[r], 1u);
  }
  __syncthreads();
  if (tid < nr) flags[r0 + tid] = fl[tid];
}

// One launch: work-groups [0, nbw) decode weight row pairs, the rest (when
// XT is not fp16) convert activation rows.
template <int BITS, int XT>
__global__ __launch_bounds__(256) void prep_kernel(const uint8_t* __restrict__ w, const void* cb, int cb_dt,
                                                   int64_t cb_rows, int cb_size, int64_t N, int64_t K,
                                                   float acc_scale, uint16_t* __restrict__ wd, float* __restrict__ rs,
                                                   int64_t nbw, const void* __restrict__ x, int64_t M, int64_t ldx,
                                                   uint16_t* __restrict__ xh, uint32_t* __restrict__ flags) {
  const int64_t b = blockIdx.x;
  if (b < nbw) {
    predecode_rows<BITS>(w, cb, cb_dt, cb_rows, cb_size, N, K, acc_scale, wd, rs, b);
  } else if constexpr (XT != DIMQ_F16) {
    convert_rows<XT>(x, M, K, ldx, xh, flags, b - nbw);
  }
}

// xop / lda: the fp16 activations the matrix cores read (x itself, or its
// converted copy); with GUARD the copy's per-row flags decide, with the
// accumulators' finiteness, whether the tile is recomputed in fp32 from p.x
// (of dtype xt) and the packed weights.
template <int WGM, int WGN, int MBLK, int NBLK, int MODE, int S, bool GUARD, int CH>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_pd_kernel(const GemmArgs p, const uint16_t* __restrict__ wd,
                                                                 const float* __restrict__ rs,
                                                                 const uint16_t* __restrict__ xop, int64_t lda,
                                                                 const uint32_t* __restrict__ flags, int xt, int bits) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int BM = WGM * MBLK * 32;
  constexpr int BN = WGN * NBLK * 32;
  constexpr int KS = 8 * CH;                // k per stage
  constexpr int RB = 16 * CH;               // bytes of a stage row
  constexpr int RPB = 64 / CH;              // rows one wave-wide 16-byte load fills
  constexpr int NSTEP = CH / 2;             // k16 steps per stage
  constexpr int RSTAGE = (BN + BM) * RB;    // bytes of one stage: weight rows, then activation rows
  constexpr int NW = NT / 64;
  constexpr int NLB = (BN + BM) / RPB;       // wave-wide 16-byte loads per stage
  constexpr int LPT = (NLB + NW - 1) / NW;   // loads per thread and stage; the last may cover only some waves
  constexpr int LPT_MIN = NLB / NW;          // loads every wave issues per stage
  static_assert(CH == 4 || CH == 8, "32 or 64 k per stage");
  static_assert(BN % RPB == 0 && BM % RPB == 0, "a wave's load covers rows of one operand");
  static_assert(LPT_MIN >= 1 && S * LPT < 64, "outstanding loads fit the vmcnt counter");
  static_assert(BN <= NT, "one thread per tile column stages the column factors");
  __shared__ __attribute__((aligned(16))) uint8_t sm[S * RSTAGE];
  // after the main loop: the tile's column factors at the end of the ring
  float* escale = reinterpret_cast<float*>(sm + S * RSTAGE) - 2 * BN;
  float* ebias = escale + BN;

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

  // the tile's column factors first: their loads are then older than every
  // stage load, so the stage waits below cover them
  float my_scale = 0.0f, my_bias = 0.0f;
  if (tid < BN) {
    const int64_t n = n0 + tid < p.N ? n0 + tid : p.N - 1;
    my_scale = rs[n];
    if (p.bias) my_bias = load_as_float(p.bias, p.bias_dt, n);
  }

  // load j of this thread: the wave's block b = j * (NT / 64) + wave holds
  // stage rows RPB b .. RPB b + RPB - 1 (weight rows first, then activation
  // rows); lane l fills LDS chunk l % CH of row RPB b + l / CH, i.e. global
  // chunk (l % CH) ^ swizzle.  Rows past N or M repeat the last row (not stored).
  const uint16_t* src[LPT];
#pragma unroll
  for (int j = 0; j < LPT; ++j) {
    const int lb = j * NW + wave < NLB ? j * NW + wave : NLB - 1;  // past NLB: not issued
    const int row = RPB * lb + lane / CH;
    const int c = (lane % CH) ^ pd_swz<CH>(row);
    if (row < BN) {
      const int64_t n = n0 + row < p.N ? n0 + row : p.N - 1;
      src[j] = wd + n * p.K + 8 * c;
    } else {
      const int64_t m = m0 + (row - BN) < p.M ? m0 + (row - BN) : p.M - 1;
      src[j] = xop + m * lda + 8 * c;
    }
  }
  const int64_t nk = p.K / KS;
  const uint32_t smb = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_g*)sm));  // LDS address of the ring
  // loads J0 .. J1 - 1 of stage kt into ring slot `slot`
  auto issue_part = [&](int64_t kt, int slot, auto j0c, auto j1c) {
    if (kt >= nk) return;
    const int64_t k = kt * KS;
    constexpr int J0 = decltype(j0c)::value, J1 = decltype(j1c)::value;
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      if (LPT != LPT_MIN && j == LPT - 1 && j * NW + wave >= NLB) break;  // wave-uniform
      dma16(src[j] + k, smb + slot * RSTAGE + (j * NW + wave) * 1024);
    }
  };
  using J0c = std::integral_constant<int, 0>;
  using JHc = std::integral_constant<int, LPT / 2>;
  using JLc = std::integral_constant<int, LPT>;
  auto issue = [&](int64_t kt, int slot) { issue_part(kt, slot, J0c{}, JLc{}); };
  // With two slots the stage that refills the slot freed by a barrier is
  // requested in two halves, after the barrier and after the next k16 step's
  // MFMAs: eight 16-byte loads per lane at once held the waves at the
  // vector-memory issue (qkv 70.8 -> 65.8 us, fc2 -3 %, same box).
  constexpr bool SPLIT = S == 2 && NSTEP >= 2;
  // s_waitcnt leaving at most n stages' worth of this thread's youngest loads
  // in flight (0 <= n < S): n LPT_MIN, which a wave that issues LPT loads per
  // stage satisfies only once some of the youngest stage's loads have landed
  // too (a conservative wait, never a short one)
  auto wait_stages = [&](int64_t n) {
    static_for<S>([&](auto ic) {
      constexpr int I = decltype(ic)::value;
      if (I == n) wait_vmcnt<I * LPT_MIN>();
    });
  };

  floatx16g acc[MBLK][NBLK];
#pragma unroll
  for (int mb = 0; mb < MBLK; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][nb][i] = 0.0f;

  // fragment offsets: rows rbase + col (rbase % 32 == 0) share the swizzle of col
  const int sw = pd_swz<CH>(col);
  // fragments of k16 step s of the stage in ring slot `slot`: chunk 2 s + g
  auto load = [&](int slot, int s, half8 (&wf)[NBLK], half8 (&xf)[MBLK]) {
    const uint8_t* base = sm + slot * RSTAGE + col * RB + (((2 * s + g) ^ sw) << 4);
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
      wf[nb] = *reinterpret_cast<const half8*>(base + (wn * NBLK + nb) * 32 * RB);
#pragma unroll
    for (int mb = 0; mb < MBLK; ++mb)
      xf[mb] = *reinterpret_cast<const half8*>(base + BN * RB + (wm * MBLK + mb) * 32 * RB);
  };
  auto mma = [&](const half8 (&wf)[NBLK], const half8 (&xf)[MBLK]) {
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int mb = 0; mb < MBLK; ++mb) acc[mb][nb] = mfma32(wf[nb], xf[mb], acc[mb][nb]);
  };

  // Ring of S slots, stage kt in slot kt % S.  Each step's fragment reads are
  // issued before the previous step's MFMAs, so LDS latency hides behind the
  // matrix cores; the barrier that publishes stage kt + 1 sits before the
  // last step of stage kt, after which slot kt % S (read completely: the
  // barrier's fence waits for this wave's LDS reads) takes stage kt + S.
#pragma unroll
  for (int s = 0; s < S; ++s) issue(s, s);
  wait_stages(nk - 1 < S - 1 ? nk - 1 : S - 1);  // stage 0 landed; stages 1 .. S - 1 may be in flight
  lds_barrier();
  half8 wfr[2][NBLK], xfr[2][MBLK];  // fragments of two consecutive k16 steps (NSTEP is even)
  load(0, 0, wfr[0], xfr[0]);
  int slot = 0;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int next = slot == S - 1 ? 0 : slot + 1;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      if (st + 1 < NSTEP) {
        load(slot, st + 1, wfr[(st + 1) & 1], xfr[(st + 1) & 1]);
      } else {
        // stage kt + 1 landed; stages kt + 2 .. min(kt + S - 1, nk - 1) may be in flight
        if (kt + 1 < nk) wait_stages(nk - 2 - kt < S - 2 ? nk - 2 - kt : S - 2);
        lds_barrier();
        if constexpr (SPLIT) issue_part(kt + S, slot, J0c{}, JHc{});
        else issue(kt + S, slot);
        if (kt + 1 < nk) load(next, 0, wfr[0], xfr[0]);
      }
      mma(wfr[st & 1], xfr[st & 1]);
      // the second half of stage kt + 1 (slot `next`), whose first half the
      // previous barrier requested; the prologue requested stage 1 whole
      if constexpr (SPLIT) {
        if (st == 0 && kt > 0) issue_part(kt + 1, next, JHc{}, JLc{});
      }
    }
    slot = next;
  }
  __syncthreads();  // every wave is done with the ring before it is reused
  if constexpr (GUARD) {
    bool big = false;
    for (int r = tid; r < BM; r += NT) big |= m0 + r < p.M && flags[m0 + r] != 0u;
    const int bad = __syncthreads_or(!finite_acc<1>(&acc[0][0], MBLK, NBLK));
    if (!__syncthreads_or(big) || bad) {
      exact_tile_out(p, xt, bits, m0, m0 + BM, n0, n0 + BN, 0);
      return;
    }
  }
  if (tid < BN) {
    escale[tid] = my_scale;
    ebias[tid] = my_bias;
  }
  __syncthreads();

  // Epilogue in NBLK passes: pass nb parks every wave's column block nb
  // (acc[mb][nb][4j + i] = tile row wm*MBLK*32 + mb*32 + col, pass column
  // wn*32 + 8j + 4g + i) as fp32 in the ring, then the work-group stores it
  // as 8-column runs of rows.
  constexpr int PW = WGN * 32;
  constexpr int OTP = PW + 4;
  static_assert(BM * OTP * 4 + 2 * BN * 4 <= S * RSTAGE, "a parked pass and the column factors fit in the ring");
  constexpr int NCHUNK = BM * PW / 8;
  constexpr int CPT = (NCHUNK + NT - 1) / NT;
  float* ot = reinterpret_cast<float*>(sm);
  const bool vec8 = p.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && p.y_dt != DIMQ_F64;
  // 16-bit residuals of pass nb + 1 are requested before pass nb's stores
  const bool rpair = (MODE & kEpiRes) && res_pairs(p.epi, vec8);
  auto res_load = [&](int nb, ResPairs<8> (&rr)[CPT]) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * NT;
      const int r = c / (PW / 8), q = c - r * (PW / 8);
      const int64_t m = m0 + r;
      const int64_t n = n0 + (q >> 2) * NBLK * 32 + nb * 32 + 8 * (q & 3);
      if (c < NCHUNK && m < p.M && n + 8 <= p.N) res_issue<8>(p.epi, m * p.ldy + n, rr[u]);
    }
  };
  ResPairs<8> rr[CPT], rn[CPT];
  if constexpr ((MODE & kEpiRes) != 0) {
    if (rpair) res_load(0, rr);
  }
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
    if constexpr ((MODE & kEpiRes) != 0) {
      if (rpair && nb + 1 < NBLK) res_load(nb + 1, rn);
    }
    // Chunk c = tid + u NT covers row c / (PW / 8) and the 8 columns nl ..
    // nl + 7 of column group q = c % (PW / 8), the same for all of this
    // thread's chunks (NT is a multiple of PW / 8): its column factors are
    // read once per pass as four aligned 16-byte loads.  Every chunk's parked
    // values are read before any is used, so the LDS latencies overlap;
    // per-chunk control flow only guards the stores.
    static_assert(NT % (PW / 8) == 0, "a thread's chunks share one column group");
    const int qg = tid % (PW / 8);
    const int nlg = (qg >> 2) * NBLK * 32 + nb * 32 + 8 * (qg & 3);  // a multiple of 8, nlg + 7 < BN
    const float4* es4 = reinterpret_cast<const float4*>(escale) + nlg / 4;
    const float4* eb4 = reinterpret_cast<const float4*>(ebias) + nlg / 4;
    const float4 s0 = es4[0], s1 = es4[1], b0 = eb4[0], b1 = eb4[1];
    float v[CPT][8];
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * NT < NCHUNK ? tid + u * NT : NCHUNK - 1;
      const int r = c / (PW / 8);
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
      if (NCHUNK % NT != 0 && c >= NCHUNK) break;
      const int r = c / (PW / 8), q = c - r * (PW / 8);
      const int64_t m = m0 + r;
      const int64_t n = n0 + (q >> 2) * NBLK * 32 + nb * 32 + 8 * (q & 3);
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
    if constexpr ((MODE & kEpiRes) != 0) {
#pragma unroll
      for (int u = 0; u < CPT; ++u) rr[u] = rn[u];
    }
  }
}

// Tile shapes (WGM x WGN waves of (MBLK*32) x (NBLK*32), a ring of S stages
// of 8 CH k), measured on the ViT-B/16 shapes at M 12,608 (kernel time, fp16
// x, bf16 y; 64-k stages in two slots measured 3-8 % faster than 32-k stages
// in three for tiles 0 and 2, the same box, pre-decode launch included):
//   0: 256 x 256, 8 waves of 64 x 128, one work-group per CU: qkv (N 2304)
//      70.3 us against 78.9 for tile 1;
//   1: 128 (m) x 256 (n), 4 waves of 64 x 128, 72 KB of LDS so two
//      work-groups share a CU and one's epilogue overlaps the other's main
//      loop: fc1 (N 3072) 93.6 us (98.7 with the fused GELU) against 100.3
//      (110.7) for tile 0, whose 600 tiles leave a third round a third full;
//   2: 128 (m) x 384 (n), 8 waves of 64 x 96: N 768 (proj, fc2) as 198 tiles
//      instead of 150 on 256 CUs, fc2 73.7 us against 79.3.
template <int TILE>
struct PdTile;
template <>
struct PdTile<0> {
  static constexpr int WGM = 4, WGN = 2, MBLK = 2, NBLK = 4, S = 2, CH = 8;
};
template <>
struct PdTile<1> {
  static constexpr int WGM = 2, WGN = 2, MBLK = 2, NBLK = 4, S = 3, CH = 4;
};
template <>
struct PdTile<2> {
  static constexpr int WGM = 2, WGN = 4, MBLK = 2, NBLK = 3, S = 2, CH = 8;
};
//   3: 128 x 128, 4 waves of 64 x 64, 48 KB of LDS: N <= 128 (M 100,352 x N
//      128 x K 1152: 77 us against 120 us on the half-empty tile 0) and shapes
//      whose tile-1 grid would leave CUs idle.
template <>
struct PdTile<3> {
  static constexpr int WGM = 2, WGN = 2, MBLK = 2, NBLK = 2, S = 3, CH = 4;
};
//   4: 160 x 256, 10 waves of 32 x 128 (the last of a stage's six 16-byte
//      loads per lane covers two waves): N 768 as 237 tiles instead of 198
//      on 256 CUs; proj (K 768) 40.3-41.5 -> 37.9-38.1 us, both launches,
//      same box; fc2 (K 3072) was first no faster (wave tiles of 32 x 128
//      read 1.25 fragments per MFMA against 0.83), and with the current
//      epilogue 81.2 against 84.7 us on tile 2 (ViT-B/16 forward 4.16-4.18
//      -> 4.14 ms, same box).
template <>
struct PdTile<4> {
  static constexpr int WGM = 5, WGN = 2, MBLK = 1, NBLK = 4, S = 2, CH = 8;
};

// Tiles 0, 2 and 4 stage 64 k at a time (two slots) and need K % 64 == 0.
// Tile sweep at the ViT-B/16 shapes (M 12,608, fp16 x, 4-bit, one process,
// both launches): qkv 68.4 us on tile 0 (tiles 1-4: 76.5-81.5), proj 30.7 on
// tile 4 (30.4 on 2), fc1 110.9 on tile 1 (118.2-129.1), fc2 (K 3072) 81.2 on
// tile 4 against 84.7 on tile 2.
int pd_pick_tile(int64_t M, int64_t N, int64_t K) {
  const bool k64 = K % 64 == 0;
  if (k64 && N % 256 == 0 && N <= 768 && M >= 4096) return 4;
  if (k64 && N % 384 == 0 && N <= 1536) return 2;
  if (N <= 128 || ((M + 127) / 128) * ((N + 255) / 256) < 256) return 3;
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t rem = tiles % 256;  // work-groups of the last round of tile 0
  return (!k64 || (rem != 0 && rem * 2 < 256)) ? 1 : 0;
}

struct PdOperands {
  const uint16_t* wd;
  const float* rs;
  const uint16_t* xa;
  int64_t lda;
  const uint32_t* flags;  // null: fp16 activations, no guard
  int xt, bits;
};

template <int TILE, int MODE>
int launch_pd_gemm(const GemmArgs& p, const PdOperands& o, hipStream_t s) {
  using T = PdTile<TILE>;
  constexpr int BM = T::WGM * T::MBLK * 32, BN = T::WGN * T::NBLK * 32;
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  if (o.flags) {
    hipLaunchKernelGGL((gemm_pd_kernel<T::WGM, T::WGN, T::MBLK, T::NBLK, MODE, T::S, true, T::CH>),
                       dim3(static_cast<unsigned>(tiles)), dim3(64 * T::WGM * T::WGN), 0, s, p, o.wd, o.rs, o.xa,
                       o.lda, o.flags, o.xt, o.bits);
  } else {
    hipLaunchKernelGGL((gemm_pd_kernel<T::WGM, T::WGN, T::MBLK, T::NBLK, MODE, T::S, false, T::CH>),
                       dim3(static_cast<unsigned>(tiles)), dim3(64 * T::WGM * T::WGN), 0, s, p, o.wd, o.rs, o.xa,
                       o.lda, o.flags, o.xt, o.bits);
  }
  return check_launch("linear_codebook (pre-decoded weights)");
}

template <int TILE>
int launch_pd_modes(const GemmArgs& p, int mode, const PdOperands& o, hipStream_t s) {
  switch (mode) {
    case kEpiRelu: return launch_pd_gemm<TILE, kEpiRelu>(p, o, s);
    case kEpiGelu: return launch_pd_gemm<TILE, kEpiGelu>(p, o, s);
    case kEpiRes: return launch_pd_gemm<TILE, kEpiRes>(p, o, s);
    default: return launch_pd_gemm<TILE, kEpiNone>(p, o, s);
  }
}

// with_w false: the weights are decoded already, only the activations are
// converted (nothing to launch for fp16 activations)
template <int BITS, int XT>
void launch_prep(const GemmArgs& p, bool with_w, uint16_t* wd, float* rs, uint16_t* xh, uint32_t* flags,
                 hipStream_t s) {
  const int64_t nbw = with_w ? (p.N + kPdRows - 1) / kPdRows : 0;
  const int64_t nbx = XT == DIMQ_F16 ? 0 : (p.M + kPxRows - 1) / kPxRows;
  if (nbw + nbx == 0) return;
  hipLaunchKernelGGL((prep_kernel<BITS, XT>), dim3(static_cast<unsigned>(nbw + nbx)), dim3(256), 0, s, p.w, p.cb,
                     p.cb_dt, p.cb_rows, p.cb_size, p.N, p.K, p.acc_scale, wd, rs, nbw, p.x, p.M, p.ldx, xh, flags);
}

template <int BITS>
void launch_prep_bits(const GemmArgs& p, int xt, bool with_w, uint16_t* wd, float* rs, uint16_t* xh,
                      uint32_t* flags, hipStream_t s) {
  switch (xt) {
    case DIMQ_F16: launch_prep<BITS, DIMQ_F16>(p, with_w, wd, rs, xh, flags, s); break;
    case DIMQ_BF16: launch_prep<BITS, DIMQ_BF16>(p, with_w, wd, rs, xh, flags, s); break;
    default: launch_prep<BITS, DIMQ_F32>(p, with_w, wd, rs, xh, flags, s); break;
  }
}

// Several layers' weights decoded in one launch (the per-call decode of the
// first launch above, batched): job j's work-groups start at b0.
constexpr int kPdBatchMax = 32;
struct PdJob {
  const uint8_t* w;
  const void* cb;
  uint16_t* wd;
  float* rs;
  int64_t cb_rows, N, K, b0;
  int cb_dt, cb_size;
};
struct PdBatch {
  PdJob job[kPdBatchMax];
  int count;
};

template <int BITS>
__global__ __launch_bounds__(256) void predecode_batch_kernel(const PdBatch bt) {
  const int64_t b = blockIdx.x;
  int j = 0;
  for (int i = 1; i < bt.count; ++i) j = b >= bt.job[i].b0 ? i : j;
  const PdJob& J = bt.job[j];
  predecode_rows<BITS>(J.w, J.cb, J.cb_dt, J.cb_rows, J.cb_size, J.N, J.K, 1.0f, J.wd, J.rs, b - J.b0);
}

}  // namespace

constexpr int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Workspace of the pre-decoded path: W_hat fp16 [N, K], N fp32 factors and,
// for bf16 / fp32 activations, their fp16 copy [M, K] and M row flags.
int64_t predecoded_ws_bytes(int64_t M, int64_t K, int64_t N, int bits, int x_dtype) {
  if (M < kPredecodeMinM || K <= 0 || N <= 0 || K % kPdK != 0 || !(bits >= 2 && bits <= 4)) return 0;
  if (!(x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16 || x_dtype == DIMQ_F32)) return 0;
  const int64_t w = align256(N * K * 2) + align256(N * 4);
  return x_dtype == DIMQ_F16 ? w : w + align256(M * K * 2) + align256(M * 4);
}

// Bytes of one layer's decoded weights: W_hat fp16 [N, K], then N fp32 row
// factors (0: the layer cannot take the pre-decoded path).
int64_t predecoded_w_bytes(int64_t N, int64_t K, int bits) {
  if (K <= 0 || N <= 0 || K % kPdK != 0 || !(bits >= 2 && bits <= 4)) return 0;
  return align256(N * K * 2) + align256(N * 4);
}

// Decodes jobs [0, count) (all of `bits`) into their wd / rs, kPdBatchMax per launch.
int launch_predecode_batch(const PdJob* jobs, int count, int bits, hipStream_t s) {
  for (int j0 = 0; j0 < count; j0 += kPdBatchMax) {
    PdBatch bt{};
    int64_t nb = 0;
    bt.count = count - j0 < kPdBatchMax ? count - j0 : kPdBatchMax;
    for (int i = 0; i < bt.count; ++i) {
      bt.job[i] = jobs[j0 + i];
      bt.job[i].b0 = nb;
      nb += (bt.job[i].N + kPdRows - 1) / kPdRows;
    }
    if (nb == 0) continue;
    switch (bits) {
      case 2: hipLaunchKernelGGL(predecode_batch_kernel<2>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s, bt); break;
      case 3: hipLaunchKernelGGL(predecode_batch_kernel<3>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s, bt); break;
      default: hipLaunchKernelGGL(predecode_batch_kernel<4>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s, bt); break;
    }
    const int rc = check_launch("codebook weight pre-decode (batch)");
    if (rc != DIMQ_OK) return rc;
  }
  return DIMQ_OK;
}

// Jobs of any bit width: one batch of launches per width present.
int launch_predecode_jobs(const DimqPredecodeJob* jobs, int count, hipStream_t s) {
  for (int bits = 2; bits <= 4; ++bits) {
    PdJob pj[kPdBatchMax];
    int n = 0;
    for (int j = 0; j < count; ++j) {
      const DimqPredecodeJob& J = jobs[j];
      if (J.bits != bits) continue;
      uint8_t* d = static_cast<uint8_t*>(J.decoded);
      pj[n++] = PdJob{J.packed_w, J.codebook, reinterpret_cast<uint16_t*>(d),
                      reinterpret_cast<float*>(d + align256(J.out_features * J.in_features * 2)), J.cb_rows,
                      J.out_features, J.in_features, 0, J.cb_dtype, static_cast<int>(J.cb_size)};
      if (n == kPdBatchMax) {
        const int rc = launch_predecode_batch(pj, n, bits, s);
        if (rc != DIMQ_OK) return rc;
        n = 0;
      }
    }
    if (n > 0) {
      const int rc = launch_predecode_batch(pj, n, bits, s);
      if (rc != DIMQ_OK) return rc;
    }
  }
  return DIMQ_OK;
}

// Runs the two launches; -1 when the call does not take this path (shape,
// dtype, epilogue, alignment or too small a workspace).  With `decoded`
// (predecoded_w_bytes of this layer, 256-byte aligned, filled by
// launch_predecode_batch) the first launch only converts bf16 / fp32
// activations, into a workspace of the activation part's size.
int launch_predecoded(const GemmArgs& p, int bits, int x_dtype, void* ws, int64_t ws_bytes, hipStream_t s,
                      const void* decoded) {
  const int64_t need_all = predecoded_ws_bytes(p.M, p.K, p.N, bits, x_dtype);
  if (need_all == 0) return -1;
  const int64_t wbytes = predecoded_w_bytes(p.N, p.K, bits);
  const int64_t need = decoded ? need_all - wbytes : need_all;
  if (decoded && (reinterpret_cast<uintptr_t>(decoded) & 255) != 0) return -1;
  if (need > 0 && (ws == nullptr || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 255) != 0)) return -1;
  const int xs = x_dtype == DIMQ_F32 ? 4 : 2;
  if (p.conv || !p.fast_b || !p.vec_a || (p.ldx * xs) % 16 != 0) return -1;
  const int mode = epi_mode(p.epi);
  if (!(mode == kEpiNone || mode == kEpiRelu || mode == kEpiGelu || mode == kEpiRes)) return -1;
  uint8_t* wbase = decoded ? static_cast<uint8_t*>(const_cast<void*>(decoded)) : static_cast<uint8_t*>(ws);
  uint16_t* wd = reinterpret_cast<uint16_t*>(wbase);
  float* rs = reinterpret_cast<float*>(wbase + align256(p.N * p.K * 2));
  uint16_t* xh = nullptr;
  uint32_t* flags = nullptr;
  if (x_dtype != DIMQ_F16) {
    xh = reinterpret_cast<uint16_t*>(decoded ? static_cast<uint8_t*>(ws) : wbase + wbytes);
    flags = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(xh) + align256(p.M * p.K * 2));
  }
  switch (bits) {
    case 2: launch_prep_bits<2>(p, x_dtype, decoded == nullptr, wd, rs, xh, flags, s); break;
    case 3: launch_prep_bits<3>(p, x_dtype, decoded == nullptr, wd, rs, xh, flags, s); break;
    default: launch_prep_bits<4>(p, x_dtype, decoded == nullptr, wd, rs, xh, flags, s); break;
  }
  const int rc = check_launch("linear_codebook (weight pre-decode)");
  if (rc != DIMQ_OK) return rc;
  const PdOperands o{wd, rs, xh ? xh : static_cast<const uint16_t*>(p.x), xh ? p.K : p.ldx, flags, x_dtype, bits};
  switch (pd_pick_tile(p.M, p.N, p.K)) {
    case 1: return launch_pd_modes<1>(p, mode, o, s);
    case 2: return launch_pd_modes<2>(p, mode, o, s);
    case 3: return launch_pd_modes<3>(p, mode, o, s);
    case 4: return launch_pd_modes<4>(p, mode, o, s);
    default: return launch_pd_modes<0>(p, mode, o, s);
  }
}

}  // namespace dimq
