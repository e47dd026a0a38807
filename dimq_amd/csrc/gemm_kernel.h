// Dequant + MFMA codebook GEMM: y[M,N] = x[M,K] . W_hat[N,K]^T (+ bias),
// W_hat[n,k] = C[n or 0][idx[n,k]], idx a b-bit LSB-first stream.
//
// Work-group = 256 threads = 4 waves; tile BM x (4*WN).  The 4 waves split the
// tile's columns: wave w owns columns [w*WN, (w+1)*WN) and all BM rows, so a
// weight is decoded by exactly one lane per work-group and B never touches LDS:
// each lane streams its row's packed chunk (4*b bytes per 128-wide k step)
// from HBM into VGPRs and decodes it with v_perm lookups into its
// codebook byte planes (decode.h).  The activation tile (BM x 128 fp16) is
// staged in LDS, double-buffered, written in the bit width's slot order, and
// read back as 16-byte MFMA A fragments (v_mfma_f32_16x16x32_f16, fp32
// accumulation).
//
// A4 (the reference's linear_lut, W4A4): the A operand is the integer
// q - zp (exact in fp16) and the 16-entry fp32 codebook enters as an fp16
// hi + lo pair (two MFMAs), so products are exact and the epilogue applies
// s * 2^-e.
#pragma once

#include "decode.h"

namespace dimq {

constexpr int kKM = 128;         // k per pipeline step
constexpr int kAPad = 8;         // fp16 padding per LDS row (bank spread)
constexpr int kLDA = kKM + kAPad;

struct GemmArgs {
  const void* x;
  int64_t M, K, ldx;
  const uint8_t* w;
  int64_t N;
  const void* cb;
  int cb_dt;
  int64_t cb_rows;
  int cb_size;
  const void* bias;
  int bias_dt;
  void* y;
  int y_dt;
  int64_t ldy;
  float act_scale;
  int act_zp;
  int fast_b;  // K % 32 == 0 and packed stream 16-byte aligned
  int vec_a;   // x rows allow 16-element vector loads
  // implicit-GEMM convolution (conv != 0): M = B*OH*OW, N = OC/groups per
  // group (blockIdx.z), K = ICg*KH*KW in conv_kcrs order (ci, kh, kw).
  int conv;
  int x_layout, y_layout;  // DIMQ_NCHW / DIMQ_NHWC
  int64_t cB, cC, cH, cW, cOH, cOW, cOC, cICg;
  int cKH, cKW, csh, csw, cph, cpw, cdh, cdw;
  int groups;  // grid z (1 for Linear)
  Epi epi;     // fused residual / activation (weight-only ops)
  // factor on every accumulator before bias/epilogue (weight-only kernels):
  // the activation scale of a W4A4 call whose activations were pre-quantized
  // to the exact fp16 integers a - zp
  float acc_scale = 1.0f;
};

// Output element offset of (row m, global column n).
__device__ __forceinline__ int64_t out_offset(const GemmArgs& p, int64_t m, int64_t n) {
  if (!p.conv) return m * p.ldy + n;
  if (p.y_layout == DIMQ_NHWC) return m * p.cOC + n;
  const int64_t hw = p.cOH * p.cOW;
  const int64_t b = m / hw;
  const int64_t r = m - b * hw;
  return (b * p.cOC + n) * hw + r;
}

// im2col gather of 16 consecutive k (conv_kcrs order) for output pixel m.
__device__ __forceinline__ void gather16_conv(const GemmArgs& p, int xt, int64_t m, int64_t k0, int64_t cbase,
                                              float v[16]) {
  const int64_t hw = p.cOH * p.cOW;
  const int64_t b = m / hw;
  const int64_t r = m - b * hw;
  const int oh = static_cast<int>(r / p.cOW);
  const int ow = static_cast<int>(r - (int64_t)oh * p.cOW);
  const int khw = p.cKH * p.cKW;
  int ci = static_cast<int>(k0 / khw);
  int t = static_cast<int>(k0 - (int64_t)ci * khw);
  int kh = t / p.cKW;
  int kw = t - kh * p.cKW;
  const int64_t K = p.K;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float val = 0.0f;
    if (k0 + j < K) {
      const int ih = oh * p.csh - p.cph + kh * p.cdh;
      const int iw = ow * p.csw - p.cpw + kw * p.cdw;
      if (ih >= 0 && ih < p.cH && iw >= 0 && iw < p.cW) {
        const int64_t c = cbase + ci;
        const int64_t off = (p.x_layout == DIMQ_NHWC) ? ((b * p.cH + ih) * p.cW + iw) * p.cC + c
                                                      : ((b * p.cC + c) * p.cH + ih) * p.cW + iw;
        val = load_as_float(p.x, xt, off);
      }
    }
    v[j] = val;
    if (++kw == p.cKW) {
      kw = 0;
      if (++kh == p.cKH) {
        kh = 0;
        ++ci;
      }
    }
  }
}

// ---- fp32 recompute of a tile outside the fp16 range (common.h, range guard) ----
// Index at bit position `bit` of the packed stream (fields LSB first).
__device__ __forceinline__ uint32_t packed_index(const uint8_t* w, int64_t bit, int bits) {
  const uint8_t* b = w + (bit >> 3);
  const int sh = static_cast<int>(bit & 7);
  uint32_t v = b[0] >> sh;
  if (sh + bits > 8) v |= (uint32_t)b[1] << (8 - sh);
  return v & ((1u << bits) - 1u);
}

// sum over k in [k0, k1) of x[m, k] * C[n][idx(n, k)] for the outputs
// m in [m0, m1), n in [n0, n1) of group z (clipped to M and N), every
// activation and centre read in its own dtype and accumulated in fp32 in k
// order; store(m, n, sum) per output.  One output per thread at a time: this
// runs only for tiles the fp16 matrix path cannot represent.
// Convolutions read the conv_kcrs stream (k = (ci, kh, kw)), or with
// tapmajor the NHWC implicit GEMM's re-packed stream (k = (kh, kw, c)).
// Thread t0 of the tstride cooperating threads takes outputs t0, t0 + tstride, ...
template <class Store>
__device__ void exact_tile(const GemmArgs& p, int xt, int bits, int64_t m0, int64_t m1, int64_t n0, int64_t n1,
                           int64_t k0, int64_t k1, int64_t z, bool tapmajor, int t0, int tstride, Store store) {
  m1 = m1 < p.M ? m1 : p.M;
  n1 = n1 < p.N ? n1 : p.N;
  k1 = k1 < p.K ? k1 : p.K;
  const int64_t nm = m1 - m0, nn = n1 - n0;
  if (nm <= 0 || nn <= 0) return;
  const int64_t cbase = z * p.cICg;
  for (int64_t o = t0; o < nm * nn; o += tstride) {
    const int64_t m = m0 + o / nn, n = n0 + o % nn;
    const int64_t row = z * p.N + n;
    const int64_t cbrow = p.cb_rows == 1 ? 0 : row;
    float acc = 0.0f;
    for (int64_t k = k0; k < k1; k += 16) {
      float v[16];
      if (p.conv && tapmajor) {
        const int64_t hw = p.cOH * p.cOW;
        const int64_t b = m / hw;
        const int r = static_cast<int>(m - b * hw);
        const int oh = r / static_cast<int>(p.cOW), ow = r - oh * static_cast<int>(p.cOW);
        for (int j = 0; j < 16; ++j) {
          v[j] = 0.0f;
          if (k + j >= k1) continue;
          const int tap = static_cast<int>((k + j) / p.cC);
          const int64_t c = k + j - tap * p.cC;
          const int kh = tap / p.cKW, kw = tap - kh * p.cKW;
          const int ih = oh * p.csh - p.cph + kh * p.cdh, iw = ow * p.csw - p.cpw + kw * p.cdw;
          if (ih >= 0 && ih < p.cH && iw >= 0 && iw < p.cW)
            v[j] = load_as_float(p.x, xt, ((b * p.cH + ih) * p.cW + iw) * p.cC + c);
        }
      } else if (p.conv) {
        gather16_conv(p, xt, m, k, cbase, v);
      } else {
        for (int j = 0; j < 16; ++j) v[j] = k + j < k1 ? load_as_float(p.x, xt, m * p.ldx + k + j) : 0.0f;
      }
      for (int j = 0; j < 16 && k + j < k1; ++j) {
        const int i = static_cast<int>(packed_index(p.w, (row * p.K + k + j) * bits, bits));
        const float c = i < p.cb_size ? load_as_float(p.cb, p.cb_dt, cbrow * p.cb_size + i) : 0.0f;
        acc = fmaf(v[j], c, acc);
      }
    }
    store(m, n, acc);
  }
}

// exact_tile over the whole k range by the work-group (or, with t0 / tstride,
// by one wave), through the kernels' epilogue.
__device__ __forceinline__ void exact_tile_out(const GemmArgs& p, int xt, int bits, int64_t m0, int64_t m1,
                                            int64_t n0, int64_t n1, int64_t z, bool tapmajor = false,
                                            int t0 = -1, int tstride = 0) {
  if (t0 < 0) {
    t0 = threadIdx.x;
    tstride = blockDim.x;
  }
  exact_tile(p, xt, bits, m0, m1, n0, n1, 0, p.K, z, tapmajor, t0, tstride, [&](int64_t m, int64_t n, float v) {
    const float b = p.bias ? load_as_float(p.bias, p.bias_dt, z * p.N + n) : 0.0f;
    const int64_t o = out_offset(p, m, z * p.N + n);
    store_from_float(p.y, p.y_dt, o, epi1(p.epi, o, v * p.acc_scale + b));
  });
}

// Every accumulator of a tile row is finite, checked on the first W entries
// of each of the n vectors given (one per row block; their column block
// holds every row of the lane).  One column per row is enough: a non-finite
// activation makes every column of its row inf or NaN (the fp16 weights are
// finite, and sums of fp16 products cannot overflow fp32).
template <int W, class V>
__device__ __forceinline__ bool finite_acc(const V* a, int n, int stride) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < n; ++i)
#pragma unroll
    for (int j = 0; j < W; ++j) ok &= __builtin_isfinite(a[i * stride][j]);
  return ok;
}

// Verdict of the range guard for kernels that track only their first k
// stage (trk): keep the fp16 tile when every accumulator is finite and an
// activation of magnitude >= 2^-7 was seen, in that stage or, failing that,
// by a scan of the tile's rows (Linear; a convolution's tile goes to the fp32
// recompute).  Work-group-uniform; every thread must call it.
__device__ __forceinline__ bool tile_needs_exact(const GemmArgs& p, int xt, int64_t m0, int64_t m1, uint32_t trk,
                                                 bool finite) {
  const int bad = __syncthreads_or(!finite);
  const int big = __syncthreads_or((trk & kRangeBigBits) != 0u);
  if (bad) return true;
  if (big) return false;
  if (p.conv) return true;
  m1 = m1 < p.M ? m1 : p.M;
  bool seen = false;
  const int64_t n = (m1 > m0 ? m1 - m0 : 0) * p.K;
  for (int64_t i = threadIdx.x; i < n && !seen; i += blockDim.x) {
    const int64_t m = m0 + i / p.K;
    seen = fabsf(load_as_float(p.x, xt, m * p.ldx + (i - (m - m0) * p.K))) >= 0x1p-7f;
  }
  return !__syncthreads_or(seen);
}

// ---- activation tile loader --------------------------------------------------
template <int XT>
__device__ __forceinline__ void load16_as_float(const void* x, int64_t off, bool vec, int64_t kvalid, float v[16]) {
  if constexpr (XT == DIMQ_F32) {
    const float* p = reinterpret_cast<const float*>(x) + off;
    if (vec) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 t = reinterpret_cast<const float4*>(p)[q];
        v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = (j < kvalid) ? p[j] : 0.0f;
    }
  } else if constexpr (XT == DIMQ_F64) {
    // the reference op accepts double activations and quantizes x.float()
    const double* p = reinterpret_cast<const double*>(x) + off;
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = (j < kvalid) ? (float)p[j] : 0.0f;
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(x) + off;
    uint32_t r[8];
    if (vec) {
      const uint4 a = reinterpret_cast<const uint4*>(p)[0];
      const uint4 b = reinterpret_cast<const uint4*>(p)[1];
      r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w; r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
    } else {
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint32_t lo = (2 * d < kvalid) ? p[2 * d] : 0u;
        const uint32_t hi = (2 * d + 1 < kvalid) ? p[2 * d + 1] : 0u;
        r[d] = lo | (hi << 16);
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t bits = (r[j >> 1] >> (16 * (j & 1))) & 0xffffu;
      v[j] = (XT == DIMQ_F16) ? f16_bits_to_float(bits) : bf16_bits_to_float(bits);
    }
  }
}

// 16 activations starting at (row gm, column k0) -> 8 dwords of fp16 pairs in
// the slot order of BITS.
// The fp16 dwords are ORed into trk (fp32/bf16 weight-only: range guard).
template <int BITS, int XT, bool A4>
__device__ __forceinline__ void load_a_group(const GemmArgs& p, int64_t gm, int64_t k0, int64_t cbase,
                                             uint32_t out[8], uint32_t& trk) {
  float v[16];
  if (p.conv) {
    if (gm < p.M && k0 < p.K) {
      gather16_conv(p, XT, gm, k0, cbase, v);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = 0.0f;
    }
  } else if (gm < p.M && k0 < p.K) {
    const int64_t kvalid = p.K - k0;
    const bool vec = p.vec_a && kvalid >= 16;
    load16_as_float<XT>(p.x, gm * p.ldx + k0, vec, kvalid, v);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = 0.0f;
  }
  if constexpr (A4) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool live = (gm < p.M) && (k0 + j < p.K);
      v[j] = live ? (float)(quantize_u4(v[j], p.act_scale, p.act_zp) - p.act_zp) : 0.0f;
    }
  }
  // one round-to-nearest v_cvt_pk_f16_f32 per pair of slots
#pragma unroll
  for (int d = 0; d < 8; ++d) out[d] = f16x2_rne(v[kperm16(BITS, 2 * d)], v[kperm16(BITS, 2 * d + 1)]);
  if constexpr (range_guarded<XT, A4>()) {
#pragma unroll
    for (int d = 0; d < 8; ++d) trk |= out[d];
  }
}

// ---- tile scheduling -------------------------------------------------------------
// The grid is 1-D over Mt x Nt tiles (n fastest).  Work-groups are dispatched
// round-robin over the 8 XCDs (each with its own L2), so work-group i runs on
// XCD i % 8.  The remap hands every XCD a contiguous run of tiles, i.e. whole
// rows of N-tiles over a few M-tiles: that XCD then reads only its own slab
// of x and the packed weight, both of which stay resident in its L2.
__device__ __forceinline__ void tile_coords(int64_t n_tiles, int64_t& mt, int64_t& nt) {
  constexpr int kXCD = 8;
  const int64_t T = gridDim.x;
  int64_t pid = blockIdx.x;
  const int64_t per = T / kXCD;
  if (pid < per * kXCD) pid = (pid % kXCD) * per + pid / kXCD;
  mt = pid / n_tiles;
  nt = pid - mt * n_tiles;
}

// ---- packed weight chunk loader ---------------------------------------------
// 32 indices of row n starting at column k (k % 32 == 0) -> BITS dwords laid
// out as if the chunk started on a byte boundary.  Columns >= K read as 0.
template <int BITS>
__device__ __forceinline__ void load_b_chunk(const GemmArgs& p, int64_t nl, int64_t n, int64_t k, uint32_t c[BITS]) {
#pragma unroll
  for (int w = 0; w < BITS; ++w) c[w] = 0u;
  if (nl >= p.N || k >= p.K) return;
  if (p.fast_b) {
    const uint8_t* src = p.w + (((n * p.K + k) * BITS) >> 3);
    if constexpr (BITS == 2) {
      const uint2 t = *reinterpret_cast<const uint2*>(src);
      c[0] = t.x; c[1] = t.y;
    } else if constexpr (BITS == 3) {
      c[0] = reinterpret_cast<const uint32_t*>(src)[0];
      c[1] = reinterpret_cast<const uint32_t*>(src)[1];
      c[2] = reinterpret_cast<const uint32_t*>(src)[2];
    } else if constexpr (BITS == 4) {
      const uint4 t = *reinterpret_cast<const uint4*>(src);
      c[0] = t.x; c[1] = t.y; c[2] = t.z; c[3] = t.w;
    } else {
      const uint4 t0 = reinterpret_cast<const uint4*>(src)[0];
      const uint4 t1 = reinterpret_cast<const uint4*>(src)[1];
      c[0] = t0.x; c[1] = t0.y; c[2] = t0.z; c[3] = t0.w;
      c[4] = t1.x; c[5] = t1.y; c[6] = t1.z; c[7] = t1.w;
    }
  } else {
    // generic: rows are not byte aligned in the stream (K*b % 8 != 0) or K % 32 != 0
    const int64_t kv = p.K - k;
    for (int i = 0; i < 32; ++i) {
      if (i >= kv) break;
      const int64_t bit = (n * p.K + k + i) * BITS;
      const uint8_t* b = p.w + (bit >> 3);
      const int sh = static_cast<int>(bit & 7);
      uint32_t v = b[0] >> sh;
      if (sh + BITS > 8) v |= (uint32_t)b[1] << (8 - sh);
      v &= (1u << BITS) - 1u;
      const int ob = i * BITS;
      c[ob >> 5] |= v << (ob & 31);
      if ((ob & 31) + BITS > 32) c[(ob >> 5) + 1] |= v >> (32 - (ob & 31));
    }
  }
}

// ---- codebook setup ------------------------------------------------------------
// Loads row `row` (cb_size entries, any float dtype), scales by 2^e, rounds to
// fp16 (A4: hi + lo pair).  Returns e.
template <int BITS, bool A4>
__device__ __forceinline__ int load_codebook_row(const GemmArgs& p, int64_t row, bool valid, CodebookRegs<BITS>& hi,
                                                 CodebookRegs<BITS>& lo) {
  constexpr int E = 1 << BITS;
  float c[E];
  // rows past N read row 0 (always present) and are zeroed: no branch
  // between the E loads (load_cb_row)
  load_cb_row<E>(p.cb, p.cb_dt, valid ? row : 0, p.cb_size, c);
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    c[j] = valid ? c[j] : 0.0f;
    mx = fmaxf(mx, fabsf(c[j]));
  }
  const int e = cb_exponent(mx);
  uint32_t h16[E], l16[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float cs = ldexpf(c[j], e);
    h16[j] = float_to_f16_bits(cs);
    if constexpr (A4) l16[j] = float_to_f16_bits(cs - f16_bits_to_float(h16[j]));
  }
  set_planes<BITS>(hi, h16);
  if constexpr (A4) set_planes<BITS>(lo, l16);
  return e;
}

template <int BITS, int BM, int WN, int XT, bool A4>
__global__ __launch_bounds__(256) void gemm_cb_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  constexpr int MB = BM / 16;
  constexpr int NB = WN / 16;
  constexpr int NCB = A4 ? 2 : 1;
  constexpr int A_TASKS = BM * (kKM / 16);
  constexpr int A_PER_T = (A_TASKS + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLDA];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  int64_t mt, nt;
  tile_coords((p.N + 4 * WN - 1) / (4 * WN), mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t nw0 = nt * (4 * WN) + wave * WN;
  const int64_t nz = static_cast<int64_t>(blockIdx.z) * p.N;      // first weight row of this group
  const int64_t cbase = static_cast<int64_t>(blockIdx.z) * p.cICg;  // first input channel of this group

  constexpr int E = 1 << BITS;
  float* cbs = reinterpret_cast<float*>(&As[1][0]);
  {
    const int64_t n0 = nt * (4 * WN);
    if constexpr (4 * WN * E * 4 <= BM * kLDA * 2) {
      stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, nz + n0, 4 * WN, nz + p.N, cbs, tid, 256);
    }
  }
  __syncthreads();
  CodebookRegs<BITS> cb[NB][NCB];
  float colscale[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = nw0 + nb * 16 + col;
    int e;
    if constexpr (4 * WN * E * 4 <= BM * kLDA * 2) {
      const int rl = (p.cb_rows == 1) ? 0 : wave * WN + nb * 16 + col;
      e = planes_from_lds<BITS, A4>(cbs + rl * E, cb[nb][0], cb[nb][NCB - 1]);
    } else {
      const int64_t row = (p.cb_rows == 1) ? 0 : nz + n;
      e = load_codebook_row<BITS, A4>(p, row, n < p.N, cb[nb][0], cb[nb][NCB - 1]);
    }
    colscale[nb] = ldexpf(A4 ? p.act_scale : p.acc_scale, -e);
  }
  __syncthreads();

  floatx4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t nk = (p.K + kKM - 1) / kKM;
  uint32_t a_st[A_PER_T][8];
  uint32_t bc[NB][BITS], bn[NB][BITS];
  uint32_t trk = 0;

  auto load_a = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int task = tid + 256 * i;
      if (A_TASKS % 256 == 0 || task < A_TASKS) {
        const int m = task >> 3, kg = task & 7;
        load_a_group<BITS, XT, A4>(p, m0 + m, kt * kKM + 16 * kg, cbase, a_st[i], trk);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int task = tid + 256 * i;
      if (A_TASKS % 256 == 0 || task < A_TASKS) {
        const int m = task >> 3, kg = task & 7;
        uint4* dst = reinterpret_cast<uint4*>(&As[buf][m * kLDA + 16 * kg]);
        dst[0] = make_uint4(a_st[i][0], a_st[i][1], a_st[i][2], a_st[i][3]);
        dst[1] = make_uint4(a_st[i][4], a_st[i][5], a_st[i][6], a_st[i][7]);
      }
    }
  };
  auto load_b = [&](int64_t kt, uint32_t (&dst)[NB][BITS]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      load_b_chunk<BITS>(p, nw0 + nb * 16 + col, nz + nw0 + nb * 16 + col, kt * kKM + 32 * g, dst[nb]);
  };

  load_a(0);
  store_a(0);
  load_b(0, bc);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    // the next tile's loads are issued unconditionally (the last trip
    // re-reads its own tile into the unused buffer): no branch around them
    const int64_t kn = kt + 1 < nk ? kt + 1 : kt;
    load_a(kn);
    load_b(kn, bn);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 bf[NB][NCB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int c = 0; c < NCB; ++c) bf[nb][c] = decode_sub<BITS>(bc[nb], s, cb[nb][c]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const half8 af = *reinterpret_cast<const half8*>(&As[buf][(mb * 16 + col) * kLDA + 32 * g + 8 * s]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int c = 0; c < NCB; ++c) acc[mb][nb] = mfma16x16x32(af, bf[nb][c], acc[mb][nb]);
      }
    }
    store_a(buf ^ 1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int w = 0; w < BITS; ++w) bc[nb][w] = bn[nb][w];
    __syncthreads();
  }

  if constexpr (range_guarded<XT, A4>()) {
    if (tile_needs_exact(trk, finite_acc<4>(&acc[0][0], MB, NB))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, nt * (4 * WN), (nt + 1) * (4 * WN), blockIdx.z);
      return;
    }
  }

  // epilogue: lane holds rows 4g..4g+3 of column `col` of each 16x16 block
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = nw0 + nb * 16 + col;
    if (n >= p.N) continue;
    const float b = p.bias ? load_as_float(p.bias, p.bias_dt, nz + n) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + mb * 16 + 4 * g + i;
        if (m < p.M) {
          const int64_t o = out_offset(p, m, nz + n);
          store_from_float(p.y, p.y_dt, o, epi1(p.epi, o, acc[mb][nb][i] * colscale[nb] + b));
        }
      }
    }
  }
}

// 8-bit codebooks (256 entries) are too large for registers: the work-group's
// 4*WN rows are staged in LDS as fp16 and looked up with ds_read_u16.
template <int BM, int WN, int XT>
__global__ __launch_bounds__(256) void gemm_cb8_kernel(const GemmArgs p) {
  constexpr int BITS = 8;
  constexpr int MB = BM / 16;
  constexpr int NB = WN / 16;
  constexpr int ROWS = 4 * WN;
  constexpr int A_TASKS = BM * (kKM / 16);
  constexpr int A_PER_T = (A_TASKS + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLDA];
  __shared__ uint16_t cbs[ROWS * 256];
  __shared__ float rscale[ROWS];
  __shared__ float rmax[ROWS][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  int64_t mt, nt;
  tile_coords((p.N + ROWS - 1) / ROWS, mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t n0 = nt * ROWS;
  const int64_t nw0 = n0 + wave * WN;
  const int64_t nz = static_cast<int64_t>(blockIdx.z) * p.N;
  const int64_t cbase = static_cast<int64_t>(blockIdx.z) * p.cICg;

  floatx4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t nk = (p.K + kKM - 1) / kKM;
  uint32_t a_st[A_PER_T][8];
  uint32_t bc[NB][BITS], bn[NB][BITS];
  uint32_t trk = 0;
  auto load_a = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int task = tid + 256 * i;
      if (A_TASKS % 256 == 0 || task < A_TASKS) {
        const int m = task >> 3, kg = task & 7;
        load_a_group<BITS, XT, false>(p, m0 + m, kt * kKM + 16 * kg, cbase, a_st[i], trk);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int task = tid + 256 * i;
      if (A_TASKS % 256 == 0 || task < A_TASKS) {
        const int m = task >> 3, kg = task & 7;
        uint4* dst = reinterpret_cast<uint4*>(&As[buf][m * kLDA + 16 * kg]);
        dst[0] = make_uint4(a_st[i][0], a_st[i][1], a_st[i][2], a_st[i][3]);
        dst[1] = make_uint4(a_st[i][4], a_st[i][5], a_st[i][6], a_st[i][7]);
      }
    }
  };
  auto load_b = [&](int64_t kt, uint32_t (&dst)[NB][BITS]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      load_b_chunk<BITS>(p, nw0 + nb * 16 + col, nz + nw0 + nb * 16 + col, kt * kKM + 32 * g, dst[nb]);
  };

  // the first k tile is requested before the codebook rows, so both are in
  // flight together
  load_a(0);
  load_b(0, bc);

  // codebook rows -> LDS (fp16, scaled by a per-row power of two).  One
  // pass: thread (row r = tid / 4, quarter part) loads its 64 entries back to
  // back into registers, the row maxima meet in LDS, and the scaled entries go
  // out from the registers.  The dtype is switched on once and rows past N /
  // entries past cb_size re-load a valid entry and are zeroed by a select, so
  // no branch separates the 64 loads (a branch around each load makes the
  // compiler wait for every load before the next: 64 round trips in a row).
  static_assert(ROWS == 64, "one codebook row per 4 threads");
  {
    const int r = tid >> 2, part = tid & 3;
    const int64_t n = n0 + r;
    const bool live = n < p.N;
    const int64_t base = ((p.cb_rows == 1) ? 0 : nz + (live ? n : p.N - 1)) * p.cb_size;
    const int last = p.cb_size - 1;
    float cv[64];
    if (p.cb_dt == DIMQ_F32) {
      const float* q = reinterpret_cast<const float*>(p.cb) + base;
#pragma unroll
      for (int i = 0; i < 64; ++i) cv[i] = q[min(part + 4 * i, last)];
    } else if (p.cb_dt == DIMQ_F16 || p.cb_dt == DIMQ_BF16) {
      const uint16_t* q = reinterpret_cast<const uint16_t*>(p.cb) + base;
      uint32_t h[64];
#pragma unroll
      for (int i = 0; i < 64; ++i) h[i] = q[min(part + 4 * i, last)];
      if (p.cb_dt == DIMQ_F16) {
#pragma unroll
        for (int i = 0; i < 64; ++i) cv[i] = f16_bits_to_float(h[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 64; ++i) cv[i] = bf16_bits_to_float(h[i]);
      }
    } else {
      const double* q = reinterpret_cast<const double*>(p.cb) + base;
#pragma unroll
      for (int i = 0; i < 64; ++i) cv[i] = static_cast<float>(q[min(part + 4 * i, last)]);
    }
#pragma unroll
    for (int i = 0; i < 64; ++i) cv[i] = (live && part + 4 * i <= last) ? cv[i] : 0.0f;
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i) mx = fmaxf(mx, fabsf(cv[i]));
    rmax[r][part] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(rmax[r][0], rmax[r][1]), fmaxf(rmax[r][2], rmax[r][3]));
    const int e = cb_exponent(mx);
#pragma unroll
    for (int i = 0; i < 64; ++i) cbs[r * 256 + part + 4 * i] = (uint16_t)float_to_f16_bits(ldexpf(cv[i], e));
    if (part == 0) rscale[r] = ldexpf(p.acc_scale, -e);
  }
  store_a(0);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    // the next tile's loads are issued unconditionally (the last trip
    // re-reads its own tile into the unused buffer): no branch around them
    const int64_t kn = kt + 1 < nk ? kt + 1 : kt;
    load_a(kn);
    load_b(kn, bn);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 bf[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint16_t* rowp = &cbs[(wave * WN + nb * 16 + col) * 256];
        u32x4 r;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t w = bc[nb][2 * s + (d >> 1)];
          const int sh = 16 * (d & 1);
          r[d] = (uint32_t)rowp[(w >> sh) & 0xffu] | ((uint32_t)rowp[(w >> (sh + 8)) & 0xffu] << 16);
        }
        bf[nb] = __builtin_bit_cast(half8, r);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const half8 af = *reinterpret_cast<const half8*>(&As[buf][(mb * 16 + col) * kLDA + 32 * g + 8 * s]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16x16x32(af, bf[nb], acc[mb][nb]);
      }
    }
    store_a(buf ^ 1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int w = 0; w < BITS; ++w) bc[nb][w] = bn[nb][w];
    __syncthreads();
  }

  if constexpr (range_guarded<XT>()) {
    if (tile_needs_exact(trk, finite_acc<4>(&acc[0][0], MB, NB))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, n0, n0 + ROWS, blockIdx.z);
      return;
    }
  }

#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = nw0 + nb * 16 + col;
    if (n >= p.N) continue;
    const float sc = rscale[wave * WN + nb * 16 + col];
    const float b = p.bias ? load_as_float(p.bias, p.bias_dt, nz + n) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + mb * 16 + 4 * g + i;
        if (m < p.M) {
          const int64_t o = out_offset(p, m, nz + n);
          store_from_float(p.y, p.y_dt, o, epi1(p.epi, o, acc[mb][nb][i] * sc + b));
        }
      }
    }
  }
}

// Small-M variant (M <= 16, decode / GEMV shapes).  A work-group of WPW waves
// owns 16 weight rows and the whole K range; wave w takes the 128-wide k steps
// kt = w, w + WPW, ...  so WPW waves per work-group (16 per CU) keep enough
// loads in flight to hide HBM latency, which is what bounds these shapes.
// The activation rows (16 lanes x 32 values per step) are read straight from
// global memory (L2-resident, shared by all work-groups), converted and put in
// slot order in registers; partial sums of the WPW waves meet in LDS.
template <int BITS, int XT, int WPW>
__global__ __launch_bounds__(WPW * 64) void gemv_cb_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  __shared__ floatx4 red[WPW][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 16 + col;
  constexpr int E = 1 << BITS;
  __shared__ float cbs[16 * E];
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, static_cast<int64_t>(blockIdx.x) * 16, 16, p.N, cbs, tid,
                    WPW * 64);
  __syncthreads();
  CodebookRegs<BITS> cb;
  const int e = planes_from_lds<BITS, false>(cbs + ((p.cb_rows == 1) ? 0 : col * E), cb, cb);
  const float colscale = ldexpf(p.acc_scale, -e);
  const int64_t nk = (p.K + kKM - 1) / kKM;
  const bool arow = col < p.M;
  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  uint32_t bc[BITS];
  uint32_t av[16];  // 32 fp16 activations in slot order
  uint32_t trk = 0;
  auto load_step = [&](int64_t kt, uint32_t (&bdst)[BITS], uint32_t (&adst)[16]) {
    load_b_chunk<BITS>(p, n, n, kt * kKM + 32 * g, bdst);
    const int64_t k0 = kt * kKM + 32 * g;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t t[8];
      load_a_group<BITS, XT, false>(p, arow ? (int64_t)col : p.M, k0 + 16 * h, 0, t, trk);
#pragma unroll
      for (int d = 0; d < 8; ++d) adst[8 * h + d] = t[d];
    }
  };
  for (int64_t kt = wave; kt < nk; kt += WPW) {
    load_step(kt, bc, av);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4 a4 = {av[4 * s], av[4 * s + 1], av[4 * s + 2], av[4 * s + 3]};
      const half8 bf = decode_sub<BITS>(bc, s, cb);
      acc = mfma16x16x32(__builtin_bit_cast(half8, a4), bf, acc);
    }
  }
  if constexpr (range_guarded<XT>()) {
    if (tile_needs_exact(trk, finite_acc<4>(&acc, 1, 1))) {
      exact_tile_out(p, XT, BITS, 0, 16, static_cast<int64_t>(blockIdx.x) * 16, static_cast<int64_t>(blockIdx.x) * 16 + 16, 0);
      return;
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    floatx4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < WPW; ++w) t += red[w][lane];
    if (n < p.N) {
      const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = 4 * g + i;
        if (m < p.M) store_from_float(p.y, p.y_dt, m * p.ldy + n, epi1(p.epi, m * p.ldy + n, t[i] * colscale + b));
      }
    }
  }
}

// ---- fast Linear kernel -------------------------------------------------------
// Same tiling as gemm_cb_kernel, for the shapes the BASELINE layers have:
// Linear, K % 128 == 0, x rows 16-byte aligned, packed stream 16-byte aligned.
// Those guarantees let the main loop be straight-line code, which is what
// lets the compiler keep loads in flight across the compute of a step:
//  * loads are raw (no conversion) into registers, issued two steps ahead for
//    the weights and one step ahead for the activations;
//  * conversion to fp16 and the LDS write ("commit") happen after the compute
//    of the current step;
//  * out-of-range rows/columns are clamped for loading and masked on store, so
//    no load sits under a branch;
//  * the k loop is unrolled twice so the two weight register sets ping-pong
//    without copies.
template <int XT>
struct RawA {
  static constexpr int kWords = (XT == DIMQ_F32) ? 16 : 8;  // 16 activations
  uint32_t w[kWords];
};

template <int XT>
__device__ __forceinline__ void issue_a16(const void* x, int64_t off, RawA<XT>& r) {
  if constexpr (XT == DIMQ_F32) {
    const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(x) + off);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = s[q];
      r.w[4 * q] = t.x; r.w[4 * q + 1] = t.y; r.w[4 * q + 2] = t.z; r.w[4 * q + 3] = t.w;
    }
  } else {
    const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4 t = s[q];
      r.w[4 * q] = t.x; r.w[4 * q + 1] = t.y; r.w[4 * q + 2] = t.z; r.w[4 * q + 3] = t.w;
    }
  }
}

// 16 raw activations -> 8 dwords of fp16 pairs in the slot order of BITS.
template <int BITS, int XT, bool A4>
__device__ __forceinline__ void convert_a16(const RawA<XT>& r, float s, int zp, uint32_t out[8]) {
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if constexpr (XT == DIMQ_F32) v[j] = __uint_as_float(r.w[j]);
    else {
      const uint32_t bits = (r.w[j >> 1] >> (16 * (j & 1))) & 0xffffu;
      v[j] = (XT == DIMQ_F16) ? f16_bits_to_float(bits) : bf16_bits_to_float(bits);
    }
    if constexpr (A4) v[j] = (float)(quantize_u4(v[j], s, zp) - zp);
  }
  // one round-to-nearest v_cvt_pk_f16_f32 per pair of slots
#pragma unroll
  for (int d = 0; d < 8; ++d) out[d] = f16x2_rne(v[kperm16(BITS, 2 * d)], v[kperm16(BITS, 2 * d + 1)]);
}

template <int BITS>
__device__ __forceinline__ void issue_b_fast(const uint8_t* w, int64_t n, int64_t K, int64_t k, uint32_t c[BITS]) {
  const uint8_t* src = w + (((n * K + k) * BITS) >> 3);
  if constexpr (BITS == 2) {
    const uint2 t = *reinterpret_cast<const uint2*>(src);
    c[0] = t.x; c[1] = t.y;
  } else if constexpr (BITS == 3) {
    c[0] = reinterpret_cast<const uint32_t*>(src)[0];
    c[1] = reinterpret_cast<const uint32_t*>(src)[1];
    c[2] = reinterpret_cast<const uint32_t*>(src)[2];
  } else {
    const uint4 t = *reinterpret_cast<const uint4*>(src);
    c[0] = t.x; c[1] = t.y; c[2] = t.z; c[3] = t.w;
  }
}

template <int BITS, int BM, int WN, int XT, bool A4>
__global__ __launch_bounds__(256) void gemm_fast_kernel(const GemmArgs p) {
  static_assert(BITS >= 2 && BITS <= 4, "register codebooks hold at most 16 entries");
  static_assert(BM >= 32, "at least one 16-wide activation group per thread");
  constexpr int MB = BM / 16;
  constexpr int NB = WN / 16;
  constexpr int NCB = A4 ? 2 : 1;
  constexpr int A_PER_T = BM * (kKM / 16) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLDA];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  int64_t mt, nt;
  tile_coords((p.N + 4 * WN - 1) / (4 * WN), mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t nw0 = nt * (4 * WN) + wave * WN;

  // codebook rows of the work-group's 4*WN columns, staged through As[1]
  // (first written by the main loop, after the barrier that ends the prologue)
  constexpr int E = 1 << BITS;
  static_assert(4 * WN * E * 4 <= BM * kLDA * 2, "codebook staging fits in one A buffer");
  float* cbs = reinterpret_cast<float*>(&As[1][0]);
  const int64_t n0 = nt * (4 * WN);
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, n0, 4 * WN, p.N, cbs, tid, 256);
  __syncthreads();
  CodebookRegs<BITS> cb[NB][NCB];
  float colscale[NB];
  int64_t brow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = nw0 + nb * 16 + col;
    brow[nb] = n < p.N ? n : p.N - 1;
    const int rl = (p.cb_rows == 1) ? 0 : wave * WN + nb * 16 + col;
    const int e = planes_from_lds<BITS, A4>(cbs + rl * E, cb[nb][0], cb[nb][NCB - 1]);
    colscale[nb] = ldexpf(A4 ? p.act_scale : p.acc_scale, -e);
  }
  // activation tasks: (row m, 16-wide group kg) per thread
  int64_t aoff[A_PER_T];
  int alds[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int task = tid + 256 * i;
    const int m = task >> 3, kg = task & 7;
    const int64_t row = (m0 + m < p.M) ? m0 + m : p.M - 1;
    aoff[i] = row * p.ldx + 16 * kg;
    alds[i] = m * kLDA + 16 * kg;
  }

  floatx4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t nk = p.K / kKM;
  // two raw activation register sets (even / odd steps) and two weight sets
  RawA<XT> ra0[A_PER_T], ra1[A_PER_T];
  uint32_t b0[NB][BITS], b1[NB][BITS];
  uint32_t trk = 0;

  auto issue_a = [&](int64_t kt, RawA<XT> (&dst)[A_PER_T]) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kKM;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) issue_a16<XT>(p.x, aoff[i] + k, dst[i]);
  };
  auto commit_a = [&](int buf, const RawA<XT> (&src)[A_PER_T], bool track = false) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      uint32_t o[8];
      convert_a16<BITS, XT, A4>(src[i], p.act_scale, p.act_zp, o);
      if (range_guarded<XT, A4>() && track) trk = range_track(trk, o);
      uint4* dst = reinterpret_cast<uint4*>(&As[buf][alds[i]]);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };
  auto issue_b = [&](int64_t kt, uint32_t (&dst)[NB][BITS]) {
    const int64_t k = (kt < nk ? kt : nk - 1) * kKM + 32 * g;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) issue_b_fast<BITS>(p.w, brow[nb], p.K, k, dst[nb]);
  };
  auto compute = [&](int buf, const uint32_t (&bq)[NB][BITS]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *reinterpret_cast<const half8*>(&As[buf][(mb * 16 + col) * kLDA + 32 * g + 8 * s]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
          const half8 bf = decode_sub<BITS>(bq[nb], s, cb[nb][c]);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16x16x32(af[mb], bf, acc[mb][nb]);
        }
      }
    }
  };

  // Pipeline: activations are committed to LDS two compute phases after
  // their loads were issued, weights are consumed two phases after theirs.
  // sched_barrier keeps the compiler from hoisting a commit (which waits for
  // its loads) into the compute phase before it.
  issue_a(0, ra0);
  issue_b(0, b0);
  issue_a(1, ra1);
  issue_b(1, b1);
  commit_a(0, ra0, true);  // the range guard looks at the first k step
  issue_a(2, ra0);
  __syncthreads();
  int64_t kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    compute(0, b0);
    __builtin_amdgcn_sched_barrier(0);
    commit_a(1, ra1);
    issue_a(kt + 3, ra1);
    issue_b(kt + 2, b0);
    __syncthreads();
    compute(1, b1);
    __builtin_amdgcn_sched_barrier(0);
    commit_a(0, ra0);
    issue_a(kt + 4, ra0);
    issue_b(kt + 3, b1);
    __syncthreads();
  }
  if (kt < nk) compute(0, b0);

  if constexpr (range_guarded<XT, A4>()) {
    if (tile_needs_exact(p, XT, m0, m0 + BM, trk, finite_acc<4>(&acc[0][0], MB, NB))) {
      exact_tile_out(p, XT, BITS, m0, m0 + BM, n0, n0 + 4 * WN, 0);
      return;
    }
  }

#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t n = nw0 + nb * 16 + col;
    if (n >= p.N) continue;
    const float b = p.bias ? load_as_float(p.bias, p.bias_dt, n) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + mb * 16 + 4 * g + i;
        if (m < p.M) store_from_float(p.y, p.y_dt, m * p.ldy + n, epi1(p.epi, m * p.ldy + n, acc[mb][nb][i] * colscale[nb] + b));
      }
    }
  }
}

// Tile shapes: (BM, WN); the work-group covers BM x 4*WN.
enum TileId {
  kTile128x64 = 0,
  kTile64x32 = 1,
  kTile16x16 = 2,
  kTileGemv = 3,
  kTileFast128x64 = 4,
  kTileFast64x32 = 5,
  kTileFast128x32 = 6,
  kTileFast64x64 = 7,
  kTileCount = 8
};

template <int BITS, int XT, bool A4>
int launch_gemm_tile(const GemmArgs& p, int tile, hipStream_t s);

// conv_halo.hip
int64_t halo_prepared_words(int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits);
int64_t halo_tile_rows(int64_t C, int64_t KH, int64_t KW, int64_t stride, int64_t OH, int64_t OW);
bool halo_weight_supported(int64_t C, int64_t KH, int64_t KW, int bits);
bool halo_eligible(int64_t C, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t dh, int64_t dw,
                   int64_t groups, int64_t OH, int64_t OW, int bits, int x_dtype, int epi_mode, int y_layout);
int launch_conv_halo(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                     const uint32_t* kw, int bits, const void* cb, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                     const void* bias, int bias_dtype, int64_t OC, int64_t KH, int64_t KW, int64_t stride,
                     int64_t ph, int64_t pw, int64_t OH, int64_t OW, void* y, int y_dtype, int y_layout,
                     const Epi& epi, hipStream_t s, float acc_scale = 1.0f);
int launch_prepare(const uint8_t* src, int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits, uint32_t* out,
                   hipStream_t s);

// conv_stem.hip
bool stem_eligible(int64_t C, int64_t OC, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t pw,
                   int64_t dh, int64_t dw, int64_t groups, int64_t OH, int64_t OW, int bits, int x_dtype,
                   int y_dtype, const void* x, const void* y, int epi_mode, const void* w, int64_t w_bytes,
                   const void* cb, int cb_dtype, int64_t cb_rows, int64_t cb_size);
int launch_conv_stem(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                     const uint8_t* w, int64_t w_bytes, int bits, const void* cb, int cb_dtype, int64_t cb_rows,
                     int64_t cb_size, const void* bias, int bias_dtype, int64_t OC, int64_t KH, int64_t KW,
                     int64_t ph, int64_t pw, int64_t OH, int64_t OW, void* y, int y_dtype, int y_layout,
                     const Epi& epi, hipStream_t s);

// quant.hip: W4A4 activations as the fp16 integers a - zp (out 16-byte aligned)
int launch_quantize_a4_f16(const void* x, int x_dtype, int64_t n, float s, int zp, uint16_t* out, hipStream_t st);
// One launch: the 4-bit halo weight layout of launch_prepare into kw and the
// activations' W4A4 form of launch_quantize_a4_f16 into q (16-byte aligned).
int launch_w4a4_conv_inputs(const uint8_t* src, int64_t OC, int64_t C, int64_t KH, int64_t KW, uint32_t* kw,
                            const void* x, int x_dtype, int64_t n, float scale, int zp, uint16_t* q, hipStream_t s);
// lut_act.hip: index x index LUT gather of the weight x activation codebook Linear
bool lut_act_supported(int64_t M, int64_t K, int bits, int64_t cb_rows, int64_t Ka);
int launch_lut_act(const uint8_t* aidx, int64_t M, int64_t K, const uint8_t* w, int bits, const void* cw, int cw_dt,
                   int64_t cb_rows, int64_t cb_size, const float* ca, int64_t Ka, int x_dtype, const void* bias,
                   int bias_dt, int64_t N, void* y, int y_dt, bool clamp, hipStream_t s);
// quant.hip: activations -> their nearest activation-codebook centre, in x's dtype
int launch_act_codebook(const void* x, int x_dtype, int64_t n, const float* centers, int K, void* out,
                        hipStream_t st);

// gemm.hip
int gemm_pick_tile(int64_t M, int64_t N, int variant);
int gemm_dispatch(const GemmArgs& p, int bits, int xt, bool a4, int tile, hipStream_t s);

}  // namespace dimq
