// Register-resident codebook decode for the matrix-core kernels.
//
// A lane that feeds the MFMA B operand owns one weight row n (its column of
// the 16x16 tile) and, per 128-wide k step, one contiguous chunk of 32 packed
// indices (4*b bytes).  The row's codebook (2^b fp16 entries, b <= 4) lives in
// VGPRs as two byte planes: L holds the low bytes of the entries, H the high
// bytes (entry e at byte e%4 of dword e/4).  v_perm_b32 then performs four
// table lookups per instruction, so decoding costs no LDS traffic:
//
//   lo = perm(L[1], L[0], D)     // D = 4 index bytes (3-bit: entries 0..7)
//   hi = perm(H[1], H[0], D)
//   V01 = perm(hi, lo, 0x05010400)   -> fp16 pair (D.b0, D.b1)
//   V23 = perm(hi, lo, 0x07030602)   -> fp16 pair (D.b2, D.b3)
//
// Each bit width extracts its index bytes with a few shifts and masks, in an
// order ("slot order") that is cheapest for it; the A operand is written to
// LDS in the same order (kperm16), so that the dot products pair up.
#pragma once

#include "common.h"

namespace dimq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Slot order: slot u of a 16-wide k group holds k offset kperm16(bits, u).
//  b=4: each packed dword holds 8 nibbles; (w & 0x0f0f0f0f) yields the even
//       k, ((w >> 4) & 0x0f0f0f0f) the odd k.
//  b=2: (w >> 2j) & 0x03030303 yields k = {j, 4+j, 8+j, 12+j}.
//  b=3, b=8: natural order.
__host__ __device__ constexpr int kperm16(int bits, int u) {
  if (bits == 4) {
    const int g = u & 8, j = u & 7;
    return g + (j < 4 ? 2 * j : 2 * (j - 4) + 1);
  }
  if (bits == 2) {
    // u = 8h + 4p + t  ->  k = 4t + 2h + p
    const int h = u >> 3, p = (u >> 2) & 1, t = u & 3;
    return 4 * t + 2 * h + p;
  }
  return u;
}

template <int BITS>
struct CodebookRegs {
  static constexpr int kPlanes = (BITS >= 2 && BITS <= 4) ? (1 << BITS) / 4 : 1;
  uint32_t L[kPlanes];
  uint32_t H[kPlanes];
};

// Fill the byte planes from 2^b fp16 bit patterns.
template <int BITS>
__device__ __forceinline__ void set_planes(CodebookRegs<BITS>& cb, const uint32_t* h16) {
#pragma unroll
  for (int q = 0; q < CodebookRegs<BITS>::kPlanes; ++q) {
    uint32_t l = 0, h = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t e = (4 * q + t < (1 << BITS)) ? h16[4 * q + t] : 0u;
      l |= (e & 0xffu) << (8 * t);
      h |= ((e >> 8) & 0xffu) << (8 * t);
    }
    cb.L[q] = l;
    cb.H[q] = h;
  }
}

// Four lookups: D holds four index bytes; returns the fp16 pairs (b0,b1), (b2,b3).
template <int BITS>
__device__ __forceinline__ void lookup4(const CodebookRegs<BITS>& cb, uint32_t D, uint32_t& v01, uint32_t& v23) {
  uint32_t lo, hi;
  if constexpr (BITS == 2) {
    lo = perm(cb.L[0], cb.L[0], D);
    hi = perm(cb.H[0], cb.H[0], D);
  } else if constexpr (BITS == 3) {
    lo = perm(cb.L[1], cb.L[0], D);
    hi = perm(cb.H[1], cb.H[0], D);
  } else {
    const uint32_t s = D & 0x07070707u;
    // byte i of sel2 = i + 4 * bit3(D.byte_i): picks the upper half table.
    // The two masks come from registers so that the and + or is one
    // v_and_or_b32 (a VOP3 instruction takes no literal on gfx9); as
    // literals they cost a v_and_b32 and a v_or_b32.
    uint32_t k4, k3210;
    asm("s_mov_b32 %0, 0x4040404" : "=s"(k4));
    asm("v_mov_b32 %0, 0x3020100" : "=v"(k3210));
    const uint32_t sel2 = ((D >> 1) & k4) | k3210;
    const uint32_t la = perm(cb.L[1], cb.L[0], s), lb = perm(cb.L[3], cb.L[2], s);
    const uint32_t ha = perm(cb.H[1], cb.H[0], s), hb = perm(cb.H[3], cb.H[2], s);
    lo = perm(lb, la, sel2);
    hi = perm(hb, ha, sel2);
  }
  v01 = perm(hi, lo, 0x05010400u);
  v23 = perm(hi, lo, 0x07030602u);
}

// 12-bit group of four 3-bit fields -> four bytes.
__device__ __forceinline__ uint32_t spread3x4(uint32_t y) {
  uint32_t t = ((y << 10) | y) & 0x003f003fu;
  return ((t << 5) | t) & 0x07070707u;
}

// Eight fields already at the bottom of G (4-bit: 8 nibbles; 2-bit: fields
// at bits 0,2 + 8i; 3-bit: 24 bits) -> B fragment (8 fp16 in slot order).
template <int BITS>
__device__ __forceinline__ half8 decode_word(uint32_t G, const CodebookRegs<BITS>& cb) {
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
  uint32_t r0, r1, r2, r3;
  lookup4<BITS>(cb, D0, r0, r1);
  lookup4<BITS>(cb, D1, r2, r3);
  const u32x4 r = {r0, r1, r2, r3};
  return __builtin_bit_cast(half8, r);
}

// Decode sub-step s (slots 8s..8s+7 of the lane's 32-index chunk c[]) into a
// B fragment (8 fp16 in slot order).  BITS in {2,3,4}.
template <int BITS>
__device__ __forceinline__ half8 decode_sub(const uint32_t (&c)[BITS], int s, const CodebookRegs<BITS>& cb) {
  uint32_t G;
  if constexpr (BITS == 4) {
    G = c[s];
  } else if constexpr (BITS == 2) {
    G = c[s >> 1] >> (4 * (s & 1));
  } else {
    if (s == 0) G = c[0];
    else if (s == 1) G = __builtin_amdgcn_alignbit(c[1], c[0], 24);
    else if (s == 2) G = __builtin_amdgcn_alignbit(c[2], c[1], 16);
    else G = c[2] >> 8;
  }
  return decode_word<BITS>(G, cb);
}

__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Power-of-two exponent e such that max|c| * 2^e lies in [2^14, 2^15):
// keeps fp16 codebook entries away from subnormals and from overflow.
__device__ __forceinline__ int cb_exponent(float maxabs) {
  if (!(maxabs > 0.0f) || !__builtin_isfinite(maxabs)) return 0;
  int ex;
  (void)frexpf(maxabs, &ex);
  int e = 15 - ex;
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  return e;
}

// Cooperative staging of codebook rows into LDS as fp32.
// Rows [row0, row0 + R) (or only row 0 for a per-layer codebook) with
// cb_size entries each are written to lds[r * E + j], entries j >= cb_size
// and rows >= n_rows as 0.  Eight independent loads per thread are issued
// before any is used, on a dtype branch taken once, so the few hundred loads
// of a work-group overlap instead of queueing one latency after another.
template <int E>
__device__ __forceinline__ void stage_codebook(const void* cb, int dt, int64_t cb_rows, int cb_size, int64_t row0,
                                               int R, int64_t n_rows, float* lds, int tid, int nthreads) {
  const int Rr = (cb_rows == 1) ? 1 : R;
  const int total = Rr * E;
  for (int base = 0; base < total; base += 8 * nthreads) {
    float v[8];
    int64_t off[8];
    bool ok[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * nthreads + tid;
      const int r = i / E, j = i % E;
      const int64_t row = (cb_rows == 1) ? 0 : row0 + r;
      ok[u] = i < total && j < cb_size && (cb_rows == 1 || row < n_rows);
      off[u] = ok[u] ? row * cb_size + j : 0;
    }
    if (dt == DIMQ_F32) {
      const float* p = reinterpret_cast<const float*>(cb);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[off[u]];
    } else if (dt == DIMQ_F16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(cb);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = f16_bits_to_float(p[off[u]]);
    } else if (dt == DIMQ_BF16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(cb);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = bf16_bits_to_float(p[off[u]]);
    } else {
      const double* p = reinterpret_cast<const double*>(cb);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = (float)p[off[u]];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * nthreads + tid;
      if (i < total) lds[i] = ok[u] ? v[u] : 0.0f;
    }
  }
}

// Byte planes (and the power-of-two exponent) of one staged codebook row.
// A4 (hi_lo): second plane set holds the fp16 residual c - fp16(c).
template <int BITS, bool HI_LO>
__device__ __forceinline__ int planes_from_lds(const float* row, CodebookRegs<BITS>& hi, CodebookRegs<BITS>& lo) {
  constexpr int E = 1 << BITS;
  float c[E];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    c[j] = row[j];
    mx = fmaxf(mx, fabsf(c[j]));
  }
  const int e = cb_exponent(mx);
  uint32_t h16[E], l16[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float cs = ldexpf(c[j], e);
    h16[j] = float_to_f16_bits(cs);
    if constexpr (HI_LO) l16[j] = float_to_f16_bits(cs - f16_bits_to_float(h16[j]));
  }
  set_planes<BITS>(hi, h16);
  if constexpr (HI_LO) set_planes<BITS>(lo, l16);
  return e;
}

}  // namespace dimq
