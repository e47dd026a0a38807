// Shared device/host helpers of libdimq_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/dimq_hip.h"

namespace dimq {

// ---------------------------------------------------------------- errors
// Thread-local message store (capi.hip).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define DIMQ_CHECK(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return ::dimq::set_error(DIMQ_ERR_INVALID, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// CUs of the current device, cached per device (conv.hip).
int device_cus();

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

inline int dtype_size(int dt) {
  switch (dt) {
    case DIMQ_F32: return 4;
    case DIMQ_F16: return 2;
    case DIMQ_BF16: return 2;
    case DIMQ_F64: return 8;
    case DIMQ_U8: return 1;
  }
  return 0;
}

inline bool is_float_dtype(int dt) {
  return dt == DIMQ_F32 || dt == DIMQ_F16 || dt == DIMQ_BF16 || dt == DIMQ_F64;
}

// ---------------------------------------------------------------- device scalars
// Raw 16-bit storage types; conversions are explicit.
struct f16raw { uint16_t v; };
struct bf16raw { uint16_t v; };

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
  return __uint_as_float(b << 16);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
  return (float)h;
}

// fp32 -> fp16 bits, round to nearest even.
__device__ __forceinline__ uint32_t float_to_f16_bits(float x) {
  _Float16 h = (_Float16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Two fp32 -> one dword of fp16 (lo in bits 0-15), round to nearest even:
// one v_cvt_pk_f16_f32.  Magnitudes >= 65520 become inf.
__device__ __forceinline__ uint32_t f16x2_rne(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, h2));
}

// Two fp32 -> one dword of bf16 (lo in bits 0-15), round to nearest even:
// one v_cvt_pk_bf16_f32, the same bits as float_to_bf16_bits for every
// non-NaN input (fp32 denormals kept); a NaN stays a NaN.
__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
}

// ---------------------------------------------------------------- fp16 range guard
// The weight-only kernels round fp32 and bf16 activations to fp16 for the
// matrix cores.  A tile's fp16 result is kept when (a) some activation of the
// tile has magnitude >= 2^-7 (fp16 exponent field >= 8: bit 13 or 14 of a
// half set), so fp16's subnormal step 2^-24 is at most 2^-17 of the tile's
// largest value, and (b) every accumulator is finite (an activation beyond
// the fp16 range rounds to inf, so its outputs come out inf or NaN).
// Otherwise the work-group recomputes the tile in fp32 (exact_tile,
// gemm_kernel.h).  For (a) threads OR the fp16 dwords they produce into a
// tracker: the generic kernels over every k step, the pipelined tile kernels
// over their first k stage only (their main loops are VALU-bound), with a
// scan of the tile's rows when that stage shows no large value.  fp16
// activations, and the integer codes of the W4A4 path, are exact in fp16 and
// are not tracked.
constexpr uint32_t kRangeBigBits = 0x60006000u;

template <int XT, bool A4 = false>
constexpr bool range_guarded() {
  return !A4 && (XT == DIMQ_F32 || XT == DIMQ_BF16);
}

// Work-group-uniform verdict; every thread of the work-group must call it.
__device__ __forceinline__ bool tile_needs_exact(uint32_t trk, bool finite) {
  const int big = __syncthreads_or((trk & kRangeBigBits) != 0u);
  const int bad = __syncthreads_or(!finite);
  return !big || bad;
}

// trk | every dword of o (fp16 pairs).
__device__ __forceinline__ uint32_t range_track(uint32_t trk, const uint32_t (&o)[8]) {
  return trk | ((o[0] | o[1]) | (o[2] | o[3])) | ((o[4] | o[5]) | (o[6] | o[7]));
}

// Wave-level halves of the verdict, for kernels whose waves own disjoint
// outputs: whether any lane of the wave saw a large activation, and whether
// every lane's accumulators are finite (both wave-uniform).
__device__ __forceinline__ bool wave_any(bool v) { return __ballot(v) != 0; }


// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t float_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Work-group barrier that orders LDS accesses only.  __syncthreads() is a
// work-group release/acquire over all memory, so it also waits for every
// global load still in flight; kernels that keep a stream of loads in flight
// across a barrier (prefetch) use this one.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Load element i of a float tensor of runtime dtype as fp32.
__device__ __forceinline__ float load_as_float(const void* p, int dt, int64_t i) {
  switch (dt) {
    case DIMQ_F32: return reinterpret_cast<const float*>(p)[i];
    case DIMQ_F16: return f16_bits_to_float(reinterpret_cast<const uint16_t*>(p)[i]);
    case DIMQ_BF16: return bf16_bits_to_float(reinterpret_cast<const uint16_t*>(p)[i]);
    case DIMQ_F64: return (float)reinterpret_cast<const double*>(p)[i];
  }
  return 0.0f;
}

// Entries [0, E) of one codebook row (size >= 1 entries) as fp32, 0 past
// `size`.  The dtype is switched on once, and entries past `size` re-load the
// last one and are zeroed by a select, so the E loads go out back to back with
// no branch between them (a branch around each load makes the compiler wait
// for every load before the next one).
template <int E>
__device__ __forceinline__ void load_cb_row(const void* cb, int dt, int64_t row, int size, float (&v)[E]) {
  const int64_t base = row * size;
  int idx[E];
#pragma unroll
  for (int j = 0; j < E; ++j) idx[j] = j < size ? j : size - 1;
  if (dt == DIMQ_F32) {
    const float* p = reinterpret_cast<const float*>(cb) + base;
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = p[idx[j]];
  } else if (dt == DIMQ_F16 || dt == DIMQ_BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(cb) + base;
    uint32_t h[E];
#pragma unroll
    for (int j = 0; j < E; ++j) h[j] = p[idx[j]];
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = dt == DIMQ_F16 ? f16_bits_to_float(h[j]) : bf16_bits_to_float(h[j]);
  } else {
    const double* p = reinterpret_cast<const double*>(cb) + base;
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = (float)p[idx[j]];
  }
#pragma unroll
  for (int j = 0; j < E; ++j) v[j] = j < size ? v[j] : 0.0f;
}

// load_cb_row in two halves for kernels that issue their other loads behind
// it: cb_row_issue only issues the row's raw loads (no conversion, so no wait
// on them), cb_row_finish converts later, once the loads issued after it are
// in flight too.
template <int E>
struct CbRaw {
  uint32_t w[2 * E];  // entry j: w[j] (32- and 16-bit dtypes), w[2j], w[2j+1] (fp64)
};

template <int E>
__device__ __forceinline__ void cb_row_issue(const void* cb, int dt, int64_t row, int size, CbRaw<E>& r) {
  const int64_t base = row * size;
#pragma unroll
  for (int j = 0; j < 2 * E; ++j) r.w[j] = 0;
  if (dt == DIMQ_F32) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(cb) + base;
#pragma unroll
    for (int j = 0; j < E; ++j) r.w[j] = p[j < size ? j : size - 1];
  } else if (dt == DIMQ_F16 || dt == DIMQ_BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(cb) + base;
#pragma unroll
    for (int j = 0; j < E; ++j) r.w[j] = p[j < size ? j : size - 1];
  } else {
    const uint2* p = reinterpret_cast<const uint2*>(cb) + base;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint2 d = p[j < size ? j : size - 1];
      r.w[2 * j] = d.x;
      r.w[2 * j + 1] = d.y;
    }
  }
}

template <int E>
__device__ __forceinline__ void cb_row_finish(const CbRaw<E>& r, int dt, int size, float (&v)[E]) {
#pragma unroll
  for (int j = 0; j < E; ++j) {
    float f;
    if (dt == DIMQ_F32) f = __uint_as_float(r.w[j]);
    else if (dt == DIMQ_F16) f = f16_bits_to_float(r.w[j]);
    else if (dt == DIMQ_BF16) f = bf16_bits_to_float(r.w[j]);
    else f = static_cast<float>(__hiloint2double(static_cast<int>(r.w[2 * j + 1]), static_cast<int>(r.w[2 * j])));
    v[j] = j < size ? f : 0.0f;
  }
}

__device__ __forceinline__ void store_from_float(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case DIMQ_F32: reinterpret_cast<float*>(p)[i] = v; break;
    case DIMQ_F16: reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)float_to_f16_bits(v); break;
    case DIMQ_BF16: reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)float_to_bf16_bits(v); break;
    case DIMQ_F64: reinterpret_cast<double*>(p)[i] = (double)v; break;
  }
}

// ---------------------------------------------------------------- fused epilogue
// Weight-only ops: y = act(v + residual[off]) with the residual in y's shape
// and memory order; a zero-initialised Epi is no residual, no activation.
struct Epi {
  const void* res;
  int res_dt;
  int act;      // enum dimq_activation
  int res_vec;  // residual 16-byte aligned: vector loads where y's stores are
  // next layer's activation quantization (quant != 0): the value becomes the
  // fp16 integer q - qzp, q = clamp(rint(v / qs) + qzp, 0, 15), stored into
  // an fp16 y -- the input form of the W4A4 kernels
  float qs = 1.0f;
  int qzp = 0;
  int quant = 0;
};

// GELU(v) = 0.5 v (1 + erf(v / sqrt 2)) with erf from Abramowitz & Stegun
// 7.1.26 (|error| <= 1.5e-7): branch-free and short, so it can sit in every
// unrolled store of an epilogue without blowing up the kernel's code.
__device__ __forceinline__ float gelu_erf(float v) {
  const float z = v * 0.70710678118654752f;
  const float a = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
  const float poly = t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  const float erf_a = 1.0f - poly * __expf(-a * a);
  return 0.5f * v * (1.0f + copysignf(erf_a, z));
}

__device__ __forceinline__ float act_apply(float v, int act) {
  if (act == DIMQ_ACT_RELU) return v < 0.0f ? 0.0f : v;  // NaN passes, as torch.relu
  if (act == DIMQ_ACT_GELU) return gelu_erf(v);
  return v;
}

__device__ __forceinline__ int quantize_u4(float x, float s, int zp);

__device__ __forceinline__ float epi_quant(const Epi& e, float v) {
  return (float)(quantize_u4(v, e.qs, e.qzp) - e.qzp);
}

// N values -> their codes q - zp (as quantize_u4), with one near-tie test for
// the whole group: t = v * RN(1/s) rounded and clamped with v_med3; a lane
// with a value within 2^-15 of a tie, a NaN / inf, or a scale whose
// reciprocal is subnormal redoes its values with quantize_u4.
// A power-of-two scale (with a normal reciprocal) needs no test: v * RN(1/s)
// is then v / s exactly (or both overflow alike, or both are below 1/2), so
// its rint is the IEEE quotient's code, ties included; a NaN gives code zp.
template <int N>
__device__ __forceinline__ void u4_codes(float (&v)[N], float s, int zp) {
  const float rcp = 1.0f / s;
  const float lo = (float)(-zp), hi = (float)(15 - zp);
  const uint32_t sb = __float_as_uint(s);
  if ((sb & 0x007fffffu) == 0u && (sb & 0x7f800000u) != 0u && fabsf(rcp) >= 0x1p-126f) {  // uniform
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float t = v[i] * rcp;
      v[i] = t == t ? __builtin_amdgcn_fmed3f(__builtin_rintf(t), lo, hi) : 0.0f;
    }
    return;
  }
  bool exact = !(fabsf(rcp) >= 0x1p-126f);
  float c[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float t = v[i] * rcp;
    const float r = __builtin_rintf(t);
    exact |= !(fabsf(fabsf(t - r) - 0.5f) > 0x1p-15f);  // near a tie, or NaN / inf
    c[i] = __builtin_amdgcn_fmed3f(r, lo, hi);
  }
  if (__builtin_expect(exact, 0)) {
#pragma unroll
    for (int i = 0; i < N; ++i) c[i] = (float)(quantize_u4(v[i], s, zp) - zp);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = c[i];
}

// Groups of 8 activations per thread in the W4A4 quantization launches.
constexpr int kQa4Groups = 4;

// The W4A4 input form (fp16 integers q - zp, u4_codes) of U groups of 8
// activations: group u of the calling thread holds elements 8 (g0 + u gstride)
// .. + 7.  Every full group's load is issued before the first is converted,
// so a thread has U 16-byte (fp16 / bf16) or 32-byte (fp32) loads in flight;
// each full group leaves as one 16-byte store, a partial last group element
// by element.  VEC: x is 16-byte aligned.
template <int XT, bool VEC, int U>
__device__ __forceinline__ void quantize_a4_f16_groups(const void* __restrict__ x, int64_t n, float s, int zp,
                                                       uint16_t* __restrict__ out, int64_t g0, int64_t gstride) {
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t base = (g0 + u * gstride) * 8;
    if (base + 8 > n) continue;
    if constexpr (VEC && XT == DIMQ_F32) {
      const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base)[0];
      const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base)[1];
      v[u][0] = a.x; v[u][1] = a.y; v[u][2] = a.z; v[u][3] = a.w;
      v[u][4] = b.x; v[u][5] = b.y; v[u][6] = b.z; v[u][7] = b.w;
    } else if constexpr (VEC && (XT == DIMQ_F16 || XT == DIMQ_BF16)) {
      const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[u][2 * j] = XT == DIMQ_F16 ? f16_bits_to_float(w[j] & 0xffffu) : bf16_bits_to_float(w[j] & 0xffffu);
        v[u][2 * j + 1] = XT == DIMQ_F16 ? f16_bits_to_float(w[j] >> 16) : bf16_bits_to_float(w[j] >> 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = load_as_float(x, XT, base + j);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t base = (g0 + u * gstride) * 8;
    if (base + 8 <= n) {
      u4_codes<8>(v[u], s, zp);
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = f16x2_rne(v[u][2 * j], v[u][2 * j + 1]);
      *reinterpret_cast<uint4*>(out + base) = make_uint4(h[0], h[1], h[2], h[3]);
    } else {
      for (int64_t i = base; i < n; ++i)
        out[i] = (uint16_t)float_to_f16_bits((float)(quantize_u4(load_as_float(x, XT, i), s, zp) - zp));
    }
  }
}

template <int N>
__device__ __forceinline__ void epi_quant_n(const Epi& e, float (&v)[N]) {
  u4_codes<N>(v, e.qs, e.qzp);
}

__device__ __forceinline__ float epi1(const Epi& e, int64_t off, float v) {
  if (e.res) v += load_as_float(e.res, e.res_dt, off);
  v = act_apply(v, e.act);
  return e.quant ? epi_quant(e, v) : v;
}

// Residual of N (a multiple of 4) consecutive outputs.  For 16-bit residuals
// on the vector path (the model case) the hot epilogues load them with
// res_issue ahead of their stores -- a load placed after an earlier store of
// the same tile cannot be hoisted over it, since the residual may alias y --
// and fold them in with epi_apply; other residuals are loaded at the store.
template <int N>
struct ResPairs {
  uint32_t w[N / 2];
};

__device__ __forceinline__ bool res_pairs(const Epi& e, bool vec) {
  return e.res && vec && e.res_vec && (e.res_dt == DIMQ_F16 || e.res_dt == DIMQ_BF16);
}

template <int N>
__device__ __forceinline__ void res_issue(const Epi& e, int64_t off, ResPairs<N>& r) {
#pragma unroll
  for (int q = 0; q < N / 4; ++q) {
    const uint2 t = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(e.res) + off + 4 * q);
    r.w[2 * q] = t.x;
    r.w[2 * q + 1] = t.y;
  }
}

// v += residual: from r when given and 16-bit, else loaded here.
template <int N>
__device__ __forceinline__ void res_add(const Epi& e, const ResPairs<N>* r, int64_t off, bool vec, float (&v)[N]) {
  if (res_pairs(e, vec)) {
    ResPairs<N> t;
    if (r) {
      t = *r;
    } else {
      res_issue<N>(e, off, t);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const uint32_t h = (t.w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
      v[i] += e.res_dt == DIMQ_F16 ? f16_bits_to_float(h) : bf16_bits_to_float(h);
    }
  } else if (vec && e.res_vec && e.res_dt == DIMQ_F32) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(e.res) + off + 4 * q);
      v[4 * q] += t.x; v[4 * q + 1] += t.y; v[4 * q + 2] += t.z; v[4 * q + 3] += t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += load_as_float(e.res, e.res_dt, off + i);
  }
}

// Runtime epilogue (generic kernels): residual and activation read from e.
template <int N>
__device__ __forceinline__ void epi_apply(const Epi& e, const ResPairs<N>* r, int64_t off, bool vec,
                                          float (&v)[N]) {
  if (e.res) res_add<N>(e, r, off, vec, v);
  if (e.act) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = act_apply(v[i], e.act);
  }
  if (e.quant) epi_quant_n<N>(e, v);
}

template <int N>
__device__ __forceinline__ void epiN(const Epi& e, int64_t off, float (&v)[N], bool vec) {
  epi_apply<N>(e, nullptr, off, vec, v);
}

// Compile-time epilogue modes of the fast kernels (a template parameter, so
// a kernel without epilogue carries none of its code): residual flag | act.
// Combinations a kernel is not instantiated for run on the generic kernels,
// whose epilogue is the runtime one above.
constexpr int kEpiNone = 0, kEpiRelu = 1, kEpiGelu = 2, kEpiRes = 4, kEpiResRelu = 5, kEpiQuant = 8;

inline int epi_mode(const Epi& e) { return (e.res ? kEpiRes : 0) | e.act | (e.quant ? kEpiQuant : 0); }

template <int MODE, int N>
__device__ __forceinline__ void epi_m(const Epi& e, const ResPairs<N>* r, int64_t off, bool vec, float (&v)[N]) {
  if constexpr ((MODE & kEpiRes) != 0) res_add<N>(e, r, off, vec, v);
  if constexpr ((MODE & 3) == kEpiRelu) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] < 0.0f ? 0.0f : v[i];
  } else if constexpr ((MODE & 3) == kEpiGelu) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = gelu_erf(v[i]);
  }
  if constexpr ((MODE & kEpiQuant) != 0) epi_quant_n<N>(e, v);
}

template <int MODE>
__device__ __forceinline__ float epi1_m(const Epi& e, int64_t off, float v) {
  if constexpr ((MODE & kEpiRes) != 0) v += load_as_float(e.res, e.res_dt, off);
  if constexpr ((MODE & 3) == kEpiRelu) v = v < 0.0f ? 0.0f : v;
  if constexpr ((MODE & 3) == kEpiGelu) v = gelu_erf(v);
  if constexpr ((MODE & kEpiQuant) != 0) v = epi_quant(e, v);
  return v;
}

// Epilogue of the quantized-activation W4A4 ops: activation, then (out_act_scale
// > 0) the next layer's activation quantization into an fp16 y.
inline int lut_q_epilogue(int activation, double out_act_scale, int64_t out_act_zp, int y_dtype, Epi& epi) {
  DIMQ_CHECK(activation >= DIMQ_ACT_NONE && activation <= DIMQ_ACT_GELU, "unknown activation %d", activation);
  epi = Epi{};
  epi.act = activation;
  if (out_act_scale > 0.0) {
    DIMQ_CHECK(out_act_zp >= 0 && out_act_zp <= 15, "out_act_zero_point must be in [0, 15]");
    DIMQ_CHECK(y_dtype == DIMQ_F16, "a quantized output (out_act_scale > 0) is written as fp16 codes");
    epi.quant = 1;
    epi.qs = static_cast<float>(out_act_scale);
    epi.qzp = static_cast<int>(out_act_zp);
  } else {
    DIMQ_CHECK(y_dtype == DIMQ_F32 || y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16,
               "output dtype must be fp32, fp16 or bf16");
  }
  return DIMQ_OK;
}

// u4 activation code: clamp(rint(x / s) + zp, 0, 15), IEEE divide
// (dimq_backend/reference.py:11-21); a NaN quotient gives zp, as the
// reference CUDA kernel's __float2int_rn (0 for NaN) plus zp does
// (csrc/dimq_common.cuh:17-21), and +-inf clamp to 15 / 0.
//
// The quotient is formed as t = x * RN(1/s): two roundings of 2^-24
// relative put t within 2^-17.9 of RN(x / s) whenever |x / s| <= 17, so both
// round to the same integer unless t lies within 2^-15 of a tie (then the
// IEEE quotient is taken); beyond 17 both clamp alike.  NaN, inf and a
// subnormal reciprocal also take the IEEE quotient.  The codes are those of
// the plain division; the divide runs only for the rare near-tie lanes.
__device__ __forceinline__ int quantize_u4(float x, float s, int zp) {
  const float rcp = 1.0f / s;  // uniform over a kernel: computed once
  const float t = x * rcp;
  float r = __builtin_rintf(t);
  if (!(fabsf(fabsf(t - r) - 0.5f) > 0x1p-15f) || !(fabsf(rcp) >= 0x1p-126f)) r = __builtin_rintf(x / s);
  float q = (r == r ? r : 0.0f) + (float)zp;
  q = q < 0.0f ? 0.0f : q;
  q = q > 15.0f ? 15.0f : q;
  return (int)q;
}

// v_perm_b32: byte i of the result = byte sel.byte[i] of the 8-byte value
// {hi:lo} (0..3 pick lo, 4..7 pick hi).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

constexpr int kWave = 64;

}  // namespace dimq
