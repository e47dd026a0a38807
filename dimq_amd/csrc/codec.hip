// b-bit index codec (b in {2,3,4,8}), LSB-first bitstream:
// index i occupies bits [b*i, b*i+b) of a little-endian byte stream.
// For b = 4 this is the reference nibble order packed[j] = i[2j] | i[2j+1] << 4
// (dimq_backend/export.py:38-55, csrc/dimq_pack.cu:11-35).
//
// One thread owns a unit of 32 indices = 4*b packed bytes: two 16-byte loads of
// indices on one side, one 8/12/16/32-byte access of packed data on the other,
// so both directions stream HBM with wide, coalesced accesses.  The last,
// partial unit (numel % 32 indices) is handled bytewise by one thread.
#include "common.h"

namespace dimq {
namespace {

constexpr int kUnit = 32;
constexpr int kThreads = 256;

template <int BITS>
__device__ __forceinline__ void pack32(const uint32_t in[8], uint32_t o[BITS]) {
#pragma unroll
  for (int w = 0; w < BITS; ++w) o[w] = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    uint32_t v = (in[i >> 2] >> (8 * (i & 3))) & ((1u << BITS) - 1u);
    const int bit = i * BITS;
    const int w = bit >> 5;
    const int sh = bit & 31;
    o[w] |= v << sh;
    if (sh + BITS > 32) o[w + 1] |= v >> (32 - sh);
  }
}

template <int BITS>
__device__ __forceinline__ void unpack32(const uint32_t in[BITS], uint32_t o[8]) {
#pragma unroll
  for (int w = 0; w < 8; ++w) o[w] = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int bit = i * BITS;
    const int w = bit >> 5;
    const int sh = bit & 31;
    uint32_t v = in[w] >> sh;
    if (sh + BITS > 32) v |= in[w + 1] << (32 - sh);
    v &= (1u << BITS) - 1u;
    o[i >> 2] |= v << (8 * (i & 3));
  }
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void pack_kernel(const uint8_t* __restrict__ idx, int64_t n,
                                                        uint8_t* __restrict__ out, int64_t nbytes,
                                                        int64_t n_units, int vec_ok) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u < n_units) {
    uint32_t in[8];
    const uint8_t* src = idx + u * kUnit;
    if (vec_ok) {
      const uint4 a = reinterpret_cast<const uint4*>(src)[0];
      const uint4 b = reinterpret_cast<const uint4*>(src)[1];
      in[0] = a.x; in[1] = a.y; in[2] = a.z; in[3] = a.w;
      in[4] = b.x; in[5] = b.y; in[6] = b.z; in[7] = b.w;
    } else {
#pragma unroll
      for (int w = 0; w < 8; ++w)
        in[w] = src[4 * w] | (src[4 * w + 1] << 8) | (src[4 * w + 2] << 16) | ((uint32_t)src[4 * w + 3] << 24);
    }
    uint32_t o[BITS];
    pack32<BITS>(in, o);
    uint8_t* dst = out + u * (4 * BITS);
    if (vec_ok) {
      if constexpr (BITS == 2) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0], o[1]);
      } else if constexpr (BITS == 3) {
        reinterpret_cast<uint32_t*>(dst)[0] = o[0];
        reinterpret_cast<uint32_t*>(dst)[1] = o[1];
        reinterpret_cast<uint32_t*>(dst)[2] = o[2];
      } else if constexpr (BITS == 4) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
        reinterpret_cast<uint4*>(dst)[0] = make_uint4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<uint4*>(dst)[1] = make_uint4(o[4], o[5], o[6], o[7]);
      }
    } else {
#pragma unroll
      for (int b = 0; b < 4 * BITS; ++b) dst[b] = (uint8_t)(o[b >> 2] >> (8 * (b & 3)));
    }
  } else if (u == n_units) {
    // Tail: indices [u*32, n) -> bytes [u*4*BITS, nbytes); unused high bits are zero.
    const int64_t first = u * kUnit;
    const int tail = static_cast<int>(n - first);
    if (tail <= 0) return;
    uint32_t o[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) o[w] = 0;
    for (int i = 0; i < tail; ++i) {
      const uint32_t v = idx[first + i] & ((1u << BITS) - 1u);
      const int bit = i * BITS;
      const int w = bit >> 5;
      const int sh = bit & 31;
      o[w] |= v << sh;
      if (sh + BITS > 32) o[w + 1] |= v >> (32 - sh);
    }
    const int64_t b0 = u * (4 * BITS);
    for (int64_t b = b0; b < nbytes; ++b) {
      const int lb = static_cast<int>(b - b0);
      out[b] = (uint8_t)(o[lb >> 2] >> (8 * (lb & 3)));
    }
  }
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint8_t* __restrict__ packed,
                                                          uint8_t* __restrict__ out, int64_t n,
                                                          int64_t n_units, int vec_ok) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u < n_units) {
    const uint8_t* src = packed + u * (4 * BITS);
    uint32_t in[BITS];
    if (vec_ok) {
      if constexpr (BITS == 2) {
        const uint2 a = *reinterpret_cast<const uint2*>(src);
        in[0] = a.x; in[1] = a.y;
      } else if constexpr (BITS == 3) {
        in[0] = reinterpret_cast<const uint32_t*>(src)[0];
        in[1] = reinterpret_cast<const uint32_t*>(src)[1];
        in[2] = reinterpret_cast<const uint32_t*>(src)[2];
      } else if constexpr (BITS == 4) {
        const uint4 a = *reinterpret_cast<const uint4*>(src);
        in[0] = a.x; in[1] = a.y; in[2] = a.z; in[3] = a.w;
      } else {
        const uint4 a = reinterpret_cast<const uint4*>(src)[0];
        const uint4 b = reinterpret_cast<const uint4*>(src)[1];
        in[0] = a.x; in[1] = a.y; in[2] = a.z; in[3] = a.w;
        in[4] = b.x; in[5] = b.y; in[6] = b.z; in[7] = b.w;
      }
    } else {
#pragma unroll
      for (int w = 0; w < BITS; ++w)
        in[w] = src[4 * w] | (src[4 * w + 1] << 8) | (src[4 * w + 2] << 16) | ((uint32_t)src[4 * w + 3] << 24);
    }
    uint32_t o[8];
    unpack32<BITS>(in, o);
    uint8_t* dst = out + u * kUnit;
    if (vec_ok) {
      reinterpret_cast<uint4*>(dst)[0] = make_uint4(o[0], o[1], o[2], o[3]);
      reinterpret_cast<uint4*>(dst)[1] = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
#pragma unroll
      for (int b = 0; b < 32; ++b) dst[b] = (uint8_t)(o[b >> 2] >> (8 * (b & 3)));
    }
  } else if (u == n_units) {
    const int64_t first = u * kUnit;
    const int tail = static_cast<int>(n - first);
    if (tail <= 0) return;
    const int64_t b0 = u * (4 * BITS);
    for (int i = 0; i < tail; ++i) {
      const int bit = i * BITS;
      uint32_t v = 0;
      // a field spans at most two bytes (b <= 8)
      const int64_t byte = b0 + (bit >> 3);
      const int sh = bit & 7;
      v = packed[byte] >> sh;
      if (sh + BITS > 8) v |= (uint32_t)packed[byte + 1] << (8 - sh);
      out[first + i] = (uint8_t)(v & ((1u << BITS) - 1u));
    }
  }
}

template <int BITS>
int launch_pack(const uint8_t* idx, int64_t n, uint8_t* out, hipStream_t s) {
  const int64_t nbytes = (n * BITS + 7) / 8;
  const int64_t units = n / kUnit;
  const int64_t total = units + ((n % kUnit) ? 1 : 0);
  if (total == 0) return DIMQ_OK;
  const int vec_ok = aligned(idx, 16) && aligned(out, 16);
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(pack_kernel<BITS>, dim3((unsigned)blocks), dim3(kThreads), 0, s, idx, n, out, nbytes,
                     units, vec_ok);
  return check_launch("pack_bits");
}

template <int BITS>
int launch_unpack(const uint8_t* packed, int64_t n, uint8_t* out, hipStream_t s) {
  const int64_t units = n / kUnit;
  const int64_t total = units + ((n % kUnit) ? 1 : 0);
  if (total == 0) return DIMQ_OK;
  const int vec_ok = aligned(packed, 16) && aligned(out, 16);
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(unpack_kernel<BITS>, dim3((unsigned)blocks), dim3(kThreads), 0, s, packed, out, n, units,
                     vec_ok);
  return check_launch("unpack_bits");
}

}  // namespace
}  // namespace dimq

using namespace dimq;

extern "C" int dimq_pack_bits(const uint8_t* indices, int64_t numel, int bits, uint8_t* packed, void* stream) {
  DIMQ_CHECK(numel >= 0, "numel must be non-negative");
  if (numel > 0) DIMQ_CHECK(indices != nullptr && packed != nullptr, "pack_bits: null pointer");
  hipStream_t s = as_stream(stream);
  switch (bits) {
    case 2: return launch_pack<2>(indices, numel, packed, s);
    case 3: return launch_pack<3>(indices, numel, packed, s);
    case 4: return launch_pack<4>(indices, numel, packed, s);
    case 8: return launch_pack<8>(indices, numel, packed, s);
  }
  return set_error(DIMQ_ERR_UNSUPPORTED, "bits must be one of 2, 3, 4, 8 (got %d)", bits);
}

extern "C" int dimq_unpack_bits(const uint8_t* packed, int64_t packed_numel, int64_t numel, int bits,
                                uint8_t* indices, void* stream) {
  DIMQ_CHECK(numel >= 0, "numel must be non-negative");
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 8))
    return set_error(DIMQ_ERR_UNSUPPORTED, "bits must be one of 2, 3, 4, 8 (got %d)", bits);
  DIMQ_CHECK(packed_numel >= (numel * bits + 7) / 8, "packed tensor is too small for requested numel");
  if (numel > 0) DIMQ_CHECK(indices != nullptr && packed != nullptr, "unpack_bits: null pointer");
  hipStream_t s = as_stream(stream);
  switch (bits) {
    case 2: return launch_unpack<2>(packed, numel, indices, s);
    case 3: return launch_unpack<3>(packed, numel, indices, s);
    case 4: return launch_unpack<4>(packed, numel, indices, s);
    default: return launch_unpack<8>(packed, numel, indices, s);
  }
}

extern "C" int dimq_pack_u4(const uint8_t* indices, int64_t numel, uint8_t* packed, void* stream) {
  return dimq_pack_bits(indices, numel, 4, packed, stream);
}

extern "C" int dimq_unpack_u4(const uint8_t* packed, int64_t packed_numel, int64_t numel, uint8_t* indices,
                              void* stream) {
  return dimq_unpack_bits(packed, packed_numel, numel, 4, indices, stream);
}
