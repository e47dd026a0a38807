// Pieces shared by the LDS-halo conv kernels (conv_halo.h, conv_band.h):
// the argument block, the 32x32x16 MFMA, the epilogue of
// one 32x32 output block and the XCD-aware tile order.
#pragma once

#include "decode.h"

namespace dimq {

struct HaloArgs {
  const void* x;
  int x_layout;  // fp16 input
  int B, C, H, W, OC, OH, OW;
  int KH, KW, pad_h, pad_w;
  int TH;              // output rows per tile (band)
  int IH_t, IW_t, CP;  // halo tile rows, cols, channel pitch (fp16 elements)
  int tiles_h;         // ceil(OH / TH): tiles (bands) per image
  int parts;           // band kernel: runs of 32-pixel blocks per image (one work-group each)
  int nblk;            // band kernel: 32-pixel blocks per image
  const uint32_t* kw;  // kernel-layout weights
  int words_per_lane;  // ceil(T/4) * BITS
  const void* cb;
  int cb_dt, cb_rows, cb_size;
  const void* bias;
  int bias_dt;
  void* y;
  int y_dt, y_layout;
  Epi epi;  // fused residual / activation
  float acc_scale = 1.0f;  // factor on every accumulator (W4A4 calls: the activation scale)
  int park_lds = 0;        // resident kernel: fp32 NCHW stores transposed through LDS (launch sized it)
};

namespace {

// Four consecutive outputs of one lane, after the fused epilogue: one 16-byte
// (fp32) or 8-byte (16-bit) store when `vec`, element stores otherwise.
template <int MODE>
__device__ __forceinline__ void store4(void* y, int dt, int64_t off, const float vin[4], bool vec, const Epi& e,
                                      const ResPairs<4>* r = nullptr) {
  float v[4] = {vin[0], vin[1], vin[2], vin[3]};
  epi_m<MODE, 4>(e, r, off, vec, v);
  if (vec && dt == DIMQ_F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (vec) {
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = dt == DIMQ_F16 ? float_to_f16_bits(v[i]) : float_to_bf16_bits(v[i]);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(y) + off) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) store_from_float(y, dt, off + i, v[i]);
  }
}

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Wave-private LDS area of the transposed fp32 NCHW stores: one 32 x 32
// block parked channel-major with a 36-float row pitch.
constexpr int kParkPitch = 36;
constexpr int kParkFloats = 32 * kParkPitch;

__device__ __forceinline__ floatx16 mfma32x32x16(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Work-group index -> tile, so that the tiles of one XCD (work-groups are
// dealt to the 8 XCDs round-robin) are consecutive row bands: the halo rows
// two bands share are then read once into that XCD's L2.
__device__ __forceinline__ int xcd_tile(int bid, int n) {
  return (n % 8 == 0) ? (bid % 8) * (n / 8) + bid / 8 : bid;
}

// Epilogue of one 32x32 MFMA block.  PXROWS: rows = pixels pix0 + 8j + 4g + i
// of output channel ocl (lane column); else rows = output channels
// ocr + 8j + 4g + i of pixel pix (lane column).
template <bool PXROWS, int MODE>
__device__ __forceinline__ void store_block(const HaloArgs& p, const floatx16& acc, int b, int oh0, int P, int mb,
                                            int col, int g, int ocl, int ocr, float scale, float bv) {
  const int64_t ohw = (int64_t)p.OH * p.OW;
  if constexpr (PXROWS) {
    if (ocl >= p.OC) return;
    const bool vec = (ohw % 4 == 0) && (p.OW % 4 == 0) && (p.y_layout == DIMQ_NCHW);
    const int64_t chan = ((int64_t)b * p.OC + ocl) * ohw + (int64_t)oh0 * p.OW;
    ResPairs<4> rr[4];  // 16-bit residuals of the block, loaded before its first store
    if ((MODE & kEpiRes) && res_pairs(p.epi, vec)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pix0 = mb * 32 + 8 * j + 4 * g;
        if (p.y_layout == DIMQ_NCHW && pix0 + 4 <= P) res_issue<4>(p.epi, chan + pix0, rr[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pix0 = mb * 32 + 8 * j + 4 * g;
      if (pix0 >= P) continue;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = acc[4 * j + i] * scale + bv;
      if (p.y_layout == DIMQ_NCHW && pix0 + 4 <= P) {
        store4<MODE>(p.y, p.y_dt, chan + pix0, v, vec, p.epi, &rr[j]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (pix0 + i < P) {
            const int64_t off = p.y_layout == DIMQ_NCHW
                                    ? chan + pix0 + i
                                    : ((int64_t)b * ohw + (int64_t)oh0 * p.OW + pix0 + i) * p.OC + ocl;
            store_from_float(p.y, p.y_dt, off, epi1_m<MODE>(p.epi, off, v[i]));
          }
        }
      }
    }
  } else {
    const int pix = mb * 32 + col;
    const bool vec = (p.OC % 4 == 0) && (p.y_layout == DIMQ_NHWC);
    const int64_t pbase = (int64_t)b * ohw + (int64_t)oh0 * p.OW + pix;
    ResPairs<4> rr[4];  // 16-bit residuals of the block, loaded before its first store
    if ((MODE & kEpiRes) && res_pairs(p.epi, vec) && pix < P && p.y_layout == DIMQ_NHWC) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ocb = ocr + 8 * j + 4 * g;
        if (ocb + 4 <= p.OC) res_issue<4>(p.epi, pbase * p.OC + ocb, rr[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ocb = ocr + 8 * j + 4 * g;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sc = __shfl(scale, 8 * j + 4 * g + i, 32);
        const float bb = __shfl(bv, 8 * j + 4 * g + i, 32);
        v[i] = acc[4 * j + i] * sc + bb;
      }
      if (pix >= P) continue;
      if (p.y_layout == DIMQ_NHWC && ocb + 4 <= p.OC) {
        store4<MODE>(p.y, p.y_dt, pbase * p.OC + ocb, v, vec, p.epi, &rr[j]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (ocb + i < p.OC) {
            const int64_t off = p.y_layout == DIMQ_NHWC ? pbase * p.OC + ocb + i
                                                        : ((int64_t)b * p.OC + ocb + i) * ohw + (int64_t)oh0 * p.OW + pix;
            store_from_float(p.y, p.y_dt, off, epi1_m<MODE>(p.epi, off, v[i]));
          }
        }
      }
    }
  }
}

}  // namespace
}  // namespace dimq
