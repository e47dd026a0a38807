// Direct KHxKW convolution over an LDS halo tile (the fast path for the
// ResNet 3x3 layers and BASELINE cfg2).
//
// Work-group = 256 threads, one tile = TH output rows x the full output width
// of one image x 64 output channels.  The input rows the tile needs (with the
// zero padding) are staged once in LDS as [row][col][channel] fp16, channel
// pitch C + 8 so that 16 consecutive pixels read 16-byte channel groups from
// 16 distinct 4-bank groups (no bank conflicts).  The im2col matrix is never
// formed: the MFMA operand for (pixel, kh, kw, 8 channels) is one ds_read_b128
// at the pixel's shifted position.
//
// The matrix cores run v_mfma_f32_32x32x16_f16 (measured on MI355X: ~2.2
// PFLOP/s sustained against ~1.2 for the 16x16x32 shape).  One MFMA covers 32
// pixels x 32 output channels x 16 input channels; lane l holds 8 channels
// (group g = l / 32) of pixel / output channel l % 32.
//
// Weights arrive in a "kernel layout" (dimq_conv2d_prepare_weight): for every
// output channel n and lane group g, the b-bit indices of the sub-steps
// t = (kh, kw, 16-channel chunk) x 8 channels, ordered so that the v_perm
// decode of decode.h yields channels in natural order.  Each lane keeps its
// row's packed indices and codebook byte planes in VGPRs for the whole tile.
#pragma once

#include "conv_common.h"

#include <algorithm>

namespace dimq {
namespace {


// Stages the input rows of one tile into LDS as fp16 [row][col][channel]
// (channel pitch p.CP), zero outside the image: halo row r <-> input row
// ih0 + r, halo column hc <-> input column hc - pad_w.  256 threads.
template <int CC16>
__device__ __forceinline__ void stage_halo(const HaloArgs& p, int b, int ih0, uint16_t* halo, int tid) {
  constexpr int C = CC16 * 16;
  if (p.x_layout == DIMQ_NCHW && (p.W & 7) == 0) {
    // task = (8-channel octet, halo row, 8 input columns): eight 16-byte row
    // loads, an 8x8 transpose in registers, eight 16-byte LDS stores.
    const int qn = p.W / 8;
    const int tasks = (C / 8) * p.IH_t * qn;
    constexpr int TPT = 2;  // tasks in flight per thread
    for (int t0 = 0; t0 < tasks; t0 += 256 * TPT) {
      uint4 v[TPT][8];
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        const int t = t0 + u * 256 + tid;
        const int tt = t < tasks ? t : 0;
        const int co = tt % (C / 8);
        const int rest = tt / (C / 8);
        const int q = rest % qn;
        const int r = rest / qn;
        const int ih = ih0 + r;
        const bool live = t < tasks && ih >= 0 && ih < p.H;
        const int ihc = live ? ih : 0;
        const uint16_t* src = reinterpret_cast<const uint16_t*>(p.x) +
                              (((int64_t)b * p.C + 8 * co) * p.H + ihc) * p.W + 8 * q;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          v[u][c] = *reinterpret_cast<const uint4*>(src + (int64_t)c * p.H * p.W);
          if (!live) v[u][c] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        const int t = t0 + u * 256 + tid;
        if (t >= tasks) continue;
        const int co = t % (C / 8);
        const int rest = t / (C / 8);
        const int q = rest % qn;
        const int r = rest / qn;
        uint32_t in[8][4];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          in[c][0] = v[u][c].x; in[c][1] = v[u][c].y; in[c][2] = v[u][c].z; in[c][3] = v[u][c].w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          // pixel j: channels 2w, 2w+1 from half (j&1) of word j/2 of rows 2w, 2w+1
          const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
          const uint4 o = make_uint4(perm(in[1][j >> 1], in[0][j >> 1], sel), perm(in[3][j >> 1], in[2][j >> 1], sel),
                                     perm(in[5][j >> 1], in[4][j >> 1], sel), perm(in[7][j >> 1], in[6][j >> 1], sel));
          const int hc = 8 * q + j + p.pad_w;
          if (hc < p.IW_t) *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + hc) * p.CP + 8 * co]) = o;
        }
      }
    }
    // zero the padding columns (hc < pad_w, hc >= pad_w + W)
    const int npad = p.IW_t - p.W;
    const int ztasks = p.IH_t * (npad > 0 ? npad : 0) * (C / 8);
    for (int t = tid; t < ztasks; t += 256) {
      const int co = t % (C / 8);
      const int rest = t / (C / 8);
      const int pc = rest % npad;
      const int r = rest / npad;
      const int hc = pc < p.pad_w ? pc : p.W + pc;
      if (hc < p.IW_t) *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + hc) * p.CP + 8 * co]) = make_uint4(0, 0, 0, 0);
    }
  } else if (p.x_layout == DIMQ_NCHW) {
    // any width: task = (channel pair, halo row, halo column)
    const int tasks = (C / 2) * p.IH_t * p.IW_t;
    for (int t = tid; t < tasks; t += 256) {
      const int hc = t % p.IW_t;
      const int rest = t / p.IW_t;
      const int r = rest % p.IH_t;
      const int c2 = rest / p.IH_t;
      const int ih = ih0 + r, iw = hc - p.pad_w;
      uint32_t a = 0, bb = 0;
      if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t off = (((int64_t)b * p.C + 2 * c2) * p.H + ih) * p.W + iw;
        a = reinterpret_cast<const uint16_t*>(p.x)[off];
        bb = reinterpret_cast<const uint16_t*>(p.x)[off + (int64_t)p.H * p.W];
      }
      *reinterpret_cast<uint32_t*>(&halo[(r * p.IW_t + hc) * p.CP + 2 * c2]) = a | (bb << 16);
    }
  } else {
    // NHWC: task = (halo pixel, 8 channels) -> one 16-byte load, one 16-byte LDS store
    const int tasks = p.IH_t * p.IW_t * (C / 8);
    constexpr int TPT = 8;
    for (int t0 = 0; t0 < tasks; t0 += 256 * TPT) {
      uint4 v[TPT];
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        const int t = t0 + u * 256 + tid;
        const int tt = t < tasks ? t : 0;
        const int c8 = tt % (C / 8);
        const int pix = tt / (C / 8);
        const int r = pix / p.IW_t;
        const int hc = pix - r * p.IW_t;
        const int ih = ih0 + r;
        const int iw = hc - p.pad_w;
        const bool live = t < tasks && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
        const int64_t off = live ? (((int64_t)b * p.H + ih) * p.W + iw) * p.C + 8 * c8 : 0;
        v[u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.x) + off);
        if (!live) v[u] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        const int t = t0 + u * 256 + tid;
        if (t >= tasks) continue;
        const int c8 = t % (C / 8);
        const int pix = t / (C / 8);
        *reinterpret_cast<uint4*>(&halo[pix * p.CP + 8 * c8]) = v[u];
      }
    }
  }
}

// T = KH*KW*CC16 sub-steps of 16 channels; CC16 = C / 16.
// Waves: wn = wave & 1 owns output channels [32*wn, 32*wn + 32) of the tile,
// wm = wave >> 1 owns the 32-pixel m-blocks wm, wm + 2, wm + 4, wm + 6, so one
// decoded weight fragment feeds 4 MFMAs.
// PXROWS: MFMA rows are pixels (lane holds 4 consecutive pixels of one output
// channel: contiguous in NCHW); otherwise rows are output channels (lane holds
// 4 consecutive channels of one pixel: contiguous in NHWC).
template <int BITS, int CC16, int STRIDE, int KHW, bool PXROWS, int MODE>
__global__ __launch_bounds__(256) void conv_halo_kernel(const HaloArgs p) {
  constexpr int T = KHW * CC16;
  constexpr int CHUNKS = (T + 3) / 4;
  constexpr int WPL = CHUNKS * BITS;  // packed words per lane
  constexpr int MBW = 4;              // 32-pixel m-blocks per wave (256 pixels per tile)
  extern __shared__ __attribute__((aligned(16))) uint16_t halo[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  const int tile = blockIdx.x;
  const int b = tile / p.tiles_h;
  const int oh0 = (tile - b * p.tiles_h) * p.TH;
  const int oc0 = blockIdx.y * 64;
  const int C = CC16 * 16;
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int ocl = oc0 + 32 * wn + col;  // this lane's weight row

  // ---- codebooks of the 64 output rows -> LDS (fp32), then byte planes
  constexpr int E = 1 << BITS;
  __shared__ float cbs[64 * E];
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, oc0, 64, p.OC, cbs, tid, 256);

  // ---- weights: this lane's packed words (independent loads)
  uint32_t wreg[WPL];
  {
    const int oc = min(ocl, p.OC - 1);
    const uint32_t* src = p.kw + ((int64_t)oc * 2 + g) * WPL;
#pragma unroll
    for (int w = 0; w < WPL; ++w) wreg[w] = src[w];
  }

  stage_halo<CC16>(p, b, oh0 * STRIDE - p.pad_h, halo, tid);
  __syncthreads();
  CodebookRegs<BITS> cbr;
  float scale;
  {
    const int rl = (p.cb_rows == 1) ? 0 : 32 * wn + col;
    const int e = planes_from_lds<BITS, false>(cbs + rl * E, cbr, cbr);
    scale = ldexpf(p.acc_scale, -e);
  }

  // ---- this lane's pixels: m-blocks mb = wm + 2*q (pixels past the tile read
  //      pixel 0 and are never stored, so the loop below has no branches)
  const int P = min(p.TH, p.OH - oh0) * p.OW;
  int base[MBW];
#pragma unroll
  for (int q = 0; q < MBW; ++q) {
    int pix = (wm + 2 * q) * 32 + col;
    if (pix >= P) pix = 0;
    const int r = pix / p.OW;
    const int c = pix - r * p.OW;
    base[q] = ((r * STRIDE) * p.IW_t + c * STRIDE) * p.CP + 8 * g;
  }

  floatx16 acc[MBW];
#pragma unroll
  for (int q = 0; q < MBW; ++q)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[q][i] = 0.0f;

#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int khw = t / CC16;
    const int cc = t - khw * CC16;
    const int kh = (KHW == 9) ? khw / 3 : 0;
    const int kw = (KHW == 9) ? khw - 3 * kh : 0;
    const int koff = (kh * p.IW_t + kw) * p.CP + 16 * cc;
    uint32_t chunk[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) chunk[w] = wreg[(t >> 2) * BITS + w];
    const half8 wf = decode_sub<BITS>(chunk, t & 3, cbr);
    half8 xf[MBW];
#pragma unroll
    for (int q = 0; q < MBW; ++q) xf[q] = *reinterpret_cast<const half8*>(&halo[base[q] + koff]);
#pragma unroll
    for (int q = 0; q < MBW; ++q) acc[q] = PXROWS ? mfma32x32x16(xf[q], wf, acc[q]) : mfma32x32x16(wf, xf[q], acc[q]);
  }

  // ---- epilogue: acc[q][4j + i] = D[row 8j + 4g + i][col], 32x32 block q
  const int64_t ohw = (int64_t)p.OH * p.OW;
  if constexpr (PXROWS) {
    // rows are pixels mb*32 + 8j + 4g + i, column = output channel ocl.
    // NCHW offset of (oc, pixel) = (b*OC + oc)*OH*OW + oh0*OW + pixel.
    if (ocl < p.OC) {
      const bool vec = (ohw % 4 == 0) && (p.OW % 4 == 0) && (p.y_layout == DIMQ_NCHW);
      const float bv = p.bias ? load_as_float(p.bias, p.bias_dt, ocl) : 0.0f;
      const int64_t chan = ((int64_t)b * p.OC + ocl) * ohw + (int64_t)oh0 * p.OW;
#pragma unroll
      for (int q = 0; q < MBW; ++q) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int pix0 = (wm + 2 * q) * 32 + 8 * j + 4 * g;
          if (pix0 >= P) continue;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = acc[q][4 * j + i] * scale + bv;
          if (p.y_layout == DIMQ_NCHW && pix0 + 4 <= P) {
            store4<MODE>(p.y, p.y_dt, chan + pix0, v, vec, p.epi);
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
      }
    }
  } else {
    // rows are output channels oc0 + 32*wn + 8j + 4g + i, column = pixel mb*32 + col.
    // NHWC offset of (pixel, oc) = (b*OH*OW + oh0*OW + pixel)*OC + oc.
    const bool vec = (p.OC % 4 == 0) && (p.y_layout == DIMQ_NHWC);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ocb = oc0 + 32 * wn + 8 * j + 4 * g;
      float sc[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = __shfl(scale, 8 * j + 4 * g + i, 32);
        bv[i] = (p.bias && ocb + i < p.OC) ? load_as_float(p.bias, p.bias_dt, ocb + i) : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < MBW; ++q) {
        const int pix = (wm + 2 * q) * 32 + col;
        if (pix >= P) continue;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = acc[q][4 * j + i] * sc[i] + bv[i];
        const int64_t pbase = (int64_t)b * ohw + (int64_t)oh0 * p.OW + pix;
        if (p.y_layout == DIMQ_NHWC && ocb + 4 <= p.OC) {
          store4<MODE>(p.y, p.y_dt, pbase * p.OC + ocb, v, vec, p.epi);
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
}

// fp32 NCHW stores of one 32-pixel x 32-channel MFMA block (PXROWS layout:
// lane (col, g) holds channel col's pixels 8j + 4g + i) through the wave's
// private LDS area: the block is parked channel-major (row pitch 36 floats),
// then lane l stores pixels 4(l % 8) .. +3 of channel l / 8 + 8 it, so each
// store instruction writes 8 whole 128-byte channel runs instead of 32
// quarter runs.  The stores are non-temporal: the output is not re-read by
// this kernel, and streaming it past the L2 leaves the L2 to the input rows
// neighbouring tiles share.  A wave's LDS operations execute in order, so the
// wave-local park / read needs no work-group barrier.
__device__ __forceinline__ void store_block_lds(const HaloArgs& p, const floatx16& acc, int b, int oh0, int P, int mb,
                                                int col, int g, int ocr, int lane, float scale, float bv,
                                                float* park) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    *reinterpret_cast<float4*>(park + col * kParkPitch + 8 * j + 4 * g) =
        make_float4(acc[4 * j] * scale + bv, acc[4 * j + 1] * scale + bv, acc[4 * j + 2] * scale + bv,
                    acc[4 * j + 3] * scale + bv);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int64_t ohw = (int64_t)p.OH * p.OW;
  const int p4 = 4 * (lane & 7);
  const int pix0 = mb * 32 + p4;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = (lane >> 3) + 8 * it;
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = *reinterpret_cast<const f4v*>(park + c * kParkPitch + p4);
    const int oc = ocr + c;
    if (oc < p.OC && pix0 < P)  // P % 4 == 0 (OW % 4 == 0): a chunk is all in or all out
      __builtin_nontemporal_store(v, reinterpret_cast<f4v*>(reinterpret_cast<float*>(p.y) +
                                                            ((int64_t)b * p.OC + oc) * ohw + (int64_t)oh0 * p.OW +
                                                            pix0));
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Resident-weight variant of the halo kernel for T = KH*KW*C/16 <= 36
// sub-steps (3x3 at C = 64, 1x1 at C <= 128): every lane decodes its output
// channel's T weight fragments once (4*T VGPRs) and keeps them for the tile,
// so the MFMA loop is one ds_read_b128 and one v_mfma_f32_32x32x16_f16 per
// sub-step and block, with no decode work.  A wave runs two m-blocks at a
// time (two independent accumulator chains: one dependent 32x32x16 chain
// leaves the matrix core idle most of the time), and stores each finished
// pair straight from registers while the next pair computes.  Launch bounds
// give two work-groups (8 waves) per CU.
template <int BITS, int CC16, int STRIDE, int KHW, bool PXROWS, int MODE>
__global__ __launch_bounds__(256, 2) void conv_resident_kernel(const HaloArgs p) {
  constexpr int T = KHW * CC16;
  static_assert(T <= 36, "resident weights are limited to 36 sub-steps");
  constexpr int CHUNKS = (T + 3) / 4;
  constexpr int WPL = CHUNKS * BITS;
  constexpr int CP = CC16 * 16 + 8;
  extern __shared__ __attribute__((aligned(16))) uint16_t halo[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int b = tile / p.tiles_h;
  const int oh0 = (tile - b * p.tiles_h) * p.TH;
  const int oc0 = blockIdx.y * 64;
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int ocl = oc0 + 32 * wn + col;
  // fp32 NCHW output without epilogue: each wave transposes its 32 x 32
  // blocks through a private LDS area after the halo (launch adds it)
  const bool lds_store = PXROWS && MODE == kEpiNone && p.y_dt == DIMQ_F32 && p.y_layout == DIMQ_NCHW &&
                         (p.OW % 4) == 0 && p.park_lds;
  float* park = reinterpret_cast<float*>(halo + (size_t)p.IH_t * p.IW_t * CP) + wave * kParkFloats;

  constexpr int E = 1 << BITS;
  __shared__ float cbs[64 * E];
  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, oc0, 64, p.OC, cbs, tid, 256);

  uint32_t wreg[WPL];
  {
    const int oc = min(ocl, p.OC - 1);
    const uint32_t* src = p.kw + ((int64_t)oc * 2 + g) * WPL;
#pragma unroll
    for (int w = 0; w < WPL; ++w) wreg[w] = src[w];
  }

  stage_halo<CC16>(p, b, oh0 * STRIDE - p.pad_h, halo, tid);
  __syncthreads();

  CodebookRegs<BITS> cbr;
  float scale;
  {
    const int rl = (p.cb_rows == 1) ? 0 : 32 * wn + col;
    const int e = planes_from_lds<BITS, false>(cbs + rl * E, cbr, cbr);
    scale = ldexpf(p.acc_scale, -e);
  }
  const float bv = (p.bias && ocl < p.OC) ? load_as_float(p.bias, p.bias_dt, ocl) : 0.0f;

  half8 wf[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t chunk[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) chunk[w] = wreg[(t >> 2) * BITS + w];
    wf[t] = decode_sub<BITS>(chunk, t & 3, cbr);
  }

  const int P = min(p.TH, p.OH - oh0) * p.OW;
  const int nblk = (P + 31) / 32;
  const int row_step = p.IW_t * CP;
  // this wave's blocks wm, wm + 2, ... in pairs (q = 0, 1 -> blocks mb, mb + 2)
  for (int mb = wm; mb < nblk; mb += 4) {
    int base[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      int pix = (mb + 2 * q) * 32 + col;
      if (pix >= P) pix = 0;  // rows past the tile read pixel 0 and are not stored
      const int r = pix / p.OW;
      const int c = pix - r * p.OW;
      base[q] = ((r * STRIDE) * p.IW_t + c * STRIDE) * CP + 8 * g;
    }
    auto frag = [&](int u) {
      const int t = u >> 1, q = u & 1;
      const int khw = t / CC16;
      const int cc = t - khw * CC16;
      const int kh = (KHW == 9) ? khw / 3 : 0;
      const int kw = (KHW == 9) ? khw - 3 * kh : 0;
      return *reinterpret_cast<const half8*>(halo + base[q] + kh * row_step + kw * CP + 16 * cc);
    };
    constexpr int U = 2 * T;
    constexpr int DEPTH = 4;
    half8 xr[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) xr[u] = frag(u);
    floatx16 acc[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][i] = acc[1][i] = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = u >> 1, q = u & 1;
      acc[q] = PXROWS ? mfma32x32x16(xr[u % DEPTH], wf[t], acc[q]) : mfma32x32x16(wf[t], xr[u % DEPTH], acc[q]);
      if (u + DEPTH < U) xr[u % DEPTH] = frag(u + DEPTH);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, DEPTH, 0);
#pragma unroll
    for (int u = 0; u < U - DEPTH; ++u) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, DEPTH, 0);
    if constexpr (PXROWS && MODE == kEpiNone) {
      if (lds_store) {
        store_block_lds(p, acc[0], b, oh0, P, mb, col, g, oc0 + 32 * wn, lane, scale, bv, park);
        if (mb + 2 < nblk) store_block_lds(p, acc[1], b, oh0, P, mb + 2, col, g, oc0 + 32 * wn, lane, scale, bv, park);
        continue;
      }
    }
    store_block<PXROWS, MODE>(p, acc[0], b, oh0, P, mb, col, g, ocl, oc0 + 32 * wn, scale, bv);
    if (mb + 2 < nblk) store_block<PXROWS, MODE>(p, acc[1], b, oh0, P, mb + 2, col, g, ocl, oc0 + 32 * wn, scale, bv);
  }
}

// Epilogue modes each kernel is instantiated for (others: generic kernels).
// Resident kernel, NHWC output: none / relu / residual / residual + relu (the
// ResNet blocks); NCHW output: none / relu, each also with the next layer's
// activation quantization (chained W4A4 layers); decode-per-step kernel: none.
inline bool halo_mode_ok(int mode, bool resident, bool nchw) {
  if (!resident) return mode == kEpiNone;
  if (nchw) return mode == kEpiNone || mode == kEpiRelu || mode == kEpiQuant || mode == (kEpiRelu | kEpiQuant);
  return mode == kEpiNone || mode == kEpiRelu || mode == kEpiRes || mode == kEpiResRelu;
}

template <int BITS, int CC, int STRIDE, int KHW, bool PXROWS, int MODE>
int launch_resident(const HaloArgs& p0, dim3 grid, size_t lds, hipStream_t s) {
  auto k = conv_resident_kernel<BITS, CC, STRIDE, KHW, PXROWS, MODE>;
  HaloArgs p = p0;
  p.park_lds = 0;
  if (PXROWS && MODE == kEpiNone && p.y_dt == DIMQ_F32 && p.y_layout == DIMQ_NCHW && p.OW % 4 == 0) {
    p.park_lds = 1;
    lds += (size_t)4 * kParkFloats * sizeof(float);
  }
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "conv2d_codebook (halo): %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(k, grid, dim3(256), lds, s, p);
  return check_launch("conv2d_codebook (halo, resident weights)");
}

template <int BITS, int CC, int STRIDE, int KHW>
int launch_halo_k(const HaloArgs& p, int mode, dim3 grid, size_t lds, hipStream_t s) {
  if constexpr (KHW * CC <= 36) {
    if (p.y_layout == DIMQ_NCHW) {
      switch (mode) {
        case kEpiRelu: return launch_resident<BITS, CC, STRIDE, KHW, true, kEpiRelu>(p, grid, lds, s);
        case kEpiQuant: return launch_resident<BITS, CC, STRIDE, KHW, true, kEpiQuant>(p, grid, lds, s);
        case kEpiRelu | kEpiQuant:
          return launch_resident<BITS, CC, STRIDE, KHW, true, kEpiRelu | kEpiQuant>(p, grid, lds, s);
        default: return launch_resident<BITS, CC, STRIDE, KHW, true, kEpiNone>(p, grid, lds, s);
      }
    }
    switch (mode) {
      case kEpiRelu: return launch_resident<BITS, CC, STRIDE, KHW, false, kEpiRelu>(p, grid, lds, s);
      case kEpiRes: return launch_resident<BITS, CC, STRIDE, KHW, false, kEpiRes>(p, grid, lds, s);
      case kEpiResRelu: return launch_resident<BITS, CC, STRIDE, KHW, false, kEpiResRelu>(p, grid, lds, s);
      default: return launch_resident<BITS, CC, STRIDE, KHW, false, kEpiNone>(p, grid, lds, s);
    }
  }
  if (p.y_layout == DIMQ_NCHW)
    hipLaunchKernelGGL((conv_halo_kernel<BITS, CC, STRIDE, KHW, true, kEpiNone>), grid, dim3(256), lds, s, p);
  else
    hipLaunchKernelGGL((conv_halo_kernel<BITS, CC, STRIDE, KHW, false, kEpiNone>), grid, dim3(256), lds, s, p);
  return check_launch("conv2d_codebook (halo)");
}

template <int BITS, int CC, int STRIDE>
int launch_halo(const HaloArgs& p, int mode, hipStream_t s) {
  const size_t lds = (size_t)p.IH_t * p.IW_t * p.CP * sizeof(uint16_t);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles_h), static_cast<unsigned>((p.OC + 63) / 64));
  return p.KH == 3 ? launch_halo_k<BITS, CC, STRIDE, 9>(p, mode, grid, lds, s)
                   : launch_halo_k<BITS, CC, STRIDE, 1>(p, mode, grid, lds, s);
}

template <int BITS>
int launch_halo_cc(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s) {
  if (CC16 == 4) return stride == 1 ? launch_halo<BITS, 4, 1>(p, mode, s) : launch_halo<BITS, 4, 2>(p, mode, s);
  return stride == 1 ? launch_halo<BITS, 8, 1>(p, mode, s) : launch_halo<BITS, 8, 2>(p, mode, s);
}

}  // namespace

// Instantiations per bit width (conv_halo_b2/3/4.hip).
int launch_halo_b2(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s);
int launch_halo_b3(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s);
int launch_halo_b4(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s);
int launch_band_b2(const HaloArgs& p, int mode, hipStream_t s);
int launch_band_b3(const HaloArgs& p, int mode, hipStream_t s);
int launch_band_b4(const HaloArgs& p, int mode, hipStream_t s);

}  // namespace dimq
