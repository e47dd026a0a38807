// Row-streaming direct convolution for the layers whose decoded weights fit
// in registers: T = KH*KW*C/16 <= 36 sub-steps of 16 channels (3x3 at C = 64,
// 1x1 at C <= 128) — ResNet-18 layer1 and BASELINE cfg2.
//
// One 256-thread work-group per CU owns a band of output rows of one image x
// 64 output channels (the launcher picks the band height so that the grid is
// about one work-group per CU).  Its input rows pass through an LDS ring of NR
// rows ([row][col][channel] fp16, channel pitch C + 8: 16-byte reads of 16
// consecutive pixels hit distinct bank groups).  The band's pixels, flattened
// row-major, are processed in steps of 128 (four 32-pixel MFMA blocks):
//
//   step s:  MFMA the step's blocks out of the ring into an LDS output tile
//            |  barrier  |  wait for the rows of step s+1 (loaded into
//            registers during step s) and write them into the ring (NCHW:
//            8x8 transposes; slots of rows no later step reads)  |  issue the
//            loads of step s+2's rows, then the tile's coalesced 16-byte
//            stores  |  barrier
//
// so reading HBM, the matrix cores and writing HBM overlap within every CU:
// the row loads for step s+2 and the stores of step s run under the MFMAs of
// step s+1.
//
// 4 waves (one per SIMD, 512 registers each): wn = wave & 1 owns output
// channels [32*wn, 32*wn + 32); pg = wave >> 1 owns blocks 4*s + pg and
// 4*s + pg + 2 of step s.  Each lane decodes its output channel's T weight
// fragments once (4*T VGPRs) and keeps them, so the inner loop is one
// ds_read_b128 and one v_mfma_f32_32x32x16_f16 per sub-step and block, with
// four independent accumulator chains per wave.
// Rows are pixels (NCHW output: 4 consecutive pixels of one channel per
// lane) or output channels (NHWC output: 4 consecutive channels).
#pragma once

#include "conv_common.h"

namespace dimq {
namespace {

constexpr int kStreamThreads = 256;
constexpr int kStepPx = 128;

// Staging tasks for `nr` input rows.  NCHW (W % 8 == 0): task = (channel
// octet co, column group q, row rr), co fastest: eight 16-byte row loads (8
// channels x 8 columns) and an 8x8 transpose.  NHWC: the rows' 16-byte
// [column][channel octet] units, task t taking units t + k*TT (k < 8) so that
// consecutive lanes read consecutive 16 bytes.
template <int CC16, bool NHWC>
__device__ __forceinline__ int row_tasks(const HaloArgs& p, int nr) {
  constexpr int C8 = CC16 * 2;
  if constexpr (NHWC) return (nr * p.W * C8 + 7) / 8;
  return nr * (p.W / 8) * C8;
}

template <int CC16, bool NHWC>
__device__ __forceinline__ void issue_rows(const HaloArgs& p, int b, int ih_a, int nr, int task, uint4 (&v)[8]) {
  constexpr int C = CC16 * 16, C8 = CC16 * 2;
  const uint16_t* x = reinterpret_cast<const uint16_t*>(p.x);
  if constexpr (NHWC) {
    const int per_row = p.W * C8;
    const int units = nr * per_row;
    const int TT = (units + 7) / 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int u = task + k * TT;
      const int uu = u < units ? u : 0;
      const int rr = uu / per_row;
      const int rem = uu - rr * per_row;
      const int iw = rem / C8;
      const int c8 = rem - iw * C8;
      const int ih = ih_a + rr;
      const bool live = u < units && ih >= 0 && ih < p.H;
      const int ihc = live ? ih : 0;
      v[k] = *reinterpret_cast<const uint4*>(x + (((int64_t)b * p.H + ihc) * p.W + iw) * C + 8 * c8);
      if (!live) v[k] = make_uint4(0, 0, 0, 0);
    }
  } else {
    const int qn = p.W / 8;
    const int co = task % C8;
    const int rest = task / C8;
    const int q = rest % qn;
    const int rr = rest / qn;
    const int ih = ih_a + rr;
    const bool live = ih >= 0 && ih < p.H;
    const int ihc = live ? ih : 0;
    const uint16_t* src = x + (((int64_t)b * C + 8 * co) * p.H + ihc) * p.W + 8 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      v[c] = *reinterpret_cast<const uint4*>(src + (int64_t)c * p.H * p.W);
      if (!live) v[c] = make_uint4(0, 0, 0, 0);
    }
  }
}

__device__ __forceinline__ uint4 to_f16x8(uint4 w, int dt) {
  if (dt == DIMQ_F16) return w;
  uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] = to_f16_bits(a[k] & 0xffffu, dt) | (to_f16_bits(a[k] >> 16, dt) << 16);
  return make_uint4(a[0], a[1], a[2], a[3]);
}

// Writes the rows loaded by issue_rows (band-relative input rows r_a ...) into
// their ring slots r & (NR - 1); columns at hc = iw + pad_w.
template <int CC16, bool NHWC>
__device__ __forceinline__ void commit_rows(const HaloArgs& p, uint16_t* ring, int r_a, int nr, int task,
                                            const uint4 (&v)[8]) {
  constexpr int C8 = CC16 * 2, CP = CC16 * 16 + 8;
  const int nrm = p.NR - 1;
  if constexpr (NHWC) {
    const int per_row = p.W * C8;
    const int units = nr * per_row;
    const int TT = (units + 7) / 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int u = task + k * TT;
      if (u >= units) continue;
      const int rr = u / per_row;
      const int rem = u - rr * per_row;
      const int iw = rem / C8;
      const int c8 = rem - iw * C8;
      const int hc = iw + p.pad_w;
      if (hc < p.IW_t)
        *reinterpret_cast<uint4*>(ring + ((((r_a + rr) & nrm) * p.IW_t + hc) * CP + 8 * c8)) = to_f16x8(v[k], p.x_dt);
    }
  } else {
    const int qn = p.W / 8;
    const int co = task % C8;
    const int rest = task / C8;
    const int q = rest % qn;
    const int rr = rest / qn;
    uint32_t in[8][4];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint4 w = to_f16x8(v[c], p.x_dt);
      in[c][0] = w.x;
      in[c][1] = w.y;
      in[c][2] = w.z;
      in[c][3] = w.w;
    }
    uint16_t* row = ring + ((r_a + rr) & nrm) * p.IW_t * CP + 8 * co;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // column j: channels 2w, 2w+1 from half (j & 1) of word j/2 of rows 2w, 2w+1
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      const uint4 o = make_uint4(perm(in[1][j >> 1], in[0][j >> 1], sel), perm(in[3][j >> 1], in[2][j >> 1], sel),
                                 perm(in[5][j >> 1], in[4][j >> 1], sel), perm(in[7][j >> 1], in[6][j >> 1], sel));
      const int hc = 8 * q + j + p.pad_w;
      if (hc < p.IW_t) *reinterpret_cast<uint4*>(row + hc * CP) = o;
    }
  }
}

// Output tile of one step in LDS, fp32: PXROWS [64 channels][kTilePitchPx]
// (pixel-contiguous, for NCHW stores), else [128 pixels][kTilePitchOc]
// (channel-contiguous, for NHWC stores).  The pitches keep the 16-byte
// writes of a 16-lane group on distinct banks.
constexpr int kTilePitchPx = kStepPx + 4;
constexpr int kTilePitchOc = 64 + 4;
constexpr int kTileFloats = 64 * kTilePitchPx > kStepPx * kTilePitchOc ? 64 * kTilePitchPx : kStepPx * kTilePitchOc;

// acc of block pg (32 pixels x 32 channels of half wn) -> tile, with the
// codebook scale 2^-e and the bias applied.
template <bool PXROWS>
__device__ __forceinline__ void write_tile(float* tile, const floatx16& acc, int pg, int wn, int col, int g, float scale,
                                           float bv) {
  if constexpr (PXROWS) {
    // lane: channel 32*wn + col, pixels 32*pg + 8j + 4g + i
    float* row = tile + (32 * wn + col) * kTilePitchPx + 32 * pg + 4 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<float4*>(row + 8 * j) = make_float4(acc[4 * j] * scale + bv, acc[4 * j + 1] * scale + bv,
                                                            acc[4 * j + 2] * scale + bv, acc[4 * j + 3] * scale + bv);
  } else {
    // lane: pixel 32*pg + col, channels 32*wn + 8j + 4g + i
    float* row = tile + (32 * pg + col) * kTilePitchOc + 32 * wn + 4 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = acc[4 * j + i] * __shfl(scale, 8 * j + 4 * g + i, 32) + __shfl(bv, 8 * j + 4 * g + i, 32);
      *reinterpret_cast<float4*>(row + 8 * j) = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

// Stores the tile of step s (band pixels [128 s, 128 s + 128) clipped to P)
// with 16-byte global stores where alignment allows.
template <bool PXROWS>
__device__ __forceinline__ void store_tile(const HaloArgs& p, const float* tile, int b, int oh0, int P, int s, int oc0,
                                           int tid) {
  const int64_t ohw = (int64_t)p.OH * p.OW;
  const int px0 = s * kStepPx;
  const int npx = min(kStepPx, P - px0);
  if constexpr (PXROWS) {
    const bool vec = p.y_layout == DIMQ_NCHW && ((int64_t)oh0 * p.OW + px0) % 4 == 0 && ohw % 4 == 0;
    for (int i = tid; i < 64 * (kStepPx / 4); i += kStreamThreads) {
      const int oc = i / (kStepPx / 4);
      const int q = 4 * (i - oc * (kStepPx / 4));
      if (q >= npx || oc0 + oc >= p.OC) continue;
      const float4 v4 = *reinterpret_cast<const float4*>(tile + oc * kTilePitchPx + q);
      const float v[4] = {v4.x, v4.y, v4.z, v4.w};
      const int64_t base = ((int64_t)b * p.OC + oc0 + oc) * ohw + (int64_t)oh0 * p.OW + px0 + q;
      if (p.y_layout == DIMQ_NCHW && q + 4 <= npx) {
        store4<kEpiNone>(p.y, p.y_dt, base, v, vec, p.epi);
      } else {
        for (int k = 0; k < 4 && q + k < npx; ++k) {
          const int64_t off = p.y_layout == DIMQ_NCHW
                                  ? base + k
                                  : ((int64_t)b * ohw + (int64_t)oh0 * p.OW + px0 + q + k) * p.OC + oc0 + oc;
          store_from_float(p.y, p.y_dt, off, v[k]);
        }
      }
    }
  } else {
    const bool vec = p.y_layout == DIMQ_NHWC && p.OC % 4 == 0;
    for (int i = tid; i < kStepPx * 16; i += kStreamThreads) {
      const int px = i / 16;
      const int o4 = 4 * (i - px * 16);
      if (px >= npx || oc0 + o4 >= p.OC) continue;
      const float4 v4 = *reinterpret_cast<const float4*>(tile + px * kTilePitchOc + o4);
      const float v[4] = {v4.x, v4.y, v4.z, v4.w};
      const int64_t pix = (int64_t)b * ohw + (int64_t)oh0 * p.OW + px0 + px;
      if (p.y_layout == DIMQ_NHWC && oc0 + o4 + 4 <= p.OC) {
        store4<kEpiNone>(p.y, p.y_dt, pix * p.OC + oc0 + o4, v, vec, p.epi);
      } else {
        for (int k = 0; k < 4 && oc0 + o4 + k < p.OC; ++k) {
          const int64_t off = p.y_layout == DIMQ_NHWC
                                  ? pix * p.OC + oc0 + o4 + k
                                  : ((int64_t)b * p.OC + oc0 + o4 + k) * ohw + (int64_t)oh0 * p.OW + px0 + px;
          store_from_float(p.y, p.y_dt, off, v[k]);
        }
      }
    }
  }
}

// Store of a full step tile (128 pixels x 64 channels, 16-byte aligned rows):
// exactly kTileStores store instructions per thread and no branches, so that
// the wait for loads issued before it can be vmcnt(kTileStores).
constexpr int kTileStores = kStepPx * 64 / 4 / kStreamThreads;

template <bool PXROWS>
__device__ __forceinline__ void store_tile_full(const HaloArgs& p, const float* tile, int b, int oh0, int s, int oc0,
                                                int tid) {
  const int64_t ohw = (int64_t)p.OH * p.OW;
  const int px0 = s * kStepPx;
#pragma unroll
  for (int k = 0; k < kTileStores; ++k) {
    const int i = tid + k * kStreamThreads;
    float v[4];
    int64_t off;
    if constexpr (PXROWS) {
      const int oc = i / (kStepPx / 4);
      const int q = 4 * (i - oc * (kStepPx / 4));
      const float4 v4 = *reinterpret_cast<const float4*>(tile + oc * kTilePitchPx + q);
      v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
      off = ((int64_t)b * p.OC + oc0 + oc) * ohw + (int64_t)oh0 * p.OW + px0 + q;
    } else {
      const int px = i / 16;
      const int o4 = 4 * (i - px * 16);
      const float4 v4 = *reinterpret_cast<const float4*>(tile + px * kTilePitchOc + o4);
      v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
      off = ((int64_t)b * ohw + (int64_t)oh0 * p.OW + px0 + px) * p.OC + oc0 + o4;
    }
    store4<kEpiNone>(p.y, p.y_dt, off, v, true, p.epi);
  }
}

template <int BITS, int CC16, int STRIDE, int KHW, bool PXROWS, bool NHWC>
__global__ __launch_bounds__(kStreamThreads) void conv_stream_kernel(const HaloArgs p) {
  constexpr int T = KHW * CC16;
  static_assert(T <= 36, "decoded weights of at most 36 sub-steps stay in registers");
  constexpr int KH = KHW == 9 ? 3 : 1;
  constexpr int C8 = CC16 * 2, CP = CC16 * 16 + 8;
  constexpr int CHUNKS = (T + 3) / 4;
  constexpr int WPL = CHUNKS * BITS;
  constexpr int E = 1 << BITS;
  extern __shared__ __attribute__((aligned(16))) uint16_t ring[];
  __shared__ float cbs[64 * E];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  const int wn = wave & 1;
  const int pg = wave >> 1;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int b = tile / p.tiles_h;
  const int oh0 = (tile - b * p.tiles_h) * p.TH;
  const int P = min(p.TH, p.OH - oh0) * p.OW;
  const int nblk = (P + 31) / 32;
  const int nsteps = (nblk + 3) / 4;
  const int ih0 = oh0 * STRIDE - p.pad_h;
  const int oc0 = blockIdx.y * 64;
  const int ocl = oc0 + 32 * wn + col;
  const int nrm = p.NR - 1;
  float* otile = reinterpret_cast<float*>(ring + p.NR * p.IW_t * CP);

  stage_codebook<E>(p.cb, p.cb_dt, p.cb_rows, p.cb_size, oc0, 64, p.OC, cbs, tid, kStreamThreads);
  uint32_t wreg[WPL];
  {
    const int oc = min(ocl, p.OC - 1);
    const uint32_t* src = p.kw + ((int64_t)oc * 2 + g) * WPL;
#pragma unroll
    for (int w = 0; w < WPL; ++w) wreg[w] = src[w];
  }

  // zero padding columns of every ring row, once (row writes never touch them)
  {
    const int right = max(0, p.IW_t - p.pad_w - p.W);
    const int ncol = p.pad_w + right;
    const int zt = p.NR * ncol * C8;
    for (int t = tid; t < zt; t += kStreamThreads) {
      const int c8 = t % C8;
      const int rest = t / C8;
      const int pc = rest % ncol;
      const int slot = rest / ncol;
      const int hc = pc < p.pad_w ? pc : p.W + pc;
      *reinterpret_cast<uint4*>(ring + (slot * p.IW_t + hc) * CP + 8 * c8) = make_uint4(0, 0, 0, 0);
    }
  }

  // last band-relative input row read by step s
  auto in_hi = [&](int s) {
    const int last_px = min((s + 1) * kStepPx, P) - 1;
    return (last_px / p.OW) * STRIDE + KH - 1;
  };

  // prologue: the rows of step 0
  int have = in_hi(0);
  {
    const int tasks = row_tasks<CC16, NHWC>(p, have + 1);
    for (int t = tid; t < tasks; t += kStreamThreads) {
      uint4 v[8];
      issue_rows<CC16, NHWC>(p, b, ih0, have + 1, t, v);
      commit_rows<CC16, NHWC>(p, ring, 0, have + 1, t, v);
    }
  }
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

  // rows step s adds to the ring: (in_hi(s - 1), in_hi(s)]
  auto added = [&](int s) { return s < nsteps ? in_hi(s) - in_hi(s - 1) : 0; };

  // loads of the rows of step 1, in flight during step 0
  uint4 pf[8];
  int pf_rows = nsteps > 1 ? added(1) : 0;
  int pf_tasks = pf_rows > 0 ? row_tasks<CC16, NHWC>(p, pf_rows) : 0;
  if (tid < pf_tasks) issue_rows<CC16, NHWC>(p, b, ih0 + have + 1, pf_rows, tid, pf);

  for (int s = 0; s < nsteps; ++s) {
    // MFMA the step's blocks 4s + pg and 4s + pg + 2 out of the ring, into
    // the LDS output tile (a second block past the band is computed on a
    // clamped pixel and not stored)
    const int mb0 = 4 * s + pg;
    if (mb0 < nblk) {
      int rowoff[2][KH];  // element offsets of this lane's pixels in the rows of taps kh
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        int pix = (mb0 + 2 * q) * 32 + col;
        if (pix >= P) pix = P - 1;
        const int r = pix / p.OW;
        const int c = pix - r * p.OW;
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) rowoff[q][kh] = (((r * STRIDE + kh) & nrm) * p.IW_t + c * STRIDE) * CP + 8 * g;
      }
      // A fragment u = 2t + q: 8 channels of block q's pixel at sub-step t
      auto frag = [&](int u) {
        const int t = u >> 1, q = u & 1;
        const int khw = t / CC16;
        const int cc = t - khw * CC16;
        const int kh = (KHW == 9) ? khw / 3 : 0;
        const int kw = (KHW == 9) ? khw - 3 * kh : 0;
        return *reinterpret_cast<const half8*>(ring + rowoff[q][kh] + kw * CP + 16 * cc);
      };
      // software pipeline: DEPTH LDS reads in flight ahead of the MFMAs;
      // four independent accumulator chains (2 blocks x even/odd sub-steps)
      // keep the matrix core busy from one wave per SIMD
      constexpr int U = 2 * T;
      constexpr int DEPTH = 6;
      half8 xr[DEPTH];
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) xr[u] = frag(u);
      floatx16 acc[2][2];
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[0][0][i] = acc[0][1][i] = acc[1][0][i] = acc[1][1][i] = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = u >> 1, q = u & 1;
        acc[q][t & 1] = PXROWS ? mfma32x32x16(xr[u % DEPTH], wf[t], acc[q][t & 1])
                               : mfma32x32x16(wf[t], xr[u % DEPTH], acc[q][t & 1]);
        if (u + DEPTH < U) xr[u % DEPTH] = frag(u + DEPTH);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, DEPTH, 0);
#pragma unroll
      for (int u = 0; u < U - DEPTH; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, DEPTH, 0);
      acc[0][0] += acc[0][1];
      acc[1][0] += acc[1][1];
      write_tile<PXROWS>(otile, acc[0][0], pg, wn, col, g, scale, bv);
      if (mb0 + 2 < nblk) write_tile<PXROWS>(otile, acc[1][0], pg + 2, wn, col, g, scale, bv);
    }
    __syncthreads();
    if (s + 1 < nsteps) {
      // the rows of step s+1 were loaded before the previous step's
      // kTileStores tile stores (gfx9 retires one wave's loads and stores in
      // issue order): vmcnt(kTileStores) waits for the loads only
      static_assert(kTileStores == 8, "the wait below encodes vmcnt(8)");
      if (s > 0) __builtin_amdgcn_s_waitcnt(0x0F78);
      else __builtin_amdgcn_s_waitcnt(0x0F70);
      if (tid < pf_tasks) commit_rows<CC16, NHWC>(p, ring, have + 1, pf_rows, tid, pf);
      for (int t = kStreamThreads + tid; t < pf_tasks; t += kStreamThreads) {
        uint4 v[8];
        issue_rows<CC16, NHWC>(p, b, ih0 + have + 1, pf_rows, t, v);
        commit_rows<CC16, NHWC>(p, ring, have + 1, pf_rows, t, v);
      }
      have += pf_rows;
      // loads for step s+2, then this step's stores: both drain under step s+1
      pf_rows = added(s + 2);
      pf_tasks = pf_rows > 0 ? row_tasks<CC16, NHWC>(p, pf_rows) : 0;
      if (tid < pf_tasks) issue_rows<CC16, NHWC>(p, b, ih0 + have + 1, pf_rows, tid, pf);
      store_tile_full<PXROWS>(p, otile, b, oh0, s, oc0, tid);
    } else {
      store_tile<PXROWS>(p, otile, b, oh0, P, s, oc0, tid);
    }
    __syncthreads();
  }
}

template <int BITS, int CC16, int STRIDE, int KHW>
int launch_stream_k(const HaloArgs& p, dim3 grid, size_t lds, hipStream_t s) {
#define DIMQ_STREAM_LAUNCH(PX, NH)                                                                  \
  {                                                                                                  \
    auto k = conv_stream_kernel<BITS, CC16, STRIDE, KHW, PX, NH>;                                    \
    static const hipError_t attr =                                                                   \
        hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, \
                            150 * 1024);                                                             \
    if (attr != hipSuccess) return set_error(DIMQ_ERR_HIP, "conv2d_codebook (stream): %s", hipGetErrorString(attr)); \
    hipLaunchKernelGGL(k, grid, dim3(kStreamThreads), lds, s, p);                                    \
  }
  const bool px = p.y_layout == DIMQ_NCHW;
  const bool nh = p.x_layout == DIMQ_NHWC;
  if (px && !nh) DIMQ_STREAM_LAUNCH(true, false)
  else if (px && nh) DIMQ_STREAM_LAUNCH(true, true)
  else if (!px && !nh) DIMQ_STREAM_LAUNCH(false, false)
  else DIMQ_STREAM_LAUNCH(false, true)
#undef DIMQ_STREAM_LAUNCH
  return check_launch("conv2d_codebook (stream)");
}

// Instantiated once per bit-width (conv_stream_b{2,3,4}.hip).
template <int BITS>
int launch_stream_bits(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s) {
  const int CC16 = p.C / 16;
  if (p.KH == 3) {
    return stride == 1 ? launch_stream_k<BITS, 4, 1, 9>(p, grid, lds, s) : launch_stream_k<BITS, 4, 2, 9>(p, grid, lds, s);
  }
  if (CC16 == 4)
    return stride == 1 ? launch_stream_k<BITS, 4, 1, 1>(p, grid, lds, s) : launch_stream_k<BITS, 4, 2, 1>(p, grid, lds, s);
  return stride == 1 ? launch_stream_k<BITS, 8, 1, 1>(p, grid, lds, s) : launch_stream_k<BITS, 8, 2, 1>(p, grid, lds, s);
}

}  // namespace

int launch_stream_b2(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s);
int launch_stream_b3(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s);
int launch_stream_b4(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s);

}  // namespace dimq
