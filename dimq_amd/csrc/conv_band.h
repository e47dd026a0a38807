// Banded direct 3x3 convolution of fp16 activations, C = 64, stride 1, pad 1:
//   NCHW in and out, fp32 (the reference op's layout: BASELINE cfg2, the
//   W4A4 conv2d_lut path) or fp16 (also the next layer's W4A4 codes from the
//   quantizing epilogue);
//   NHWC in and out (ResNet-18's layer1 in channels_last), fp32 or fp16, the
//   residual and ReLU of a basic block's second conv fused.
//
// One 512-thread work-group (8 waves, two per SIMD) owns a contiguous run of
// 32-pixel blocks of one image (the image's OH*OW output pixels, flattened
// row-major, split into `parts` runs) x 64 output channels.  Blocks are
// 128-byte aligned runs of every output channel plane, so no two work-groups
// write the same cache line.
//
// Schedule of a work-group:
//   1. every thread requests its share of stage A (the halo rows of the
//      first round of blocks), then each lane loads its output channel's
//      packed weights and codebook row and decodes its 36 weight fragments
//      into VGPRs (resident for the whole work-group) while the rows land;
//   2. stage A is written into LDS as [row][col][channel] fp16 (NCHW: 8x8
//      transposes in registers; NHWC: as it is), barrier, the loads of stage B (the
//      remaining rows) go out, round 0 runs (one block-half per wave), stage B
//      is committed, barrier, round 0's blocks are stored, the remaining
//      blocks run two accumulator chains per wave.  Round 0's stores leave
//      after stage B's commit because vmcnt counts loads and stores in issue
//      order: stores issued before the commit would make its wait for stage B
//      also wait for them to complete;
//   3. each finished 32x32 block goes through a wave-private LDS area and
//      leaves as 16-byte stores: NCHW fp32 non-temporal, 8 channels x 128
//      bytes per instruction (the output is written once and never re-read
//      here, and streaming it past the L2 keeps the 25 MB fp32 output of a
//      cfg2 call from evicting the input rows other work-groups still read);
//      NHWC each pixel's 32 channels as one run of 64 (fp16) or 128 (fp32)
//      bytes, through the L2.
#pragma once

#include "conv_common.h"

namespace dimq {
namespace {

constexpr int kBandThreads = 512;
constexpr int kBandBlocksPerRound = 4;

// Geometry of one part (work-group) of an image.
struct BandPart {
  int px0, px1;     // output pixels [px0, px1) of the image
  int blk0, blk1;   // 32-pixel blocks
  int r_first;      // first output row
  int IH;           // halo rows (input rows r_first - pad .. r_last + KH - 1 - pad)
  int ra;           // halo rows of stage A (rows round 0 reads)
};

__host__ __device__ inline BandPart band_part(int nblk, int parts, int part, int OH, int OW) {
  BandPart q;
  q.blk0 = nblk * part / parts;
  q.blk1 = nblk * (part + 1) / parts;
  q.px0 = 32 * q.blk0;
  q.px1 = 32 * q.blk1 < OH * OW ? 32 * q.blk1 : OH * OW;
  q.r_first = q.px0 / OW;
  const int r_last = (q.px1 - 1) / OW;
  q.IH = r_last - q.r_first + 3;
  const int last0 = (q.px0 + 32 * kBandBlocksPerRound < q.px1 ? q.px0 + 32 * kBandBlocksPerRound : q.px1) - 1;
  const int ra = last0 / OW - q.r_first + 3;
  q.ra = ra < q.IH ? ra : q.IH;
  return q;
}

// Staging task: (channel octet co, piece lp of the stage), the stage's rows
// cut into 16-byte pieces of 8 columns, row-major (qn = W / 8 per row): eight
// 16-byte loads, one per channel of the octet.  A row outside the image
// loads a clamped piece of the plane and is written as zeros at commit
// (zeroing the registers here would make every stage wait for its loads
// before the next is issued).
struct BandTask {
  uint4 v[8];
  bool live;
};

// NCHW: lanes 8j .. 8j + 7 of a wave load 8 consecutive pieces of each
// channel of the octet, so one load instruction reads 8 channels' 128-byte
// runs.  When those runs can start on 128-byte lines (the planes are whole
// lines apart and x is line-aligned), the stage's pieces are shifted by the
// returned lead-in s0 (< 8 pieces, taken from the row before the stage and
// not committed), so that every run is one whole line: unshifted, a run of
// a row that starts mid-line spans two lines, each requested by two load
// instructions.  0 when the shift does not apply or the lead-in tasks would
// not fit one per thread.
__device__ __forceinline__ int band_shift(const HaloArgs& p, int ih0, int tasks) {
  const int s0 = (ih0 * (p.W >> 3)) & 7;  // the stage's first piece within its line (two's complement & 7: ih0 may be -1)
  const bool ok = ((p.H * p.W) & 63) == 0 && (reinterpret_cast<uintptr_t>(p.x) & 127) == 0 &&
                  tasks + 8 * s0 <= kBandThreads;
  return ok ? s0 : 0;
}

__device__ __forceinline__ void band_issue(const HaloArgs& p, int b, int ih_first, int t, int tasks, int s0,
                                           BandTask& tk) {
  const int qn = p.W >> 3;
  const int n = tasks + 8 * s0;  // with the lead-in
  const int tt = t < n ? t : 0;
  const int co = tt & 7, lp = (tt >> 3) - s0;
  const int ih = ih_first + (lp >= 0 ? lp / qn : -1);
  tk.live = t < n && lp >= 0 && ih >= 0 && ih < p.H;
  const int a = min(max(ih_first * qn + lp, 0), p.H * qn - 1);  // piece of the plane, clamped into it
  const uint16_t* src = reinterpret_cast<const uint16_t*>(p.x) + ((int64_t)b * p.C + 8 * co) * p.H * p.W + 8 * a;
#pragma unroll
  for (int c = 0; c < 8; ++c) tk.v[c] = *reinterpret_cast<const uint4*>(src + (int64_t)c * p.H * p.W);
}

// Halo row r0 + r of task t: pixels 8q .. 8q + 7 (halo columns + 1 for the
// left padding column), channels 8co .. 8co + 7, as fp16.
__device__ __forceinline__ void band_commit(const HaloArgs& p, int r0, int t, int tasks, int s0, const BandTask& tk,
                                            uint16_t* halo) {
  const int lp = (t >> 3) - s0;
  if (t >= tasks + 8 * s0 || lp < 0) return;
  constexpr int CP = 72;
  const int qn = p.W >> 3;
  const int co = t & 7, q = lp % qn, r = r0 + lp / qn;
  uint32_t in[8][4];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    in[c][0] = tk.v[c].x; in[c][1] = tk.v[c].y; in[c][2] = tk.v[c].z; in[c][3] = tk.v[c].w;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // pixel j: channels 2w, 2w+1 from half (j & 1) of word j / 2 of rows 2w, 2w+1
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const uint32_t m = tk.live ? 0xffffffffu : 0u;  // rows outside the image: zeros (a mask, not a branch)
    const uint4 o = make_uint4(perm(in[1][j >> 1], in[0][j >> 1], sel) & m, perm(in[3][j >> 1], in[2][j >> 1], sel) & m,
                               perm(in[5][j >> 1], in[4][j >> 1], sel) & m, perm(in[7][j >> 1], in[6][j >> 1], sel) & m);
    *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + 8 * q + j + 1) * CP + 8 * co]) = o;
  }
}

// NHWC input: the same tasks (channel octet co, stage row r, 8 columns q),
// each eight 16-byte loads of the octet's channels of one pixel (128-byte
// pixel runs, C = 64), written to the halo as they are: the pixel-major layout
// needs no transpose.
__device__ __forceinline__ void band_issue_nhwc(const HaloArgs& p, int b, int ih_first, int t, int tasks,
                                                BandTask& tk) {
  const int qn = p.W >> 3;
  const int tt = t < tasks ? t : 0;
  const int co = tt & 7, rest = tt >> 3, q = rest % qn, r = rest / qn;
  const int ih = ih_first + r;
  tk.live = t < tasks && ih >= 0 && ih < p.H;
  const int ihc = tk.live ? ih : 0;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(p.x) + (((int64_t)b * p.H + ihc) * p.W + 8 * q) * 64 + 8 * co;
#pragma unroll
  for (int j = 0; j < 8; ++j) tk.v[j] = *reinterpret_cast<const uint4*>(src + 64 * j);
}

__device__ __forceinline__ void band_commit_nhwc(const HaloArgs& p, int r0, int t, int tasks, const BandTask& tk,
                                                 uint16_t* halo) {
  if (t >= tasks) return;
  constexpr int CP = 72;
  const int qn = p.W >> 3;
  const int co = t & 7, rest = t >> 3, q = rest % qn, r = r0 + rest / qn;
  const uint32_t m = tk.live ? 0xffffffffu : 0u;  // rows outside the image: zeros
#pragma unroll
  for (int j = 0; j < 8; ++j)
    *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + 8 * q + j + 1) * CP + 8 * co]) =
        make_uint4(tk.v[j].x & m, tk.v[j].y & m, tk.v[j].z & m, tk.v[j].w & m);
}

// NHWC output with a residual (16-bit, in y's layout): the two 8-channel
// pieces lane l stores for a block (pixels l / 4 and l / 4 + 16, channels
// 8 (l % 4) .. + 7), requested before the round's MFMAs, so they land while
// the MFMAs run and waiting for them does not wait for the round's stores
// (vmcnt counts loads and stores in issue order).  ResNet-18 layer1 shape,
// bs128, same process: 64.6 -> 59.8 us with the remapped stores, against
// requesting them after the MFMAs.  Past the last pixel of the part the
// address is clamped (the value is not stored).
__device__ __forceinline__ void band_res_issue_nhwc(const HaloArgs& p, int b, int px1, int mb, int ocr, int lane,
                                                    ResPairs<8> (&rr)[2]) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int pix = min(mb * 32 + (lane >> 2) + 16 * it, px1 - 1);
    res_issue<8>(p.epi, ((int64_t)b * p.OH * p.OW + pix) * p.OC + min(ocr, p.OC - 32) + 8 * (lane & 3), rr[it]);
  }
}

// One 32-pixel x 32-channel block (lane (col, g) holds channel col's pixels
// 8j + 4g + i), after the epilogue (ReLU, the next layer's activation
// quantization), -> wave-private LDS, channel-major, then
//   NCHW fp32 y: non-temporal 16-byte stores of 8 whole 128-byte channel runs
//           per instruction;
//   NCHW fp16 y: 16-byte stores of 16 channels x 64 bytes (a channel's 32
//           pixels) per instruction, through the L2, which joins the two
//           64-byte halves of a line written by neighbouring blocks;
//   NHWC fp32 y: non-temporal 16-byte stores of 8 pixels' whole 128-byte runs
//           (the wave's 32 channels) per instruction: cfg2 NHWC, same
//           process, 16.89 -> 12.97 us against 32-byte pieces of 32 pixels
//           per instruction through the L2;
//   NHWC fp16 y: 16-byte stores of 16 pixels' 64-byte runs per instruction
//           (a pixel's 32 channels; the other half of its line is the other
//           channel half's wave), through the L2: the next layer reads them
//           back.  ResNet-18 layer1 shape, bs128, one conv timed alone over
//           rotated buffers: 52.6 -> 47.2 us (ReLU) non-temporal against
//           32-byte pieces of 32 pixels per instruction; in the bs128
//           forward the non-temporal form was no faster than this one.
template <int MODE, bool NHWC>
__device__ __forceinline__ void band_store(const HaloArgs& p, const floatx16& acc, int b, int px1, int mb, int col,
                                           int g, int ocr, int lane, float scale, float bv, float* park,
                                           const ResPairs<8> (&rr)[2]) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = acc[i] * scale + bv;
  if constexpr (!NHWC) epi_m<MODE, 16>(p.epi, nullptr, 0, false, v);  // NHWC: per stored piece, below
#pragma unroll
  for (int j = 0; j < 4; ++j)
    *reinterpret_cast<float4*>(park + col * kParkPitch + 8 * j + 4 * g) =
        make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  typedef float f4v __attribute__((ext_vector_type(4)));
  const int64_t ohw = (int64_t)p.OH * p.OW;
  if constexpr (NHWC) {
    // lane l: fp16 pixel l / 4 + 16 it, channels 8 (l % 4) .. + 7: an
    // instruction writes 16 pixels' 64-byte runs (the wave's 32 channels);
    // the residual pieces were requested by band_res_issue_nhwc in the same
    // layout
    if (p.y_dt == DIMQ_F16) {
      const int c8 = 8 * (lane & 3);
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int pxs = (lane >> 2) + 16 * it;
        const int pixs = mb * 32 + pxs;
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = park[(c8 + j) * kParkPitch + pxs];
        if constexpr ((MODE & kEpiRes) != 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t h = (rr[it].w[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            w[j] += p.epi.res_dt == DIMQ_F16 ? f16_bits_to_float(h) : bf16_bits_to_float(h);
          }
        }
        if constexpr ((MODE & 3) == kEpiRelu) {
#pragma unroll
          for (int j = 0; j < 8; ++j) w[j] = w[j] < 0.0f ? 0.0f : w[j];
        }
        const u32x4 h = {f16x2_rne(w[0], w[1]), f16x2_rne(w[2], w[3]), f16x2_rne(w[4], w[5]), f16x2_rne(w[6], w[7])};
        if (pixs < px1 && ocr < p.OC)
          *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.y) + ((int64_t)b * ohw + pixs) * p.OC + ocr + c8) = h;
      }
    } else {  // fp32 y (no residual: setup)
      // lane l: pixel l / 8 + 8 it, channels 4 (l % 8) .. + 3, so that an
      // instruction writes 8 pixels' whole 128-byte runs (non-temporal)
      const int c4 = 4 * (lane & 7);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int pxs = (lane >> 3) + 8 * it;
        const int pixs = mb * 32 + pxs;
        f4v w;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = park[(c4 + j) * kParkPitch + pxs];
        if constexpr ((MODE & 3) == kEpiRelu) {
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = w[j] < 0.0f ? 0.0f : w[j];
        }
        if (pixs < px1 && ocr < p.OC)
          __builtin_nontemporal_store(w, reinterpret_cast<f4v*>(reinterpret_cast<float*>(p.y) +
                                                                ((int64_t)b * ohw + pixs) * p.OC + ocr + c4));
      }
    }
  } else if (p.y_dt == DIMQ_F32) {
    const int p4 = 4 * (lane & 7);
    const int pix0 = mb * 32 + p4;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = (lane >> 3) + 8 * it;
      const f4v v = *reinterpret_cast<const f4v*>(park + c * kParkPitch + p4);
      const int oc = ocr + c;
      if (oc < p.OC && pix0 < px1)  // OH*OW % 4 == 0: a 4-pixel chunk is all in or all out
        __builtin_nontemporal_store(v, reinterpret_cast<f4v*>(reinterpret_cast<float*>(p.y) +
                                                              ((int64_t)b * p.OC + oc) * ohw + pix0));
    }
  } else {
    const int p8 = 8 * (lane & 3);
    const int pix0 = mb * 32 + p8;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int c = (lane >> 2) + 16 * it;
      const f4v a = *reinterpret_cast<const f4v*>(park + c * kParkPitch + p8);
      const f4v d = *reinterpret_cast<const f4v*>(park + c * kParkPitch + p8 + 4);
      const uint4 h = make_uint4(f16x2_rne(a[0], a[1]), f16x2_rne(a[2], a[3]), f16x2_rne(d[0], d[1]),
                                 f16x2_rne(d[2], d[3]));
      const int oc = ocr + c;
      uint16_t* dst = reinterpret_cast<uint16_t*>(p.y) + ((int64_t)b * p.OC + oc) * ohw + pix0;
      if (oc < p.OC && pix0 < px1) *reinterpret_cast<uint4*>(dst) = h;  // OH*OW % 8 == 0 (setup)
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Waves: wn = wave & 1 owns output channels oc0 + [32 wn, 32 wn + 32), wq =
// wave >> 1 the blocks blk0 + wq + 4i.  KH = KW = 3, stride 1, pad 1, C = 64.
template <int BITS, int MODE, bool NHWC>
__global__ __launch_bounds__(kBandThreads, 1) void conv_band_kernel(const HaloArgs p) {
  constexpr bool RES = NHWC && (MODE & kEpiRes) != 0;
  constexpr int T = 36, WPL = 9 * BITS, CP = 72, E = 1 << BITS;
  extern __shared__ __attribute__((aligned(16))) uint16_t halo[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 31, g = lane >> 5;
  const int wg = xcd_tile(blockIdx.x, gridDim.x);
  const int b = wg / p.parts, part = wg - b * p.parts;
  const BandPart bp = band_part(p.nblk, p.parts, part, p.OH, p.OW);
  const int ih_first = bp.r_first - p.pad_h;
  const int oc0 = blockIdx.y * 64;
  const int wn = wave & 1, wq = wave >> 1;
  const int ocl = oc0 + 32 * wn + col;
  float* park = reinterpret_cast<float*>(halo + (size_t)p.IH_t * p.IW_t * CP) + wave * kParkFloats;

  // stage A's input rows are requested first, then this lane's codebook row,
  // bias and packed weights, decoded while the rows land; stage B is requested
  // only once A is in LDS and lands while round 0 runs.  Measured: with stage B
  // in flight beside A, or the rows requested after the decode, the first MFMA
  // starts 1.5-2 us later.
  const int tA = bp.ra * p.W, tB = (bp.IH - bp.ra) * p.W;  // 8 * rows * W / 8
  BandTask tka, tkb;
  const int sA = NHWC ? 0 : band_shift(p, ih_first, tA), sB = NHWC ? 0 : band_shift(p, ih_first + bp.ra, tB);
  auto issue = [&](int ih0, int tasks, int s0, BandTask& tk) {
    if constexpr (NHWC) band_issue_nhwc(p, b, ih0, tid, tasks, tk);
    else band_issue(p, b, ih0, tid, tasks, s0, tk);
  };
  auto commit = [&](int r0, int tasks, int s0, const BandTask& tk) {
    if constexpr (NHWC) band_commit_nhwc(p, r0, tid, tasks, tk, halo);
    else band_commit(p, r0, tid, tasks, s0, tk, halo);
  };
  issue(ih_first, tA, sA, tka);
  CbRaw<E> cbraw;
  cb_row_issue<E>(p.cb, p.cb_dt, p.cb_rows == 1 ? 0 : min(ocl, p.OC - 1), p.cb_size, cbraw);
  const bool has_bias = p.bias && ocl < p.OC;
  CbRaw<1> braw{};
  if (has_bias) cb_row_issue<1>(p.bias, p.bias_dt, ocl, 1, braw);
  uint32_t wreg[WPL];
  {
    const uint32_t* src = p.kw + ((int64_t)min(ocl, p.OC - 1) * 2 + g) * WPL;
#pragma unroll
    for (int w = 0; w < WPL; ++w) wreg[w] = src[w];
  }
  float cbv[E];
  cb_row_finish<E>(cbraw, p.cb_dt, p.cb_size, cbv);
  float bvv[1];
  cb_row_finish<1>(braw, p.bias_dt, 1, bvv);
  const float bv = has_bias ? bvv[0] : 0.0f;
  CodebookRegs<BITS> cbr;
  const int e = planes_from_lds<BITS, false>(cbv, cbr, cbr);
  const float scale = ldexpf(p.acc_scale, -e);
  half8 wf[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t chunk[BITS];
#pragma unroll
    for (int w = 0; w < BITS; ++w) chunk[w] = wreg[(t >> 2) * BITS + w];
    wf[t] = decode_sub<BITS>(chunk, t & 3, cbr);
  }
  commit(0, tA, sA, tka);
  for (int t = tid; t < bp.IH * 16; t += kBandThreads) {  // left and right padding columns
    const int co = t & 7, side = (t >> 3) & 1, r = t >> 4;
    *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + (side ? p.IW_t - 1 : 0)) * CP + 8 * co]) = make_uint4(0, 0, 0, 0);
  }
  lds_barrier();
  issue(ih_first + bp.ra, tB, sB, tkb);  // in flight through round 0

  const int row_step = p.IW_t * CP;
  // nq = 1 or 2 blocks (independent accumulator chains) of this wave
  auto compute = [&](int nq, const int (&mbs)[2], floatx16 (&acc)[2]) {
    int base[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      int pix = mbs[q] * 32 + col;
      if (pix >= bp.px1) pix = bp.px0;  // rows past the part read a valid pixel and are not stored
      const int oh = pix / p.OW;
      const int ow = pix - oh * p.OW;
      base[q] = ((oh - bp.r_first) * p.IW_t + ow) * CP + 8 * g;
    }
    auto frag = [&](int t, int q) {
      const int khw = t >> 2, cc = t & 3, kh = khw / 3, kw = khw - 3 * kh;
      return *reinterpret_cast<const half8*>(halo + base[q] + kh * row_step + kw * CP + 16 * cc);
    };
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][i] = acc[1][i] = 0.0f;
    // fragment reads issued DEPTH MFMAs ahead, the order pinned: left to the
    // scheduler, the reads trail the MFMAs by one or two and every MFMA waits
    // for the LDS
    constexpr int DEPTH = 6;
    half8 xr[DEPTH];
    if (nq == 2) {
      constexpr int U = 2 * T;
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) xr[u] = frag(u >> 1, u & 1);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc[u & 1] = mfma32x32x16(xr[u % DEPTH], wf[u >> 1], acc[u & 1]);
        __builtin_amdgcn_sched_barrier(0);
        if (u + DEPTH < U) xr[u % DEPTH] = frag((u + DEPTH) >> 1, (u + DEPTH) & 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) xr[u] = frag(u, 0);
#pragma unroll
      for (int u = 0; u < T; ++u) {
        acc[0] = mfma32x32x16(xr[u % DEPTH], wf[u], acc[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (u + DEPTH < T) xr[u % DEPTH] = frag(u + DEPTH, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // round 0: one block-half per wave, reading stage A only; its stores leave after stage B's commit
  const int ocr = oc0 + 32 * wn;
  ResPairs<8> rr[2][2];  // NHWC residual pieces of this wave's (up to two) blocks
  {
    const int mb = bp.blk0 + wq;
    floatx16 acc[2];
    if (mb < bp.blk1) {
      const int mbs[2] = {mb, mb};
      if constexpr (RES) band_res_issue_nhwc(p, b, bp.px1, mb, ocr, lane, rr[0]);  // in flight through the MFMAs
      compute(1, mbs, acc);
    }
    commit(bp.ra, tB, sB, tkb);
    lds_barrier();
    if (mb < bp.blk1) band_store<MODE, NHWC>(p, acc[0], b, bp.px1, mb, col, g, ocr, lane, scale, bv, park, rr[0]);
  }
  for (int mb = bp.blk0 + wq + kBandBlocksPerRound; mb < bp.blk1; mb += 2 * kBandBlocksPerRound) {
    const bool two = mb + kBandBlocksPerRound < bp.blk1;
    const int mbs[2] = {mb, mb + kBandBlocksPerRound};
    floatx16 acc[2];
    if constexpr (RES) {  // in flight through the MFMAs
      band_res_issue_nhwc(p, b, bp.px1, mb, ocr, lane, rr[0]);
      if (two) band_res_issue_nhwc(p, b, bp.px1, mb + kBandBlocksPerRound, ocr, lane, rr[1]);
    }
    compute(two ? 2 : 1, mbs, acc);
    band_store<MODE, NHWC>(p, acc[0], b, bp.px1, mb, col, g, ocr, lane, scale, bv, park, rr[0]);
    if (two)
      band_store<MODE, NHWC>(p, acc[1], b, bp.px1, mb + kBandBlocksPerRound, col, g, ocr, lane, scale, bv, park, rr[1]);
  }
}

template <int BITS>
int launch_band_bits(const HaloArgs& p, int mode, hipStream_t s) {
  auto k = conv_band_kernel<BITS, kEpiNone, false>;
  if (p.x_layout == DIMQ_NHWC) {
    switch (mode) {
      case kEpiRelu: k = conv_band_kernel<BITS, kEpiRelu, true>; break;
      case kEpiRes: k = conv_band_kernel<BITS, kEpiRes, true>; break;
      case kEpiResRelu: k = conv_band_kernel<BITS, kEpiResRelu, true>; break;
      default: k = conv_band_kernel<BITS, kEpiNone, true>; break;
    }
  } else {
    switch (mode) {
      case kEpiRelu: k = conv_band_kernel<BITS, kEpiRelu, false>; break;
      case kEpiQuant: k = conv_band_kernel<BITS, kEpiQuant, false>; break;
      case kEpiRelu | kEpiQuant: k = conv_band_kernel<BITS, kEpiRelu | kEpiQuant, false>; break;
      default: break;
    }
  }
  const size_t lds = (size_t)p.IH_t * p.IW_t * 72 * sizeof(uint16_t) + (size_t)8 * kParkFloats * sizeof(float);
  const hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "conv2d_codebook (band): %s", hipGetErrorString(e));
  const dim3 grid(static_cast<unsigned>(p.B * p.parts), static_cast<unsigned>((p.OC + 63) / 64));
  hipLaunchKernelGGL(k, grid, dim3(kBandThreads), lds, s, p);
  return check_launch("conv2d_codebook (band)");
}

}  // namespace
}  // namespace dimq
