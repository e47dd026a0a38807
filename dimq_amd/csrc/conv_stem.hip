// Codebook Conv2d for network stems: few input channels (C <= 4), stride 2,
// 64 output channels -- ResNet-18's 7x7/2 conv on RGB (BASELINE cfg3, 8-bit
// per-output-channel codebook).  The generic implicit GEMM spends most of its
// time gathering one 3-channel pixel at a time; here the im2col operand comes
// out of LDS as one 16-byte read per MFMA k-octet.
//
// Input staging.  A band of TH output rows needs IR = 2(TH-1)+KH input rows.
// Each staged row is a list of column *pairs*: pair j holds the C channels of
// input columns 2j-padc and 2j-padc+1 as fp16 (2C <= 8 halves, zero padded to
// 16 bytes).  With padc = pad_w + (pad_w & 1), the KW-wide window of output
// column ow (input columns 2ow-pad_w ...) starts inside pair ow, so the window
// is the NP consecutive pairs ow .. ow+NP-1 (NP = ceil((KW + (pad_w&1))/2),
// rounded up to 2 or 4).  A k-octet of the MFMA operand is one pair: the k
// order of the GEMM is (kh, pair, slot) with slot = px*C + c, and slots whose
// tap kw = 2*pair + px - (pad_w&1) falls outside [0, KW) carry zero weights.
// ResNet stem: 7 kh x 4 pairs x 8 slots = K 224 for 147 real taps.
//
// Weights.  Each persistent work-group decodes the whole layer once (64 x K
// halves, looked up from the packed LSB-first stream and the codebook, each
// output channel scaled by 2^e so its largest weight lies in [2^14, 2^15))
// into LDS in MFMA fragment order; each wave then keeps all fragments in VGPRs
// (2 x KH*NP/2 x 4 registers: 112 for the 7x7 stem).
//
// MFMA v_mfma_f32_32x32x16_f16 with the weights as the A operand (rows =
// output channels) and the activations as B (columns = pixels); each wave
// takes 32-pixel blocks of the band, two at a time (4 accumulator chains).
// Epilogue through a per-wave LDS tile [32 px][64 oc] fp32, read back so that
// every store is a 16-byte piece of a contiguous run: NHWC 32 pixels x 64
// channels are 4 KB (fp16) of consecutive memory; NCHW 8-pixel runs per
// channel.  The 2^-e scale and the bias are applied at the read-back, where a
// lane's channels are fixed.
//
// Work distribution: grid = enough work-groups for two per CU; bands are split
// into 8 contiguous ranges, one per XCD (work-groups are dealt to XCDs
// round-robin), so the bands that share halo rows run on one L2.
#include "conv_common.h"

namespace dimq {

struct StemArgs {
  const void* x;
  int x_layout;  // fp16 input
  int B, C, H, W, OC, OH, OW;
  int KW, pad_h, pad_w;
  int par, padc;        // pad_w & 1, pad_w + par
  int npairs;           // OW + NP - 1 pairs per staged row
  int TH, IR;           // output rows per band, staged input rows
  int bands_h, nbands;  // bands per image, bands in total
  int per_xcd;          // bands per XCD range
  const uint8_t* w;
  int64_t w_bytes;
  int bits;
  const void* cb;
  int cb_dt, cb_rows, cb_size;
  int cb_pass;  // decode: output channels per pass whose codebook rows are staged in LDS
  const void* bias;
  int bias_dt;
  void* y;
  int y_dt, y_layout;
  Epi epi;  // fused residual / activation
};

namespace {

constexpr int kStemThreads = 256;
constexpr int kStemOutPitch = 68;  // floats per pixel row of the epilogue tile (16-byte aligned, 4 spare)
constexpr int kStemOutFloats = 32 * kStemOutPitch;

// One staged pair: input row ih, columns iw0, iw0+1 -> 8 fp16 (slot px*C+c).
__device__ __forceinline__ uint4 stem_load_pair(const StemArgs& p, int b, int ih, int iw0) {
  uint32_t h[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  if (ih >= 0 && ih < p.H) {
    const int C = p.C;
    if (p.x_layout == DIMQ_NHWC) {
      const int64_t pix = ((int64_t)b * p.H + ih) * p.W + iw0;
      if (iw0 >= 0 && iw0 + 1 < p.W && ((p.W * C) & 1) == 0) {
        // 2C halves = C dwords, 4-byte aligned (iw0 even, W*C even)
        const uint32_t* src = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(p.x) + pix * C);
        uint32_t d[4] = {0u, 0u, 0u, 0u};
        if (C == 4) {
          const uint4 t = *reinterpret_cast<const uint4*>(src);
          d[0] = t.x; d[1] = t.y; d[2] = t.z; d[3] = t.w;
        } else if (C == 3) {
          const uint3 t = *reinterpret_cast<const uint3*>(src);
          d[0] = t.x; d[1] = t.y; d[2] = t.z;
        } else if (C == 2) {
          const uint2 t = *reinterpret_cast<const uint2*>(src);
          d[0] = t.x; d[1] = t.y;
        } else {
          d[0] = src[0];
        }
        return make_uint4(d[0], d[1], d[2], d[3]);
      }
#pragma unroll
      for (int px = 0; px < 2; ++px) {
        const int iw = iw0 + px;
        if (iw < 0 || iw >= p.W) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c < C) h[px * C + c] = reinterpret_cast<const uint16_t*>(p.x)[(pix + px) * C + c];
      }
    } else {
#pragma unroll
      for (int px = 0; px < 2; ++px) {
        const int iw = iw0 + px;
        if (iw < 0 || iw >= p.W) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c < C) h[px * C + c] = reinterpret_cast<const uint16_t*>(p.x)[(((int64_t)b * C + c) * p.H + ih) * p.W + iw];
      }
    }
  }
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// Staging of NHWC input with C in {3, 4}, W and padc even (the ResNet stem):
// every pair lies wholly inside a row or wholly in the padding, and is one
// 12- or 16-byte load, so kStemPairs of a thread's pairs are requested
// without a branch, in one round trip, before any is written to LDS; `live`
// has bit u set for pair u inside the image (outside pairs re-read pixel 0 and
// are written as zeros). A whole band per thread at once (10 pairs), or
// holding it through the previous band's MFMAs, needs more VGPRs than the 7x7
// kernel has left at two waves per SIMD beside its weight fragments (it spills
// 7 and 84).
constexpr int kStemPairs = 5;
struct StemStage {
  uint4 v[kStemPairs];
  uint32_t live;
};

__device__ __forceinline__ bool stem_fast_nhwc(const StemArgs& p) {
  return p.x_layout == DIMQ_NHWC && (p.C == 3 || p.C == 4) && p.W % 2 == 0 && p.padc % 2 == 0;
}

// Pairs base + u * kStemThreads, u < kStemPairs, of the band at (b, ih0).
__device__ __forceinline__ void stem_issue_band(const StemArgs& p, int b, int ih0, int base, int units, StemStage& st) {
  st.live = 0u;
#pragma unroll
  for (int u = 0; u < kStemPairs; ++u) {
    const int i = base + u * kStemThreads;
    const int r = i / p.npairs;
    const int j = i - r * p.npairs;
    const int ih = ih0 + r, iw0 = 2 * j - p.padc;
    const bool live = i < units && ih >= 0 && ih < p.H && iw0 >= 0 && iw0 < p.W;
    const int64_t pix = live ? ((int64_t)b * p.H + ih) * p.W + iw0 : 0;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(p.x) + pix * p.C;
    if (p.C == 4) {
      st.v[u] = *reinterpret_cast<const uint4*>(src);
    } else {
      const uint3 t = *reinterpret_cast<const uint3*>(src);
      st.v[u] = make_uint4(t.x, t.y, t.z, 0u);
    }
    st.live |= live ? (1u << u) : 0u;
  }
}

__device__ __forceinline__ void stem_commit_band(int base, int units, const StemStage& st, uint4* xs) {
#pragma unroll
  for (int u = 0; u < kStemPairs; ++u) {
    const int i = base + u * kStemThreads;
    if (i >= units) break;
    const uint32_t m = (st.live >> u) & 1u ? 0xffffffffu : 0u;
    xs[i] = make_uint4(st.v[u].x & m, st.v[u].y & m, st.v[u].z & m, st.v[u].w & m);
  }
}

// The two stream bytes holding index `flat` of the LSB-first packed stream
// (the second clamped to the stream), loaded without a branch so that a
// thread's loads all go out before the first is used; stem_index_of decodes.
// (32-bit arithmetic: a stem's OC x C x KH x KW x bits is far below 2^31.)
__device__ __forceinline__ uint32_t stem_index_bytes(const StemArgs& p, int flat) {
  const int byte = (flat * p.bits) >> 3;
  const int next = byte + 1 < p.w_bytes ? byte + 1 : byte;
  return static_cast<uint32_t>(p.w[byte]) | (static_cast<uint32_t>(p.w[next]) << 8);
}

__device__ __forceinline__ int stem_index_of(const StemArgs& p, int flat, uint32_t bytes) {
  const int sh = (flat * p.bits) & 7;
  return static_cast<int>((bytes >> sh) & ((1u << p.bits) - 1u));
}

template <int KH, int NP, int MODE>
__global__ __launch_bounds__(kStemThreads, 2) void conv_stem_kernel(const StemArgs p) {
  constexpr int SPK = NP / 2;  // k16 steps per kh
  constexpr int T = KH * SPK;  // k16 steps in all
  extern __shared__ __attribute__((aligned(16))) uint4 stem_lds[];
  __shared__ float sc_s[64], bias_s[64];
  // Layout: [0, max(wdec, xs)) decoded weights, then the staged band; then 4 epilogue tiles.
  const int xs_units = p.IR * p.npairs;
  const int wdec_units = 2 * T * 64;
  uint4* xs = stem_lds;
  uint4* wdec = stem_lds;
  float* otile_all = reinterpret_cast<float*>(stem_lds + (xs_units > wdec_units ? xs_units : wdec_units));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int g = lane >> 5;
  float* otile = otile_all + wave * kStemOutFloats;

  // ---- decode the layer's weights into fragment order (thread: channel oc, pair o)
  // One item: its 8 KH taps' indices and codebook entries, read from LDS
  // (taps outside the kernel read index 0 and are zeroed by a select);
  // index_bytes(flat) returns the two stream bytes holding index `flat`,
  // entry(oc, i) entry i of oc's codebook row.
  auto decode_item = [&](int item, auto&& index_bytes, auto&& entry) {
    const int oc = item / NP;
    const int o = item - oc * NP;
    const bool ocv = oc < p.OC;
    bool tap[KH][8];
    float v[KH][8];
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int px = e >= p.C ? 1 : 0;
        const int c = e - px * p.C;
        const int kw = 2 * o + px - p.par;
        const bool in = ocv && e < 2 * p.C && kw >= 0 && kw < p.KW;
        const int flat = in ? ((oc * p.C + c) * KH + kh) * p.KW + kw : 0;
        const int i = stem_index_of(p, flat, index_bytes(flat));
        tap[kh][e] = in && i < p.cb_size;
        v[kh][e] = entry(oc, tap[kh][e] ? i : 0);
      }
    }
    float mx = 0.0f;
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[kh][e] = tap[kh][e] ? v[kh][e] : 0.0f;
        mx = fmaxf(mx, fabsf(v[kh][e]));
      }
    // the NP threads of one channel are NP consecutive lanes of one wave
#pragma unroll
    for (int d = 1; d < NP; d <<= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
    const int ex = cb_exponent(mx);
    if (o == 0) {
      sc_s[oc] = ldexpf(1.0f, -ex);
      bias_s[oc] = (ocv && p.bias) ? load_as_float(p.bias, p.bias_dt, oc) : 0.0f;
    }
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = float_to_f16_bits(ldexpf(v[kh][e], ex));
      const int t = kh * SPK + (o >> 1);
      const int l = (oc & 31) + 32 * (o & 1);
      wdec[((oc >> 5) * T + t) * 64 + l] =
          make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
  };
  {
    // The packed stream and, p.cb_pass output channels at a time, their
    // codebook rows are first copied into LDS behind the decode area with
    // coalesced 16-byte loads (all of a thread's loads of a batch in flight);
    // the items then gather from LDS.  Gathered from global memory, each
    // wave-wide load of 64 lanes' indices or entries touched ~30 cache lines
    // (ResNet-18 stem: ~17.6 us of decode per work-group).
    uint8_t* wst = reinterpret_cast<uint8_t*>(stem_lds + wdec_units);
    const int wb = static_cast<int>(p.w_bytes);
    float* cbs = reinterpret_cast<float*>(wst + ((wb + 15) & ~15));
    const int nfull = wb >> 4;
    if (nfull > 0) {
      for (int c0 = 0; c0 < nfull; c0 += kStemThreads * 4) {
        uint4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int ci = c0 + j * kStemThreads + tid;
          t[j] = *reinterpret_cast<const uint4*>(p.w + 16 * (ci < nfull ? ci : nfull - 1));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int ci = c0 + j * kStemThreads + tid;
          if (ci < nfull) *reinterpret_cast<uint4*>(wst + 16 * ci) = t[j];
        }
      }
    }
    if (tid < (wb & 15)) wst[(nfull << 4) + tid] = p.w[(nfull << 4) + tid];
    const bool f32 = p.cb_dt == DIMQ_F32;
    const int per = f32 ? 4 : 8;  // entries per 16-byte chunk
    const int rows = p.cb_rows == 1 ? 1 : p.cb_pass;
    const int dsz = f32 ? 4 : 2;
    for (int r0 = 0; r0 < 64; r0 += p.cb_pass) {
      const int nrows = p.cb_rows == 1 ? 1 : (r0 + rows <= p.cb_rows ? rows : p.cb_rows - r0);
      if (nrows > 0) {
        const int nch = nrows * p.cb_size / per;
        const uint8_t* src = static_cast<const uint8_t*>(p.cb) + (size_t)(p.cb_rows == 1 ? 0 : r0) * p.cb_size * dsz;
        for (int c0 = 0; c0 < nch; c0 += kStemThreads * 8) {
          uint4 t[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int ci = c0 + j * kStemThreads + tid;
            t[j] = *reinterpret_cast<const uint4*>(src + 16 * (ci < nch ? ci : nch - 1));
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int ci = c0 + j * kStemThreads + tid;
            if (ci >= nch) continue;
            if (f32) {
              *reinterpret_cast<uint4*>(cbs + 4 * ci) = t[j];
            } else {
              const uint32_t u[4] = {t[j].x, t[j].y, t[j].z, t[j].w};
              float f[8];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const bool h16 = p.cb_dt == DIMQ_F16;
                f[2 * q] = h16 ? f16_bits_to_float(u[q] & 0xffffu) : bf16_bits_to_float(u[q] & 0xffffu);
                f[2 * q + 1] = h16 ? f16_bits_to_float(u[q] >> 16) : bf16_bits_to_float(u[q] >> 16);
              }
              *reinterpret_cast<float4*>(cbs + 8 * ci) = make_float4(f[0], f[1], f[2], f[3]);
              *reinterpret_cast<float4*>(cbs + 8 * ci + 4) = make_float4(f[4], f[5], f[6], f[7]);
            }
          }
        }
      }
      __syncthreads();  // stream and rows staged
      for (int item = tid; item < 64 * NP; item += kStemThreads) {
        const int oc = item / NP;
        if (oc < r0 || oc >= r0 + p.cb_pass) continue;  // whole channels: NP consecutive lanes
        decode_item(
            item,
            [&](int flat) {
              const int byte = (flat * p.bits) >> 3;
              const int next = byte + 1 < wb ? byte + 1 : byte;
              return static_cast<uint32_t>(wst[byte]) | (static_cast<uint32_t>(wst[next]) << 8);
            },
            [&](int ch, int i) { return cbs[(p.cb_rows == 1 ? 0 : ch - r0) * p.cb_size + i]; });
      }
      __syncthreads();  // the next pass overwrites the rows
    }
  }
  __syncthreads();
  half8 wf[2][T];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int t = 0; t < T; ++t) wf[nb][t] = __builtin_bit_cast(half8, wdec[(nb * T + t) * 64 + lane]);
  // read-back channels of this lane: NHWC chunk lane%8 (8 channels), NCHW channel `lane`
  const bool nhwc = p.y_layout == DIMQ_NHWC;
  float rsc[8], rbs[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int oc = nhwc ? (lane & 7) * 8 + u : lane;
    rsc[u] = sc_s[oc];
    rbs[u] = bias_s[oc];
  }
  __syncthreads();  // the band staging below overwrites the decode area

  // ---- bands of this work-group: XCD x owns bands [x*per, (x+1)*per)
  const int gx = gridDim.x / 8;
  const int xcd = blockIdx.x % 8;
  const int local = blockIdx.x / 8;
  const int band_end = min((xcd + 1) * p.per_xcd, p.nbands);
  const int64_t ohw = (int64_t)p.OH * p.OW;
  const bool vec_nchw = (ohw % 8 == 0) && (p.OW % 8 == 0 || p.TH * p.OW % 8 == 0);

  const bool fast = stem_fast_nhwc(p);
  for (int band = xcd * p.per_xcd + local; band < band_end; band += gx) {
    const int b = band / p.bands_h;
    const int oh0 = (band - b * p.bands_h) * p.TH;
    const int ih0 = 2 * oh0 - p.pad_h;
    if (fast) {
      for (int base = tid; base < xs_units; base += kStemPairs * kStemThreads) {
        StemStage stage;
        stem_issue_band(p, b, ih0, base, xs_units, stage);
        stem_commit_band(base, xs_units, stage, xs);
      }
      __syncthreads();
    } else {
      // stage IR rows x npairs pairs, four loads in flight per thread
      for (int base = tid; base < xs_units; base += 4 * kStemThreads) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = base + u * kStemThreads;
          v[u] = make_uint4(0u, 0u, 0u, 0u);
          if (i < xs_units) {
            const int r = i / p.npairs;
            const int j = i - r * p.npairs;
            v[u] = stem_load_pair(p, b, ih0 + r, 2 * j - p.padc);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = base + u * kStemThreads;
          if (i < xs_units) xs[i] = v[u];
        }
      }
      __syncthreads();
    }

    const int P = min(p.TH, p.OH - oh0) * p.OW;
    const int nblk = (P + 31) / 32;
    const int pmax = p.TH * p.OW - 1;
    for (int blk0 = wave; blk0 < nblk; blk0 += 8) {
      const int blk1 = blk0 + 4;
      const bool two = blk1 < nblk;
      floatx16 acc[2][2];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[q][nb][r] = 0.0f;
      int abase[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int pix = min((q == 0 ? blk0 : blk1) * 32 + col, pmax);
        const int ro = pix / p.OW;
        const int ow = pix - ro * p.OW;
        abase[q] = 2 * ro * p.npairs + ow + g;
      }
      if (two) {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
          for (int s = 0; s < SPK; ++s) {
            const half8 a0 = __builtin_bit_cast(half8, xs[abase[0] + kh * p.npairs + 2 * s]);
            const half8 a1 = __builtin_bit_cast(half8, xs[abase[1] + kh * p.npairs + 2 * s]);
            const int t = kh * SPK + s;
            acc[0][0] = mfma32x32x16(wf[0][t], a0, acc[0][0]);
            acc[0][1] = mfma32x32x16(wf[1][t], a0, acc[0][1]);
            acc[1][0] = mfma32x32x16(wf[0][t], a1, acc[1][0]);
            acc[1][1] = mfma32x32x16(wf[1][t], a1, acc[1][1]);
          }
        }
      } else {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
          for (int s = 0; s < SPK; ++s) {
            const half8 a0 = __builtin_bit_cast(half8, xs[abase[0] + kh * p.npairs + 2 * s]);
            const int t = kh * SPK + s;
            acc[0][0] = mfma32x32x16(wf[0][t], a0, acc[0][0]);
            acc[0][1] = mfma32x32x16(wf[1][t], a0, acc[0][1]);
          }
        }
      }

      // ---- epilogue of the one or two blocks, each through the wave's tile
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (q == 1 && !two) break;
        const int pb = (q == 0 ? blk0 : blk1) * 32;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            *reinterpret_cast<float4*>(otile + col * kStemOutPitch + nb * 32 + 8 * jj + 4 * g) =
                make_float4(acc[q][nb][4 * jj], acc[q][nb][4 * jj + 1], acc[q][nb][4 * jj + 2],
                            acc[q][nb][4 * jj + 3]);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (nhwc) {
          // 32 pixels x 8 chunks of 8 channels; lane: chunk lane%8, pixels lane/8 + 8*it
          const int64_t gp0 = ((int64_t)b * p.OH + oh0) * p.OW + pb;
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int px = (lane >> 3) + 8 * it;
            const int ch = lane & 7;
            const float4 u0 = *reinterpret_cast<const float4*>(otile + px * kStemOutPitch + ch * 8);
            const float4 u1 = *reinterpret_cast<const float4*>(otile + px * kStemOutPitch + ch * 8 + 4);
            float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = v[u] * rsc[u] + rbs[u];
            if (pb + px >= P || ch * 8 >= p.OC) continue;
            const int64_t off = (gp0 + px) * p.OC + ch * 8;
            epi_m<MODE, 8>(p.epi, nullptr, off, true, v);
            if (p.y_dt == DIMQ_F32) {
              float* yp = reinterpret_cast<float*>(p.y) + off;
              *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
              *reinterpret_cast<float4*>(yp + 4) = make_float4(v[4], v[5], v[6], v[7]);
            } else {
              uint32_t h[8];
#pragma unroll
              for (int u = 0; u < 8; ++u)
                h[u] = p.y_dt == DIMQ_F16 ? float_to_f16_bits(v[u]) : float_to_bf16_bits(v[u]);
              *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.y) + off) =
                  make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
            }
          }
        } else {
          // channel `lane`, 4 runs of 8 pixels
          const int64_t cbase = ((int64_t)b * p.OC + lane) * ohw + (int64_t)oh0 * p.OW + pb;
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = otile[(8 * it + u) * kStemOutPitch + lane] * rsc[0] + rbs[0];
            if (lane >= p.OC) continue;
            const int px0 = 8 * it;
            if (vec_nchw && pb + px0 + 8 <= P) {
              epi_m<MODE, 8>(p.epi, nullptr, cbase + px0, true, v);
              if (p.y_dt == DIMQ_F32) {
                float* yp = reinterpret_cast<float*>(p.y) + cbase + px0;
                *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
                *reinterpret_cast<float4*>(yp + 4) = make_float4(v[4], v[5], v[6], v[7]);
              } else {
                uint32_t h[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                  h[u] = p.y_dt == DIMQ_F16 ? float_to_f16_bits(v[u]) : float_to_bf16_bits(v[u]);
                *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p.y) + cbase + px0) =
                    make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
              }
            } else {
#pragma unroll
              for (int u = 0; u < 8; ++u)
                if (pb + px0 + u < P) store_from_float(p.y, p.y_dt, cbase + px0 + u, epi1_m<MODE>(p.epi, cbase + px0 + u, v[u]));
            }
          }
        }
      }
    }
    __syncthreads();  // all waves are done with the staged band
  }
}

int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// NP the kernel instantiation uses for a kernel width, or 0.
int stem_np(int64_t KW, int64_t pw) {
  const int64_t np = (KW + (pw & 1) + 1) / 2;
  return np <= 2 ? 2 : (np <= 4 ? 4 : 0);
}

constexpr int kStemMaxTH = 8;
constexpr int64_t kStemStageBytes = 40 * 1024;  // staged band

int64_t stem_rows(int64_t KH, int64_t OH, int64_t OW, int np) {
  const int64_t npairs = OW + np - 1;
  for (int64_t th = std::min<int64_t>(kStemMaxTH, OH); th >= 1; --th)
    if ((2 * (th - 1) + KH) * npairs * 16 <= kStemStageBytes) return th;
  return 0;
}

// Dynamic LDS of a band: the staged input rows or the decode area, then the
// four epilogue tiles.
size_t stem_band_lds(int64_t KH, int64_t OH, int64_t OW, int np) {
  const int64_t th = stem_rows(KH, OH, OW, np);
  const int64_t units = std::max<int64_t>((2 * (th - 1) + KH) * (OW + np - 1), KH * np * 64);
  return (size_t)units * 16 + 4 * kStemOutFloats * sizeof(float);
}

// Output channels per decode pass: the packed stream and the codebook rows of
// that many channels are staged behind the decode area (2 T 64 16-byte
// units), the most that fit in the band's LDS or in 80 KB (two work-groups
// per CU); *lds gets the LDS bytes the launch needs.  0: the stream or the
// codebook is not 16-byte aligned, or a row is not whole 16-byte chunks.
int stem_cb_pass(int64_t KH, int np, size_t band_lds, const void* w, int64_t w_bytes, const void* cb, int cb_dtype,
                 int64_t cb_rows, int64_t cb_size, size_t* lds) {
  const int64_t esz = cb_dtype == DIMQ_F32 ? 4 : (cb_dtype == DIMQ_F16 || cb_dtype == DIMQ_BF16 ? 2 : 0);
  if (esz == 0 || !aligned(w, 16) || !aligned(cb, 16) || cb_size < 1 || (cb_size * esz) % 16 != 0) return 0;
  const size_t limit = std::max<size_t>(band_lds, 80 * 1024);
  for (int pass = 64; pass >= 8; pass /= 2) {
    const size_t rows = cb_rows == 1 ? 1 : (size_t)pass;
    const size_t need = (size_t)KH * np * 64 * 16 + (((size_t)w_bytes + 15) & ~(size_t)15) + rows * cb_size * 4;
    if (need <= limit) {
      *lds = std::max(band_lds, need);
      return pass;
    }
  }
  return 0;
}

}  // namespace

bool stem_eligible(int64_t C, int64_t OC, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t pw,
                   int64_t dh, int64_t dw, int64_t groups, int64_t OH, int64_t OW, int bits, int x_dtype,
                   int y_dtype, const void* x, const void* y, int epi_mode_, const void* w, int64_t w_bytes,
                   const void* cb, int cb_dtype, int64_t cb_rows, int64_t cb_size) {
  if (epi_mode_ != kEpiNone && epi_mode_ != kEpiRelu) return false;  // other epilogues: generic kernel
  if (x_dtype != DIMQ_F16) return false;  // fp16 staging (other dtypes: the guarded generic kernel)
  if (groups != 1 || C < 1 || C > 4 || OC < 1 || OC > 64 || OC % 8 != 0) return false;
  if (sh != 2 || sw != 2 || dh != 1 || dw != 1) return false;
  if (bits < 2 || bits > 8) return false;
  const int np = stem_np(KW, pw);
  if (!((KH == 7 && np == 4) || (KH == 3 && np == 2))) return false;
  if (!aligned(x, 4) || !aligned(y, 16)) return false;
  (void)y_dtype;
  if (stem_rows(KH, OH, OW, np) <= 0) return false;
  size_t lds = 0;
  return stem_cb_pass(KH, np, stem_band_lds(KH, OH, OW, np), w, w_bytes, cb, cb_dtype, cb_rows, cb_size, &lds) > 0;
}

int launch_conv_stem(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                     const uint8_t* w, int64_t w_bytes, int bits, const void* cb, int cb_dtype, int64_t cb_rows,
                     int64_t cb_size, const void* bias, int bias_dtype, int64_t OC, int64_t KH, int64_t KW,
                     int64_t ph, int64_t pw, int64_t OH, int64_t OW, void* y, int y_dtype, int y_layout,
                     const Epi& epi, hipStream_t s) {
  const int np = stem_np(KW, pw);
  StemArgs p{};
  p.x = x;
  if (x_dtype != DIMQ_F16) return set_error(DIMQ_ERR_UNSUPPORTED, "conv stem kernel takes fp16 activations");
  p.x_layout = x_layout;
  p.B = (int)B; p.C = (int)C; p.H = (int)H; p.W = (int)W;
  p.OC = (int)OC; p.OH = (int)OH; p.OW = (int)OW;
  p.KW = (int)KW;
  p.pad_h = (int)ph;
  p.pad_w = (int)pw;
  p.par = (int)(pw & 1);
  p.padc = p.pad_w + p.par;
  p.npairs = (int)(OW + np - 1);
  p.TH = (int)stem_rows(KH, OH, OW, np);
  p.IR = (int)(2 * (p.TH - 1) + KH);
  p.bands_h = (int)((OH + p.TH - 1) / p.TH);
  const int64_t nbands = B * p.bands_h;
  DIMQ_CHECK(nbands < (1LL << 31) && (int64_t)p.IR * p.npairs < (1 << 30), "conv2d_codebook (stem): too many bands");
  p.nbands = (int)nbands;
  p.w = w;
  p.w_bytes = w_bytes;
  p.bits = bits;
  p.cb = cb;
  p.cb_dt = cb_dtype;
  p.cb_rows = (int)cb_rows;
  p.cb_size = (int)cb_size;
  p.bias = bias;
  p.bias_dt = bias_dtype;
  p.y = y;
  p.y_dt = y_dtype;
  p.y_layout = y_layout;
  p.epi = epi;

  // two work-groups per CU, as many rounds as needed, whole multiple of 8 work-groups
  const int64_t slots = 2LL * device_cu_count();
  const int64_t rounds = (nbands + slots - 1) / slots;
  int64_t G = (nbands + rounds - 1) / rounds;
  G = std::max<int64_t>(8, (G + 7) / 8 * 8);
  p.per_xcd = (int)((nbands + 7) / 8);

  size_t lds = 0;
  p.cb_pass = stem_cb_pass(KH, np, stem_band_lds(KH, OH, OW, np), w, w_bytes, cb, cb_dtype, cb_rows, cb_size, &lds);
  if (p.cb_pass == 0) return set_error(DIMQ_ERR_UNSUPPORTED, "conv stem kernel: codebook or stream not stageable");
  const bool relu = epi_mode(epi) == kEpiRelu;
  auto k = KH == 7 ? (relu ? conv_stem_kernel<7, 4, kEpiRelu> : conv_stem_kernel<7, 4, kEpiNone>)
                   : (relu ? conv_stem_kernel<3, 2, kEpiRelu> : conv_stem_kernel<3, 2, kEpiNone>);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "conv2d_codebook (stem): %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(k, dim3((unsigned)G), dim3(kStemThreads), lds, s, p);
  return check_launch("conv2d_codebook (stem)");
}

}  // namespace dimq
