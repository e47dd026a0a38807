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
// Weights arrive in a "kernel layout" (dimq_conv2d_prepare_weight): for every
// output channel n and lane group g, the b-bit indices of the sub-steps
// t = (kh, kw, 32-channel chunk) x 8 channels, ordered so that the v_perm
// decode of decode.h yields channels in natural order.  Each lane keeps its
// rows' packed indices and codebook byte planes in VGPRs for the whole tile.
//
// The MFMA computes D[oc][pixel] (weights as the A operand), so lane l ends
// with 4 output channels of pixel l%16 and the fp32 NCHW stores of 16 lanes
// are 64-byte contiguous runs.
#include "decode.h"

#include <algorithm>

namespace dimq {
namespace {

struct HaloArgs {
  const void* x;
  int x_dt, x_layout;
  int B, C, H, W, OC, OH, OW;
  int KH, KW, pad_h, pad_w;
  int TH;              // output rows per tile
  int IH_t, IW_t, CP;  // halo tile rows, cols, channel pitch (fp16 elements)
  int tiles_h;         // ceil(OH / TH)
  const uint32_t* kw;  // kernel-layout weights
  int words_per_lane;  // ceil(T/4) * BITS
  const void* cb;
  int cb_dt, cb_rows, cb_size;
  const void* bias;
  int bias_dt;
  void* y;
  int y_dt, y_layout;
};

template <int BITS>
__device__ __forceinline__ void load_cb_row(const HaloArgs& p, int row, bool valid, CodebookRegs<BITS>& cb, int& e) {
  constexpr int E = 1 << BITS;
  float c[E];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    c[j] = (valid && j < p.cb_size) ? load_as_float(p.cb, p.cb_dt, (int64_t)row * p.cb_size + j) : 0.0f;
    mx = fmaxf(mx, fabsf(c[j]));
  }
  e = cb_exponent(mx);
  uint32_t h16[E];
#pragma unroll
  for (int j = 0; j < E; ++j) h16[j] = float_to_f16_bits(ldexpf(c[j], e));
  set_planes<BITS>(cb, h16);
}

__device__ __forceinline__ uint32_t to_f16_bits(uint32_t raw, int dt) {
  return dt == DIMQ_F16 ? raw : float_to_f16_bits(bf16_bits_to_float(raw));
}

// T = KH*KW*CC sub-steps of 32 channels; CC = C / 32.
template <int BITS, int CC, int STRIDE, int KHW>
__global__ __launch_bounds__(256) void conv_halo_kernel(const HaloArgs p) {
  constexpr int T = KHW * CC;
  constexpr int CHUNKS = (T + 3) / 4;
  constexpr int WPL = CHUNKS * BITS;  // packed words per lane per output row
  constexpr int NB = 4;               // 64 output channels per work-group
  constexpr int MBW = 4;              // m-blocks (16 pixels) per wave, at most
  extern __shared__ __attribute__((aligned(16))) uint16_t halo[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int tile = blockIdx.x;
  const int b = tile / p.tiles_h;
  const int oh0 = (tile - b * p.tiles_h) * p.TH;
  const int oc0 = blockIdx.y * 64;
  const int C = CC * 32;

  // ---- stage the input halo: rows ih = oh0*S - pad + r, cols iw = -pad + c
  const int ih0 = oh0 * STRIDE - p.pad_h;
  const int rows_valid = p.IH_t;
  if (p.x_layout == DIMQ_NCHW) {
    // task = (channel pair, halo row, 8 halo columns)
    const int cg = (p.IW_t + 7) / 8;
    const int tasks = (C / 2) * rows_valid * cg;
    for (int t = tid; t < tasks; t += 256) {
      const int c8 = t % cg;
      const int rest = t / cg;
      const int r = rest % rows_valid;
      const int c2 = rest / rows_valid;
      const int ih = ih0 + r;
      const int cbase = c8 * 8;
      uint32_t v0[8], v1[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int iw = cbase + j - p.pad_w;
        uint32_t a = 0, bb = 0;
        if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
          const int64_t off = (((int64_t)b * p.C + 2 * c2) * p.H + ih) * p.W + iw;
          a = reinterpret_cast<const uint16_t*>(p.x)[off];
          bb = reinterpret_cast<const uint16_t*>(p.x)[off + (int64_t)p.H * p.W];
          a = to_f16_bits(a, p.x_dt);
          bb = to_f16_bits(bb, p.x_dt);
        }
        v0[j] = a;
        v1[j] = bb;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int hc = cbase + j;
        if (hc < p.IW_t)
          *reinterpret_cast<uint32_t*>(&halo[(r * p.IW_t + hc) * p.CP + 2 * c2]) = v0[j] | (v1[j] << 16);
      }
    }
  } else {
    // NHWC: task = (halo pixel, 8 channels) -> one 16-byte load, one 16-byte LDS store
    const int tasks = rows_valid * p.IW_t * (C / 8);
    for (int t = tid; t < tasks; t += 256) {
      const int c8 = t % (C / 8);
      const int pix = t / (C / 8);
      const int r = pix / p.IW_t;
      const int hc = pix - r * p.IW_t;
      const int ih = ih0 + r;
      const int iw = hc - p.pad_w;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t off = (((int64_t)b * p.H + ih) * p.W + iw) * p.C + 8 * c8;
        v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.x) + off);
        if (p.x_dt != DIMQ_F16) {
          uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
            w4[q] = to_f16_bits(w4[q] & 0xffffu, p.x_dt) | (to_f16_bits(w4[q] >> 16, p.x_dt) << 16);
          v = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
      }
      *reinterpret_cast<uint4*>(&halo[(r * p.IW_t + hc) * p.CP + 8 * c8]) = v;
    }
  }

  // ---- weights and codebooks for this lane's 4 output rows
  uint32_t wreg[NB][WPL];
  CodebookRegs<BITS> cbr[NB];
  float scale[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int oc = oc0 + nb * 16 + col;
    const bool valid = oc < p.OC;
    const uint32_t* src = p.kw + ((int64_t)oc * 4 + g) * WPL;
#pragma unroll
    for (int w = 0; w < WPL; ++w) wreg[nb][w] = valid ? src[w] : 0u;
    int e;
    load_cb_row<BITS>(p, p.cb_rows == 1 ? 0 : oc, valid, cbr[nb], e);
    scale[nb] = ldexpf(1.0f, -e);
  }

  // ---- this lane's pixels: m-blocks mb = wave + 4*q
  const int P = min(p.TH, p.OH - oh0) * p.OW;
  const int MBT = (P + 15) / 16;
  int base[MBW];
#pragma unroll
  for (int q = 0; q < MBW; ++q) {
    const int mb = wave + 4 * q;
    int pix = mb * 16 + col;
    if (pix >= P) pix = 0;
    const int r = pix / p.OW;
    const int c = pix - r * p.OW;
    base[q] = ((r * STRIDE) * p.IW_t + c * STRIDE) * p.CP + 8 * g;
  }
  __syncthreads();

  floatx4 acc[MBW][NB];
#pragma unroll
  for (int q = 0; q < MBW; ++q)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[q][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int khw = t / CC;
    const int cc = t - khw * CC;
    const int kh = (KHW == 9) ? khw / 3 : 0;
    const int kw = (KHW == 9) ? khw - 3 * kh : 0;
    const int koff = (kh * p.IW_t + kw) * p.CP + 32 * cc;
    half8 wf[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      uint32_t chunk[BITS];
#pragma unroll
      for (int w = 0; w < BITS; ++w) chunk[w] = wreg[nb][(t >> 2) * BITS + w];
      wf[nb] = decode_sub<BITS>(chunk, t & 3, cbr[nb]);
    }
#pragma unroll
    for (int q = 0; q < MBW; ++q) {
      if (wave + 4 * q < MBT) {
        const half8 xf = *reinterpret_cast<const half8*>(&halo[base[q] + koff]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[q][nb] = mfma16x16x32(wf[nb], xf, acc[q][nb]);
      }
    }
  }

  // ---- epilogue: lane holds D[oc = nb*16 + 4g + i][pixel = mb*16 + col]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int orow = 4 * g + i;
      const float sc = __shfl(scale[nb], orow, 64);
      const int oc = oc0 + nb * 16 + orow;
      if (oc >= p.OC) continue;
      const float bv = p.bias ? load_as_float(p.bias, p.bias_dt, oc) : 0.0f;
#pragma unroll
      for (int q = 0; q < MBW; ++q) {
        const int mb = wave + 4 * q;
        const int pix = mb * 16 + col;
        if (mb < MBT && pix < P) {
          const int r = pix / p.OW;
          const int c = pix - r * p.OW;
          const int oh = oh0 + r;
          const int64_t off = p.y_layout == DIMQ_NCHW
                                  ? (((int64_t)b * p.OC + oc) * p.OH + oh) * p.OW + c
                                  : (((int64_t)b * p.OH + oh) * p.OW + c) * p.OC + oc;
          store_from_float(p.y, p.y_dt, off, acc[q][nb][i] * sc + bv);
        }
      }
    }
  }
}

// ---- weight preparation: conv_kcrs b-bit stream -> kernel layout
// out[((n*4 + g)*CHUNKS + chunk)*BITS + w]: sub-steps t = 4*chunk + s, slot j
// holds channel c = 32*(t % CC) + 8*g + j at (kh, kw) = divmod(t / CC, KW),
// at the field position that decode_sub<BITS>(chunk, s) reads as slot j.
template <int BITS>
__device__ __forceinline__ int field_of(int s, int j) {
  if constexpr (BITS == 4) {
    return 8 * s + (j < 4 ? 2 * j : 2 * (j - 4) + 1);  // nibble position in the chunk
  } else if constexpr (BITS == 2) {
    const int h = s & 1, u = s >> 1;
    return 16 * u + (j < 4 ? 4 * j + 2 * h : 4 * (j - 4) + 2 * h + 1);
  } else {
    return 8 * s + j;
  }
}

template <int BITS>
__global__ void prepare_kernel(const uint8_t* __restrict__ src, int OC, int C, int KH, int KW, int CC, int T,
                               int chunks, uint32_t* __restrict__ out) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)OC * 4 * chunks;
  if (id >= total) return;
  const int chunk = static_cast<int>(id % chunks);
  const int g = static_cast<int>((id / chunks) % 4);
  const int n = static_cast<int>(id / (4 * chunks));
  uint32_t words[BITS];
#pragma unroll
  for (int w = 0; w < BITS; ++w) words[w] = 0;
  for (int s = 0; s < 4; ++s) {
    const int t = 4 * chunk + s;
    if (t >= T) break;
    const int khw = t / CC;
    const int cc = t - khw * CC;
    const int kh = khw / KW;
    const int kw = khw - kh * KW;
    for (int j = 0; j < 8; ++j) {
      const int c = 32 * cc + 8 * g + j;
      const int64_t i = (((int64_t)n * C + c) * KH + kh) * KW + kw;
      const int64_t bit = i * BITS;
      uint32_t v = src[bit >> 3] >> (bit & 7);
      if ((bit & 7) + BITS > 8) v |= (uint32_t)src[(bit >> 3) + 1] << (8 - (bit & 7));
      v &= (1u << BITS) - 1u;
      const int f = field_of<BITS>(s, j) * BITS;
      words[f >> 5] |= v << (f & 31);
      if ((f & 31) + BITS > 32) words[(f >> 5) + 1] |= v >> (32 - (f & 31));
    }
  }
  uint32_t* dst = out + id * BITS;
#pragma unroll
  for (int w = 0; w < BITS; ++w) dst[w] = words[w];
}

template <int BITS, int CC, int STRIDE>
int launch_halo(const HaloArgs& p, hipStream_t s) {
  const size_t lds = (size_t)p.IH_t * p.IW_t * p.CP * sizeof(uint16_t);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles_h), static_cast<unsigned>((p.OC + 63) / 64));
  if (p.KH == 3) {
    hipLaunchKernelGGL((conv_halo_kernel<BITS, CC, STRIDE, 9>), grid, dim3(256), lds, s, p);
  } else {
    hipLaunchKernelGGL((conv_halo_kernel<BITS, CC, STRIDE, 1>), grid, dim3(256), lds, s, p);
  }
  return check_launch("conv2d_codebook (halo)");
}

template <int BITS>
int launch_halo_cc(const HaloArgs& p, int CC, int stride, hipStream_t s) {
  if (CC == 2) return stride == 1 ? launch_halo<BITS, 2, 1>(p, s) : launch_halo<BITS, 2, 2>(p, s);
  return stride == 1 ? launch_halo<BITS, 4, 1>(p, s) : launch_halo<BITS, 4, 2>(p, s);
}

}  // namespace

int64_t halo_prepared_words(int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits) {
  const int64_t T = KH * KW * (C / 32);
  return OC * 4 * ((T + 3) / 4) * bits;
}

// Output rows per tile: at most 256 pixels (16 m-blocks over 4 waves) and a
// halo tile of at most 64 KiB of LDS.  0 = the shape does not fit.
int64_t halo_tile_rows(int64_t C, int64_t KH, int64_t KW, int64_t stride, int64_t OH, int64_t OW) {
  if (OW < 1 || OW > 256 || OH < 1) return 0;
  for (int64_t th = std::min<int64_t>(OH, 256 / OW); th >= 1; --th) {
    const int64_t lds = ((th - 1) * stride + KH) * ((OW - 1) * stride + KW) * (C + 8) * 2;
    if (lds <= 64 * 1024) return th;
  }
  return 0;
}

// Weight shapes the kernel layout (and the halo kernel) support.
bool halo_weight_supported(int64_t C, int64_t KH, int64_t KW, int bits) {
  return (bits == 2 || bits == 3 || bits == 4) && (C == 64 || C == 128) &&
         ((KH == 3 && KW == 3) || (KH == 1 && KW == 1));
}

// Full eligibility of a conv call for the halo kernel.
bool halo_eligible(int64_t C, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t dh, int64_t dw,
                   int64_t groups, int64_t OH, int64_t OW, int bits, int x_dtype) {
  if (!halo_weight_supported(C, KH, KW, bits)) return false;
  if (!(x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16)) return false;
  if (groups != 1 || dh != 1 || dw != 1 || sh != sw || (sh != 1 && sh != 2)) return false;
  return halo_tile_rows(C, KH, KW, sh, OH, OW) > 0;
}

int launch_conv_halo(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                     const uint32_t* kw, int bits, const void* cb, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                     const void* bias, int bias_dtype, int64_t OC, int64_t KH, int64_t KW, int64_t stride,
                     int64_t ph, int64_t pw, int64_t OH, int64_t OW, void* y, int y_dtype, int y_layout,
                     hipStream_t s) {
  HaloArgs p{};
  p.x = x;
  p.x_dt = x_dtype;
  p.x_layout = x_layout;
  p.B = (int)B;
  p.C = (int)C;
  p.H = (int)H;
  p.W = (int)W;
  p.OC = (int)OC;
  p.OH = (int)OH;
  p.OW = (int)OW;
  p.KH = (int)KH;
  p.KW = (int)KW;
  p.pad_h = (int)ph;
  p.pad_w = (int)pw;
  p.TH = (int)halo_tile_rows(C, KH, KW, stride, OH, OW);
  p.IH_t = (p.TH - 1) * (int)stride + (int)KH;
  p.IW_t = ((int)OW - 1) * (int)stride + (int)KW;
  p.CP = (int)C + 8;
  p.tiles_h = (int)((OH + p.TH - 1) / p.TH);
  p.kw = kw;
  const int64_t T = KH * KW * (C / 32);
  p.words_per_lane = (int)(((T + 3) / 4) * bits);
  p.cb = cb;
  p.cb_dt = cb_dtype;
  p.cb_rows = (int)cb_rows;
  p.cb_size = (int)cb_size;
  p.bias = bias;
  p.bias_dt = bias_dtype;
  p.y = y;
  p.y_dt = y_dtype;
  p.y_layout = y_layout;
  const int CC = (int)(C / 32);
  switch (bits) {
    case 2: return launch_halo_cc<2>(p, CC, (int)stride, s);
    case 3: return launch_halo_cc<3>(p, CC, (int)stride, s);
    default: return launch_halo_cc<4>(p, CC, (int)stride, s);
  }
}

int launch_prepare(const uint8_t* src, int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits, uint32_t* out,
                   hipStream_t s) {
  const int CC = (int)(C / 32);
  const int T = (int)(KH * KW * CC);
  const int chunks = (T + 3) / 4;
  const int64_t total = OC * 4 * chunks;
  const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
  switch (bits) {
    case 2: hipLaunchKernelGGL(prepare_kernel<2>, dim3(blocks), dim3(256), 0, s, src, (int)OC, (int)C, (int)KH,
                               (int)KW, CC, T, chunks, out); break;
    case 3: hipLaunchKernelGGL(prepare_kernel<3>, dim3(blocks), dim3(256), 0, s, src, (int)OC, (int)C, (int)KH,
                               (int)KW, CC, T, chunks, out); break;
    default: hipLaunchKernelGGL(prepare_kernel<4>, dim3(blocks), dim3(256), 0, s, src, (int)OC, (int)C, (int)KH,
                                (int)KW, CC, T, chunks, out); break;
  }
  return check_launch("conv2d_prepare_weight");
}

}  // namespace dimq
