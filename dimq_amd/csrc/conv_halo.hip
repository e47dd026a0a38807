// Host side of the LDS-halo conv kernels (conv_halo.h): weight preparation
// into the kernel layout, shape eligibility, launch.
#include "conv_halo.h"
#include "conv_band.h"

namespace dimq {
namespace {

// ---- weight preparation: conv_kcrs b-bit stream -> kernel layout
// out[((n*2 + g)*CHUNKS + chunk)*BITS + w]: sub-steps t = 4*chunk + s, slot j
// holds channel c = 16*(t % CC16) + 8*g + j at (kh, kw) = divmod(t / CC16, KW),
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

// Thread id's BITS words of the layout (ids past OC * 2 * chunks: none).
template <int BITS>
__device__ __forceinline__ void prepare_words(int64_t id, const uint8_t* __restrict__ src, int OC, int C, int KH,
                                              int KW, int CC, int T, int chunks, uint32_t* __restrict__ out) {
  const int64_t total = (int64_t)OC * 2 * chunks;
  if (id >= total) return;
  const int chunk = static_cast<int>(id % chunks);
  const int g = static_cast<int>((id / chunks) % 2);
  const int n = static_cast<int>(id / (2 * chunks));
  uint32_t words[BITS];
#pragma unroll
  for (int w = 0; w < BITS; ++w) words[w] = 0;
  // fully unrolled and predicated (no early exit), so all 32 index loads
  // of the thread go out back to back instead of in four latency rounds
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int t = 4 * chunk + s;
    if (t >= T) continue;
    const int khw = t / CC;
    const int cc = t - khw * CC;
    const int kh = khw / KW;
    const int kw = khw - kh * KW;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = 16 * cc + 8 * g + j;
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

template <int BITS>
__global__ void prepare_kernel(const uint8_t* __restrict__ src, int OC, int C, int KH, int KW, int CC, int T,
                               int chunks, uint32_t* __restrict__ out) {
  prepare_words<BITS>(static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x, src, OC, C, KH, KW, CC, T, chunks,
                      out);
}

// The two inputs of a W4A4 conv2d_lut call on the halo / band kernels in one
// launch: work-groups [0, wblocks) lay out the 4-bit weight (prepare_words),
// the rest quantize the activations to the fp16 integers q - zp
// (quantize_a4_f16_groups, as quantize_a4_f16_kernel); the weight's few
// work-groups then cost no launch of their own.
template <int XT, bool VEC>
__global__ __launch_bounds__(256) void w4a4_conv_inputs_kernel(const uint8_t* __restrict__ src, int OC, int C, int KH,
                                                              int KW, int CC, int T, int chunks,
                                                              uint32_t* __restrict__ kw, int wblocks,
                                                              const void* __restrict__ x, int64_t n, float s, int zp,
                                                              uint16_t* __restrict__ q) {
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < wblocks) {
    prepare_words<4>(static_cast<int64_t>(bid) * 256 + threadIdx.x, src, OC, C, KH, KW, CC, T, chunks, kw);
    return;
  }
  quantize_a4_f16_groups<XT, VEC, kQa4Groups>(x, n, s, zp, q,
                                              static_cast<int64_t>(bid - wblocks) * 256 * kQa4Groups + threadIdx.x, 256);
}

}  // namespace

// Band kernel (conv_band.h) for a halo call: C = 64, 3x3, stride 1, pad 1,
// fp32 or fp16 output, and either
//   NCHW in and out (fp16: OH*OW % 8 == 0), epilogue none / ReLU, either with
//   the next layer's activation quantization (fp16 out), or
//   NHWC in and out (OC % 32 == 0), epilogue none / ReLU, or a 16-bit
//   16-byte aligned residual (+ ReLU) with an fp16 output.
// Picks the parts per image (about one work-group per CU, at most 13 blocks
// of 32 pixels per part) and checks that every part's stages fit one task per
// thread and its halo fits in LDS; fills p.parts, p.nblk, p.IH_t, p.IW_t.
// False: the call takes the tile kernels.
static bool band_setup(HaloArgs& p, int stride, int mode) {
  if (!(p.y_dt == DIMQ_F32 || p.y_dt == DIMQ_F16)) return false;
  if (p.C != 64 || p.KH != 3 || p.KW != 3 || stride != 1 || p.pad_h != 1 || p.pad_w != 1) return false;
  if (p.x_layout == DIMQ_NHWC) {
    if (p.y_layout != DIMQ_NHWC || p.OC % 32 != 0) return false;
    const bool res16 = p.epi.res_vec && (p.epi.res_dt == DIMQ_F16 || p.epi.res_dt == DIMQ_BF16) &&
                       p.y_dt == DIMQ_F16;
    if (!(mode == kEpiNone || mode == kEpiRelu || ((mode == kEpiRes || mode == kEpiResRelu) && res16))) return false;
  } else {
    if (p.x_layout != DIMQ_NCHW || p.y_layout != DIMQ_NCHW) return false;
    if (!(mode == kEpiNone || mode == kEpiRelu || mode == kEpiQuant || mode == (kEpiRelu | kEpiQuant))) return false;
    if ((mode & kEpiQuant) != 0 && p.y_dt != DIMQ_F16) return false;
    if (p.y_dt == DIMQ_F16 && ((int64_t)p.OH * p.OW) % 8 != 0) return false;  // 16-byte fp16 stores of 8 pixels
  }
  if (p.W % 8 != 0 || p.OW != p.W || p.OH != p.H || ((int64_t)p.OH * p.OW) % 4 != 0) return false;
  if (!aligned(p.y, 16)) return false;
  const int64_t npx = (int64_t)p.OH * p.OW;
  if (npx > (1 << 24)) return false;
  const int nblk = (int)((npx + 31) / 32);
  const int cus = device_cus();
  int parts = std::max<int>((cus + p.B - 1) / p.B, (nblk + 12) / 13);
  parts = std::min(parts, nblk);
  if ((int64_t)p.B * parts >= (1ll << 31)) return false;
  int ihmax = 0;
  for (int part = 0; part < parts; ++part) {
    const BandPart q = band_part(nblk, parts, part, p.OH, p.OW);
    if (q.blk1 <= q.blk0) return false;
    if (q.ra * p.W > kBandThreads || (q.IH - q.ra) * p.W > kBandThreads) return false;
    ihmax = std::max(ihmax, q.IH);
  }
  const int64_t lds = (int64_t)ihmax * (p.W + 2) * 72 * 2 + 8 * kParkFloats * 4;
  if (lds > 160 * 1024) return false;
  p.parts = parts;
  p.nblk = nblk;
  p.IH_t = ihmax;
  p.IW_t = p.W + 2;
  return true;
}

int64_t halo_prepared_words(int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits) {
  const int64_t T = KH * KW * (C / 16);
  return OC * 2 * ((T + 3) / 4) * bits;
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
                   int64_t groups, int64_t OH, int64_t OW, int bits, int x_dtype, int epi_mode_, int y_layout) {
  if (!halo_weight_supported(C, KH, KW, bits)) return false;
  if (!halo_mode_ok(epi_mode_, KH * KW * (C / 16) <= 36, y_layout == DIMQ_NCHW)) return false;
  if (x_dtype != DIMQ_F16) return false;  // fp16 staging (other dtypes: the guarded implicit GEMM)
  if (groups != 1 || dh != 1 || dw != 1 || sh != sw || (sh != 1 && sh != 2)) return false;
  return halo_tile_rows(C, KH, KW, sh, OH, OW) > 0;
}

int launch_conv_halo(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                     const uint32_t* kw, int bits, const void* cb, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                     const void* bias, int bias_dtype, int64_t OC, int64_t KH, int64_t KW, int64_t stride,
                     int64_t ph, int64_t pw, int64_t OH, int64_t OW, void* y, int y_dtype, int y_layout,
                     const Epi& epi, hipStream_t s, float acc_scale) {
  HaloArgs p{};
  p.epi = epi;
  p.acc_scale = acc_scale;
  p.x = x;
  if (x_dtype != DIMQ_F16) return set_error(DIMQ_ERR_UNSUPPORTED, "conv halo kernel takes fp16 activations");
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
  const int64_t T = KH * KW * (C / 16);
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
  const int CC = (int)(C / 16);
  const int mode = epi_mode(epi);
  if (band_setup(p, (int)stride, mode)) {
    switch (bits) {
      case 2: return launch_band_b2(p, mode, s);
      case 3: return launch_band_b3(p, mode, s);
      default: return launch_band_b4(p, mode, s);
    }
  }
  switch (bits) {
    case 2: return launch_halo_b2(p, CC, (int)stride, mode, s);
    case 3: return launch_halo_b3(p, CC, (int)stride, mode, s);
    default: return launch_halo_b4(p, CC, (int)stride, mode, s);
  }
}

int launch_w4a4_conv_inputs(const uint8_t* src, int64_t OC, int64_t C, int64_t KH, int64_t KW, uint32_t* kw,
                            const void* x, int x_dtype, int64_t n, float scale, int zp, uint16_t* q, hipStream_t s) {
  const int CC = (int)(C / 16);
  const int T = (int)(KH * KW * CC);
  const int chunks = (T + 3) / 4;
  const int64_t wblocks = (OC * 2 * chunks + 255) / 256;
  const int64_t qblocks = ((n + 7) / 8 + 256 * kQa4Groups - 1) / (256 * kQa4Groups);
  const dim3 grid(static_cast<unsigned>(wblocks + qblocks));
  const bool vec = aligned(x, 16);
#define DIMQ_W4A4_IN(XT, V)                                                                                      \
  hipLaunchKernelGGL((w4a4_conv_inputs_kernel<XT, V>), grid, dim3(256), 0, s, src, (int)OC, (int)C, (int)KH,       \
                     (int)KW, CC, T, chunks, kw, (int)wblocks, x, n, scale, zp, q)
  switch (x_dtype) {
    case DIMQ_F32: if (vec) DIMQ_W4A4_IN(DIMQ_F32, true); else DIMQ_W4A4_IN(DIMQ_F32, false); break;
    case DIMQ_F16: if (vec) DIMQ_W4A4_IN(DIMQ_F16, true); else DIMQ_W4A4_IN(DIMQ_F16, false); break;
    case DIMQ_BF16: if (vec) DIMQ_W4A4_IN(DIMQ_BF16, true); else DIMQ_W4A4_IN(DIMQ_BF16, false); break;
    default: DIMQ_W4A4_IN(DIMQ_F64, false); break;
  }
#undef DIMQ_W4A4_IN
  return check_launch("conv2d_lut (weight layout and activation quantization)");
}

int launch_prepare(const uint8_t* src, int64_t OC, int64_t C, int64_t KH, int64_t KW, int bits, uint32_t* out,
                   hipStream_t s) {
  const int CC = (int)(C / 16);
  const int T = (int)(KH * KW * CC);
  const int chunks = (T + 3) / 4;
  const int64_t total = OC * 2 * chunks;
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
