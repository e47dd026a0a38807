// Weight x activation codebook Linear as a true LUT GEMM (index x index
// gather) for decode shapes, and the codebook product table it reads.
//
// The QAT wrapper quantizes activations to its activation_centers C_a
// (quant/dimq_wrapper.py:80-85, hard_quantize_weight, quant/dimq.py:197-221)
// before F.linear with W_hat = C_w[idx]; every product in that GEMM is
// C_w[w] * C_a[a] for a weight index w and an activation index a, so
//   y[m, n] = sum_k T[t(n)][w[n, k]][a[m, k]] + bias[n],
//   T[g][w][a] = C_w[g][w] * C_a[a]   (fp32, one rounding),
// with t(n) = n for per-channel weight codebooks, 0 for a per-layer one.
//
// lut_gather_kernel: 256 threads = 4 waves; a column's k range is split over
// KL lanes of a wave (64 / KL columns per wave), so a wave reads contiguous
// runs of each weight row.  The work-group stages both codebooks in LDS,
// forms its columns' product table there (one table for a per-layer
// codebook; rows padded to a power of two, so an entry's address is two
// shifts and an add), and then each lane walks 32-index chunks of its column:
// the chunk's BITS packed words, the activation indices of the same 32 k for
// MR rows (two 16-byte loads per row), and per (k, m) one LDS lookup and one
// add.  The KL partial sums of a column meet through cross-lane adds.
//
// M rows cost M lookups per weight index; the lanes' lookups land on random
// LDS banks, and on MI355X that bounds the kernel at about 10 CU cycles per
// wave-wide lookup: at 4096 x 4096 it takes 7.9 us for one row against
// 6.7 us for the dequantize-then-GEMV form (both after the same
// nearest-centre pass), so dimq_linear_codebook_act runs it on request
// (DIMQ_VARIANT_SMALL_M) and dimq_linear_lut_act exposes it directly.
#include "gemm_kernel.h"

namespace dimq {
namespace {

constexpr int kLutThreads = 256;

__global__ __launch_bounds__(256) void codebook_table_kernel(const void* __restrict__ cw, int cw_dt, int64_t total,
                                                             int Kw, const float* __restrict__ ca, int Ka,
                                                             float* __restrict__ table) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t gw = i / Ka;  // g * Kw + w
  const int a = static_cast<int>(i - gw * Ka);
  table[i] = load_as_float(cw, cw_dt, gw) * ca[a];
}

// Activation centre a as the reference multiplies it: C_a[a].to(x.dtype).
__device__ __forceinline__ float act_centre(const float* ca, int a, int xdt) {
  const float v = ca[a];
  if (xdt == DIMQ_F16) return f16_bits_to_float(float_to_f16_bits(v));
  if (xdt == DIMQ_BF16) return bf16_bits_to_float(float_to_bf16_bits(v));
  return v;
}

// CLAMP: activation indices may reach Ka or beyond (a caller's indices; they
// read centre Ka - 1); the library's own nearest-centre indices are < Ka.
template <int BITS, int MR, int KL, bool CLAMP>
__global__ __launch_bounds__(kLutThreads) void lut_gather_kernel(const uint8_t* __restrict__ aidx, int M, int64_t K,
                                                                 const uint8_t* __restrict__ w,
                                                                 const void* __restrict__ cw, int cw_dt,
                                                                 int per_channel, int cb_size,
                                                                 const float* __restrict__ ca, int Ka, int lp, int xdt,
                                                                 const void* __restrict__ bias, int bias_dt,
                                                                 int64_t N, void* __restrict__ y, int y_dt) {
  constexpr int Kw = 1 << BITS, LC = 64 / KL, CW = 4 * LC;  // columns per wave / work-group
  extern __shared__ float tab[];                            // [ncols][Kw][P], P = 2^lp >= Ka
  __shared__ float ca_s[256];
  __shared__ float cw_s[CW * Kw];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * CW;
  const int m0 = static_cast<int>(blockIdx.y) * MR;
  const int ncols = per_channel ? CW : 1;
  const int col = wave * LC + lane / KL, kl = lane % KL;
  const int64_t n = n0 + col;
  const int64_t nn = n < N ? n : N - 1;
  const int64_t nchunks = K / 32;
  // K % 32 == 0: every row starts on a word, a chunk is BITS words
  const uint32_t* wrow = reinterpret_cast<const uint32_t*>(w + ((nn * K * BITS) >> 3));
  const uint8_t* arow[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) arow[m] = aidx + static_cast<int64_t>(m0 + m < M ? m0 + m : M - 1) * K;
  // one chunk's BITS weight words and, per row, its 32 activation indices
  struct Chunk {
    uint32_t wd[BITS];
    uint32_t ad[MR][8];
  };
  auto load = [&](Chunk& ch, int64_t c) {
#pragma unroll
    for (int q = 0; q < BITS; ++q) ch.wd[q] = wrow[c * BITS + q];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint4* src = reinterpret_cast<const uint4*>(arow[m] + 32 * c);
      const uint4 lo = src[0], hi = src[1];
      ch.ad[m][0] = lo.x; ch.ad[m][1] = lo.y; ch.ad[m][2] = lo.z; ch.ad[m][3] = lo.w;
      ch.ad[m][4] = hi.x; ch.ad[m][5] = hi.y; ch.ad[m][6] = hi.z; ch.ad[m][7] = hi.w;
    }
  };
  // the lane's first two chunks are requested before the table is formed, so
  // their latency and the codebook loads' overlap
  Chunk A, B;
  if (kl < nchunks) load(A, kl);
  if (kl + KL < nchunks) load(B, kl + KL);

  for (int a = tid; a < Ka; a += kLutThreads) ca_s[a] = act_centre(ca, a, xdt);
  for (int i = tid; i < ncols * Kw; i += kLutThreads) {
    const int c = i / Kw, wi = i % Kw;
    const int64_t row = per_channel ? (n0 + c < N ? n0 + c : N - 1) : 0;
    cw_s[i] = wi < cb_size ? load_as_float(cw, cw_dt, row * cb_size + wi) : 0.0f;  // past the codebook: 0
  }
  __syncthreads();
  // T[c][w][a] = C_w[n0 + c][w] * C_a[a]: fp32, one rounding (rows padded to
  // P entries, so an index is two shifts; the padding is never read)
  const int ts = Kw << lp;
  for (int i = tid; i < ncols * ts; i += kLutThreads) {
    const int a = i & ((1 << lp) - 1);
    tab[i] = a < Ka ? cw_s[i >> lp] * ca_s[a] : 0.0f;
  }
  __syncthreads();

  const char* tb = reinterpret_cast<const char*>(tab + (per_channel ? col * ts : 0));
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
  auto gather = [&](const Chunk& ch) {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int bit = j * BITS;
      uint32_t wi = ch.wd[bit >> 5] >> (bit & 31);
      if ((bit & 31) + BITS > 32) wi |= ch.wd[(bit >> 5) + 1] << (32 - (bit & 31));
      const uint32_t woff = (wi & (Kw - 1)) << (lp + 2);  // byte offset of the weight index's row
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        uint32_t a = (ch.ad[m][j >> 2] >> (8 * (j & 3))) & 0xffu;
        if (CLAMP) a = min(a, static_cast<uint32_t>(Ka - 1));
        acc[m] += *reinterpret_cast<const float*>(tb + woff + (a << 2));
      }
    }
  };
  // two chunks in flight: A holds chunk c, B chunk c + KL
  for (int64_t c = kl; c < nchunks; c += 2 * KL) {
    gather(A);
    if (c + 2 * KL < nchunks) load(A, c + 2 * KL);
    if (c + KL < nchunks) {
      gather(B);
      if (c + 3 * KL < nchunks) load(B, c + 3 * KL);
    }
  }
  // the column's KL partial sums, pairwise across lanes (fp32)
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int off = KL / 2; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  if (kl != 0 || n >= N) return;
  const float b = bias ? load_as_float(bias, bias_dt, n) : 0.0f;
#pragma unroll
  for (int m = 0; m < MR; ++m)
    if (m0 + m < M) store_from_float(y, y_dt, static_cast<int64_t>(m0 + m) * N + n, acc[m] + b);
}

struct LutArgs {
  const uint8_t* aidx;
  int M;
  int64_t K;
  const uint8_t* w;
  const void* cw;
  int cw_dt, per_channel, cb_size;
  const float* ca;
  int Ka, lp, xdt;
  bool clamp;
  const void* bias;
  int bias_dt;
  int64_t N;
  void* y;
  int y_dt;
};

template <int BITS, int MR, int KL>
int launch_lut_kl(const LutArgs& a, hipStream_t s) {
  constexpr int CW = 4 * (64 / KL);
  const size_t lds = static_cast<size_t>(a.per_channel ? CW : 1) * ((1 << BITS) << a.lp) * sizeof(float);
  auto k = a.clamp ? lut_gather_kernel<BITS, MR, KL, true> : lut_gather_kernel<BITS, MR, KL, false>;
  if (lds > 64 * 1024) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DIMQ_ERR_HIP, "linear_lut_act: %s", hipGetErrorString(e));
  }
  const dim3 grid(static_cast<unsigned>((a.N + CW - 1) / CW), static_cast<unsigned>((a.M + MR - 1) / MR));
  hipLaunchKernelGGL(k, grid, dim3(kLutThreads), lds, s, a.aidx, a.M, a.K, a.w, a.cw, a.cw_dt, a.per_channel,
                     a.cb_size, a.ca, a.Ka, a.lp, a.xdt, a.bias, a.bias_dt, a.N, a.y, a.y_dt);
  return check_launch("linear_lut_act");
}

// Lanes per column: enough 32-index chunks for every lane (64 from K = 2048),
// and a per-channel table of the work-group's columns within 64 KiB.
template <int BITS, int MR>
int launch_lut_mr(const LutArgs& a, hipStream_t s) {
  const int64_t chunks = a.K / 32;
  int kl = chunks >= 64 ? 64 : (chunks >= 32 ? 32 : 16);
  while (a.per_channel && kl < 64 && (static_cast<int64_t>(4 * (64 / kl)) * (1 << BITS) << a.lp) * 4 > 64 * 1024) kl *= 2;
  if (kl == 64) return launch_lut_kl<BITS, MR, 64>(a, s);
  if (kl == 32) return launch_lut_kl<BITS, MR, 32>(a, s);
  return launch_lut_kl<BITS, MR, 16>(a, s);
}

template <int BITS>
int launch_lut_bits(const LutArgs& a, hipStream_t s) {
  if (a.M == 1) return launch_lut_mr<BITS, 1>(a, s);
  if (a.M == 2) return launch_lut_mr<BITS, 2>(a, s);
  return launch_lut_mr<BITS, 4>(a, s);
}

}  // namespace

// Shapes the gather kernel runs: M <= 16, K % 32 == 0 (whole index words per
// row), bits 1-4 and up to 256 activation centres (every such product table
// fits the work-group's LDS).
bool lut_act_supported(int64_t M, int64_t K, int bits, int64_t cb_rows, int64_t Ka) {
  (void)cb_rows;
  return M >= 1 && M <= 16 && K % 32 == 0 && bits >= 1 && bits <= 4 && Ka >= 1 && Ka <= 256;
}

int launch_lut_act(const uint8_t* aidx, int64_t M, int64_t K, const uint8_t* w, int bits, const void* cw, int cw_dt,
                   int64_t cb_rows, int64_t cb_size, const float* ca, int64_t Ka, int x_dtype, const void* bias,
                   int bias_dt, int64_t N, void* y, int y_dt, bool clamp, hipStream_t s) {
  int lp = 0;
  while ((int64_t(1) << lp) < Ka) ++lp;
  const LutArgs a{aidx, static_cast<int>(M), K, w, cw, cw_dt, cb_rows == 1 ? 0 : 1, static_cast<int>(cb_size), ca,
                  static_cast<int>(Ka), lp, x_dtype, clamp, bias, bias_dt, N, y, y_dt};
  switch (bits) {
    case 1: return launch_lut_bits<1>(a, s);
    case 2: return launch_lut_bits<2>(a, s);
    case 3: return launch_lut_bits<3>(a, s);
    default: return launch_lut_bits<4>(a, s);
  }
}

int launch_codebook_table(const void* cw, int cw_dt, int64_t G, int64_t Kw, const float* ca, int64_t Ka,
                          float* table, hipStream_t s) {
  const int64_t total = G * Kw * Ka;
  if (total == 0) return DIMQ_OK;
  hipLaunchKernelGGL(codebook_table_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s, cw,
                     cw_dt, total, static_cast<int>(Kw), ca, static_cast<int>(Ka), table);
  return check_launch("codebook product table");
}

}  // namespace dimq

using namespace dimq;

extern "C" int dimq_build_codebook_product_table(const void* w_codebook, int cw_dtype, int64_t rows, int64_t Kw,
                                                 const float* act_centers, int64_t Ka, float* table, void* stream) {
  DIMQ_CHECK(is_float_dtype(cw_dtype), "codebook must be floating point");
  DIMQ_CHECK(rows >= 1 && Kw >= 1 && Ka >= 1 && Ka <= 256, "codebook product table needs rows, Kw >= 1, Ka in [1, 256]");
  DIMQ_CHECK(w_codebook != nullptr && act_centers != nullptr && table != nullptr, "codebooks and table are required");
  return launch_codebook_table(w_codebook, cw_dtype, rows, Kw, act_centers, Ka, table, as_stream(stream));
}

extern "C" int dimq_linear_lut_act(const uint8_t* act_idx, int64_t M, int64_t K, const uint8_t* packed_w,
                                   int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                                   int64_t cb_size, const float* act_centers, int64_t n_act, int x_dtype,
                                   const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype, void* stream) {
  DIMQ_CHECK(M >= 0 && K > 0 && N > 0, "linear dimensions must be positive");
  DIMQ_CHECK(is_float_dtype(cb_dtype), "codebook must be floating point");
  DIMQ_CHECK(cb_rows == 1 || cb_rows == N, "codebook must have 1 (per layer) or out_features (per channel) rows");
  DIMQ_CHECK(cb_size >= 1 && cb_size <= (1 << bits), "codebook rows must hold between 1 and 2^bits entries");
  DIMQ_CHECK(act_centers != nullptr && n_act >= 1 && n_act <= 256, "activation codebook must hold 1 to 256 centres");
  DIMQ_CHECK(x_dtype == DIMQ_F32 || x_dtype == DIMQ_F16 || x_dtype == DIMQ_BF16,
             "x_dtype (the dtype activation centres are rounded to) must be fp32, fp16 or bf16");
  DIMQ_CHECK(packed_numel >= (N * K * bits + 7) / 8, "packed_weight is too small for out_features * in_features");
  DIMQ_CHECK(bias == nullptr || is_float_dtype(bias_dtype), "bias must be floating point");
  DIMQ_CHECK(y_dtype == DIMQ_F32 || y_dtype == DIMQ_F16 || y_dtype == DIMQ_BF16,
             "output dtype must be fp32, fp16 or bf16");
  if (M == 0) return DIMQ_OK;
  DIMQ_CHECK(lut_act_supported(M, K, bits, cb_rows, n_act),
             "linear_lut_act runs M <= 16, in_features % 32 == 0, bits 1-4 and at most 256 activation centres");
  DIMQ_CHECK(aligned(act_idx, 16) && aligned(packed_w, 4),
             "activation indices must be 16-byte and packed weights 4-byte aligned");
  return launch_lut_act(act_idx, M, K, packed_w, bits, codebook, cb_dtype, cb_rows, cb_size, act_centers, n_act,
                        x_dtype, bias, bias_dtype, N, y, y_dtype, /*clamp=*/true, as_stream(stream));
}
