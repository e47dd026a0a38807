/*
 * CPU restatement of the DIMQ packed-index inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (dimq_amd/) links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only as the checker.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the fengchao32/DIMQ tree).  The reference implements only the 4-bit,
 * per-layer-codebook case; the functions below generalise it to b in
 * {2,3,4,8} bits and per-output-channel codebooks, keeping the u4 case
 * byte-identical.
 *
 * Bit layout ("LSB-first bitstream"): index i occupies bits [b*i, b*i+b) of a
 * little-endian byte stream, which for b=4 is exactly
 * packed[j] = idx[2j] | idx[2j+1] << 4 (dimq_backend/export.py:43).
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that no multiply-add is
 * fused: the reference computes every product and sum in separately rounded
 * fp32 operations).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Number of bytes that n b-bit indices occupy.  u4: (n+1)/2
 * (dimq_backend/export.py:69, csrc/dimq_pack.cu:57). */
int64_t dimq_oracle_packed_nbytes(int64_t n, int bits) {
  return (n * (int64_t)bits + 7) / 8;
}

/* Pack: dimq_backend/export.py:38-55 (u4: low nibble = even index, odd tail
 * padded with a zero nibble, :51-54) and csrc/dimq_pack.cu:11-25 (values are
 * masked to the field width, :19-22).  Generalised to b bits LSB-first; the
 * unused high bits of the last byte are zero. */
void dimq_oracle_pack_bits(const uint8_t* idx, int64_t n, int bits, uint8_t* out) {
  int64_t nbytes = dimq_oracle_packed_nbytes(n, bits);
  memset(out, 0, (size_t)nbytes);
  uint32_t mask = (1u << bits) - 1u;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t v = idx[i] & mask;
    int64_t bit = i * bits;
    for (int j = 0; j < bits; ++j) {
      if ((v >> j) & 1u) {
        int64_t p = bit + j;
        out[p >> 3] |= (uint8_t)(1u << (p & 7));
      }
    }
  }
}

/* Unpack: dimq_backend/export.py:58-78 and csrc/dimq_pack.cu:27-35 with
 * get_u4 (csrc/dimq_common.cuh:9-15).  Returns 0, or -1 when the packed buffer
 * is too small (export.py:69-71, dimq_pack.cu:73). */
int dimq_oracle_unpack_bits(const uint8_t* packed, int64_t nbytes, int64_t n, int bits, uint8_t* out) {
  if (n < 0) return -1;
  if (nbytes < dimq_oracle_packed_nbytes(n, bits)) return -1;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t v = 0;
    int64_t bit = i * bits;
    for (int j = 0; j < bits; ++j) {
      int64_t p = bit + j;
      v |= (uint32_t)((packed[p >> 3] >> (p & 7)) & 1u) << j;
    }
    out[i] = (uint8_t)v;
  }
  return 0;
}

/* Nearest-centre assignment: quant/dimq.py:197-221 (dist = (w - c)^2 in fp32,
 * argmin keeps the first minimum, :214-215) and dimq_backend/export.py:24-35.
 * A NaN distance wins and the first NaN is kept, as torch.argmin does.
 * Per-channel (per_channel=1): row r uses centers[r*K : r*K+K]; per-layer
 * (per_channel=0): every row uses centers[0:K].  val_out may be NULL; it
 * receives centers[idx] (dimq.py:216). */
void dimq_oracle_hard_quantize(const float* w, int64_t rows, int64_t row_len,
                               const float* centers, int K, int per_channel,
                               uint8_t* idx_out, float* val_out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* c = centers + (per_channel ? r * (int64_t)K : 0);
    for (int64_t k = 0; k < row_len; ++k) {
      float x = w[r * row_len + k];
      int best = 0;
      float best_d = 0.0f;
      int have = 0;
      int have_nan = 0;
      for (int j = 0; j < K; ++j) {
        float diff = x - c[j];
        float d = diff * diff;
        if (isnan(d)) {
          if (!have_nan) {
            best = j;
            have_nan = 1;
          }
          continue;
        }
        if (have_nan) continue;
        if (!have || d < best_d) {
          best = j;
          best_d = d;
          have = 1;
        }
      }
      idx_out[r * row_len + k] = (uint8_t)best;
      if (val_out) val_out[r * row_len + k] = c[best];
    }
  }
}

/* Uniform affine u4 activation code: dimq_backend/reference.py:11-21,
 * q = clamp(round_half_even(x / s) + zp, 0, 15), IEEE fp32 divide.  A NaN
 * quotient gives zp: the reference CUDA kernel computes
 * __float2int_rn(x / s) + zp (csrc/dimq_common.cuh:17-21), and the PTX
 * conversion maps NaN to 0; +-inf and other out-of-range quotients clamp to
 * 15 / 0 as the torch reference does. */
static int quant_u4(float x, float s, int zp) {
  float r = rintf(x / s);
  float q = (r == r ? r : 0.0f) + (float)zp;
  if (q < 0.0f) q = 0.0f;
  if (q > 15.0f) q = 15.0f;
  return (int)q;
}

void dimq_oracle_quantize_act_u4(const float* x, int64_t n, float s, int zp, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)quant_u4(x[i], s, zp);
}

/* Product table: dimq_backend/reference.py:32-44 and
 * csrc/dimq_product_table.cu:11-25.  P[g][w][a] = C[g][w] * (s * (a - zp)),
 * each product rounded to fp32.  G = 1 is the reference's per-layer table. */
void dimq_oracle_product_table(const float* cb, int G, int Kw, float s, int zp, float* table) {
  for (int g = 0; g < G; ++g)
    for (int w = 0; w < Kw; ++w)
      for (int a = 0; a < 16; ++a) {
        float ahat = s * (float)(a - zp);
        table[((int64_t)g * Kw + w) * 16 + a] = cb[(int64_t)g * Kw + w] * ahat;
      }
}

/* Dequantize packed weights: dimq_backend/reference.py:47-56,
 * W_hat[n,k] = C[idx[n,k]] (per-channel: C[n, idx[n,k]]). */
int dimq_oracle_dequantize(const uint8_t* packed, int64_t nbytes, int bits, const float* cb, int Kc,
                           int per_channel, int64_t N, int64_t K, float* w_hat) {
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t k = 0; k < K; ++k) {
      int64_t i = n * K + k;
      int64_t bit = i * bits;
      uint32_t v = 0;
      for (int j = 0; j < bits; ++j) {
        int64_t p = bit + j;
        if ((p >> 3) >= nbytes) return -1;
        v |= (uint32_t)((packed[p >> 3] >> (p & 7)) & 1u) << j;
      }
      if ((int)v >= Kc) return -1;
      w_hat[i] = cb[(per_channel ? n * Kc : 0) + v];
    }
  }
  return 0;
}

/* W4A4 LUT Linear: dimq_backend/reference.py:59-88 (y[m,n] = sum_k
 * P[w[n,k], a[m,k]] + bias[n]) with the k-order of csrc/dimq_gemm_lut.cu:45-49
 * (sequential fp32 sum, then bias). */
void dimq_oracle_linear_lut(const float* x, int64_t M, int64_t N, int64_t K, const uint8_t* packed_w,
                            const float* cb16, float s, int zp, const float* bias, float* y) {
  float table[256];
  dimq_oracle_product_table(cb16, 1, 16, s, zp, table);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        int q = quant_u4(x[m * K + k], s, zp);
        int64_t i = n * K + k;
        int w = (packed_w[i >> 1] >> ((i & 1) * 4)) & 15;
        acc += table[w * 16 + q];
      }
      if (bias) acc += bias[n];
      y[m * N + n] = acc;
    }
  }
}

/* W4A4 LUT Conv2d (NCHW, zero padding, stride, dilation, groups):
 * dimq_backend/reference.py:147-205 and csrc/dimq_conv2d_lut.cu:14-86. */
void dimq_oracle_conv2d_lut(const float* x, int B, int C, int H, int W, const uint8_t* packed_w,
                            const float* cb16, float s, int zp, const float* bias, int OC, int ICg,
                            int KH, int KW, int sh, int sw, int ph, int pw, int dh, int dw, int groups,
                            float* y) {
  float table[256];
  dimq_oracle_product_table(cb16, 1, 16, s, zp, table);
  int OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
  int OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  int ocg = OC / groups;
  for (int b = 0; b < B; ++b)
    for (int co = 0; co < OC; ++co) {
      int g = co / ocg;
      for (int oh = 0; oh < OH; ++oh)
        for (int ow = 0; ow < OW; ++ow) {
          float acc = 0.0f;
          for (int cig = 0; cig < ICg; ++cig) {
            int ci = g * ICg + cig;
            for (int kh = 0; kh < KH; ++kh) {
              int ih = oh * sh + kh * dh - ph;
              if (ih < 0 || ih >= H) continue;
              for (int kw = 0; kw < KW; ++kw) {
                int iw = ow * sw + kw * dw - pw;
                if (iw < 0 || iw >= W) continue;
                int q = quant_u4(x[(((int64_t)b * C + ci) * H + ih) * W + iw], s, zp);
                int64_t i = (((int64_t)co * ICg + cig) * KH + kh) * KW + kw;
                int w = (packed_w[i >> 1] >> ((i & 1) * 4)) & 15;
                acc += table[w * 16 + q];
              }
            }
          }
          if (bias) acc += bias[co];
          y[(((int64_t)b * OC + co) * OH + oh) * OW + ow] = acc;
        }
    }
}
