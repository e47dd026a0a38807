/*
 * dimq_hip.h — C ABI of libdimq_hip.so, the MI355X (gfx950) DIMQ packed-index
 * inference library.
 *
 * Every entry point takes raw device pointers, element counts and a HIP stream
 * (hipStream_t passed as void*; NULL = the legacy default stream), launches
 * asynchronously on that stream, and returns DIMQ_OK (0) or an error code.  On
 * error dimq_last_error() returns a thread-local message; the message text of
 * the reference's TORCH_CHECKs is kept where a reference check exists.  No
 * entry point allocates device memory: outputs are caller-allocated.
 *
 * Citations are relative to the fengchao32/DIMQ tree.  The reference binds its
 * six ops through TORCH_LIBRARY(dimq) (dimq_cuda_backend/csrc/dimq_ops.cpp:37-53);
 * the dimq_* functions in section 1 replace those CUDA impls one for one, with
 * the tensor arguments flattened to pointer + size + dtype.
 */
#ifndef DIMQ_HIP_H_
#define DIMQ_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of tensors crossing the boundary. */
enum dimq_dtype {
  DIMQ_F32 = 0,
  DIMQ_F16 = 1,
  DIMQ_BF16 = 2,
  DIMQ_F64 = 3,
  DIMQ_U8 = 4
};

/* Return codes. */
enum dimq_status {
  DIMQ_OK = 0,
  DIMQ_ERR_INVALID = 1,     /* argument check failed (reference: TORCH_CHECK) */
  DIMQ_ERR_UNSUPPORTED = 2, /* dtype / bit-width / layout not implemented */
  DIMQ_ERR_HIP = 3          /* HIP runtime error at launch */
};

/* Conv activation layouts. */
enum dimq_layout { DIMQ_NCHW = 0, DIMQ_NHWC = 1 };

/* Kernel variant selector for the weight-only ops. */
/* Activation of the fused epilogue of the *_ex weight-only ops. */
enum dimq_activation {
  DIMQ_ACT_NONE = 0,
  DIMQ_ACT_RELU = 1, /* max(v, 0); NaN stays NaN as in torch.relu */
  DIMQ_ACT_GELU = 2  /* exact: 0.5 v (1 + erf(v / sqrt 2)), torch's F.gelu default */
};

enum dimq_variant {
  DIMQ_VARIANT_AUTO = 0,
  DIMQ_VARIANT_SMALL_M = 1, /* register-codebook gather, 16-row tiles (decode / GEMV) */
  DIMQ_VARIANT_MFMA = 2     /* dequant-to-fp16 + MFMA, 64/128-row tiles; for a conv with a prepared weight
                               and NHWC 16-bit input, the implicit-GEMM tiles even where the LDS-halo
                               kernel is the default */
};

/* Thread-local message of the last failing call on this thread. */
const char* dimq_last_error(void);
/* ABI version of this header (bumped on incompatible changes). */
int dimq_abi_version(void);

/* ---------------------------------------------------------------------------
 * 1. The reference's ops (dimq_cuda_backend/csrc/dimq_ops.cpp:38-43)
 * ------------------------------------------------------------------------- */

/* pack_u4: replaces pack_u4_cuda (csrc/dimq_pack.cu:52-67).  packed receives
 * (numel+1)/2 bytes, packed[j] = idx[2j]&15 | (idx[2j+1]&15)<<4. */
int dimq_pack_u4(const uint8_t* indices, int64_t numel, uint8_t* packed, void* stream);

/* unpack_u4: replaces unpack_u4_cuda (csrc/dimq_pack.cu:69-85). */
int dimq_unpack_u4(const uint8_t* packed, int64_t packed_numel, int64_t numel, uint8_t* indices,
                   void* stream);

/* quantize_activation_u4: replaces quantize_activation_u4_cuda
 * (csrc/dimq_pack.cu:87-109).  x_dtype in {F32, F16, BF16, F64}; out u8. */
int dimq_quantize_activation_u4(const void* x, int x_dtype, int64_t numel, double act_scale,
                                int64_t act_zp, uint8_t* out, void* stream);

/* build_product_table: replaces build_product_table_cuda
 * (csrc/dimq_product_table.cu:29-46).  table receives [16,16] fp32. */
int dimq_build_product_table(const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale,
                             int64_t act_zp, float* table, void* stream);

/* linear_lut: replaces linear_lut_cuda (csrc/dimq_gemm_lut.cu:58-117).
 * x [M, in_features] row-major; packed_w u4 [out_features*in_features];
 * 16-entry per-layer codebook; bias (nullable) [out_features];
 * y [M, out_features] fp32.  y = sum_k P[w,a] + bias, P = C[w]*s*(a-zp). */
int dimq_linear_lut(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                    const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale, int64_t act_zp,
                    const void* bias, int bias_dtype, int64_t bias_numel, int64_t out_features,
                    int64_t in_features, float* y, void* stream);

/* conv2d_lut: replaces conv2d_lut_cuda (csrc/dimq_conv2d_lut.cu:90-186).
 * x NCHW [B,C,H,W]; packed_w u4 in conv_kcrs order [OC, C/groups, KH, KW];
 * y NCHW fp32 [B, OC, OH, OW]. */
int dimq_conv2d_lut(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                    const uint8_t* packed_w, int64_t packed_numel, const void* codebook, int cb_dtype,
                    int64_t cb_numel, double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                    int64_t bias_numel, int64_t out_channels, int64_t in_channels_per_group, int64_t kernel_h,
                    int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                    int64_t dilation_h, int64_t dilation_w, int64_t groups, float* y, void* stream);

/* Workspace forms of linear_lut / conv2d_lut (same reference ops, same
 * arguments, checks and messages as the two entry points above, plus a
 * caller-owned device workspace; the library allocates nothing).  With an
 * fp16 codebook — the reference exporter's default
 * (dimq_backend/export.py:167,217, codebook_dtype=torch.float16) — and a
 * workspace of at least the *_workspace_bytes size, 16-byte aligned, the
 * activations are quantized once to the exact fp16 integers a - zp and the
 * weight-only kernels run on them with act_scale applied to the fp32
 * accumulator: y = s * sum_k C[w] * (a - zp) + bias, equal to the reference's
 * sum_k C[w] * (s * (a - zp)) up to fp32 rounding and summation order.
 * Otherwise (workspace NULL or short, codebook not fp16) they run the same
 * kernels as dimq_linear_lut / dimq_conv2d_lut.  The workspace is read and
 * written on `stream`: calls that share one must be ordered on that stream.
 * *_workspace_bytes returns 0 when no workspace is used for the shape. */
int64_t dimq_linear_lut_workspace_bytes(int64_t M, int64_t in_features, int cb_dtype);
int dimq_linear_lut_ws(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                       const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale, int64_t act_zp,
                       const void* bias, int bias_dtype, int64_t bias_numel, int64_t out_features,
                       int64_t in_features, float* y, void* workspace, int64_t workspace_bytes, void* stream);
int64_t dimq_conv2d_lut_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t out_channels,
                                        int64_t in_channels_per_group, int64_t kernel_h, int64_t kernel_w,
                                        int64_t groups, int cb_dtype);
int dimq_conv2d_lut_ws(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                       const uint8_t* packed_w, int64_t packed_numel, const void* codebook, int cb_dtype,
                       int64_t cb_numel, double act_scale, int64_t act_zp, const void* bias, int bias_dtype,
                       int64_t bias_numel, int64_t out_channels, int64_t in_channels_per_group, int64_t kernel_h,
                       int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                       int64_t dilation_h, int64_t dilation_w, int64_t groups, float* y, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* No-allocation form of linear_lut.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, checks, messages and results as
 * dimq_linear_lut_ws with a workspace; the fp16 activations go to a scratch
 * array the library holds on each GPU it runs on (16 MiB per device, kept
 * until the process ends), so M * in_features is limited to 8,388,608 with an
 * fp16 codebook (DIMQ_ERR_INVALID beyond; other codebook dtypes use no
 * scratch).  All calls on one GPU share that GPU's scratch: calls that
 * overlap on one GPU (other streams or host threads) race and must be
 * ordered by the caller. */
int dimq_linear_lut_noalloc(const void* x, int x_dtype, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                            const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale, int64_t act_zp,
                            const void* bias, int bias_dtype, int64_t bias_numel, int64_t out_features,
                            int64_t in_features, float* y, void* stream);

/* Chained W4A4 layers with the next layer's activation quantization fused
 * into the producing layer's epilogue (no kernel counterpart in the
 * reference, whose linear_lut / conv2d_lut each quantize
 * their float input themselves, csrc/dimq_gemm_lut.cu:45-49,
 * csrc/dimq_conv2d_lut.cu:62-81).  The activations travel between layers as
 * the fp16 integers a - zp (a = clamp(rint(x / s) + zp, 0, 15), the
 * reference's u4 code; exact in fp16):
 *  - dimq_quantize_activation_f16 writes that form of a float tensor (the
 *    chain's first input; out 16-byte aligned);
 *  - dimq_linear_lut_q / dimq_conv2d_lut_q take it (xq [M, in_features] /
 *    NCHW, with its act_scale s) and compute
 *      y = act(s * sum_k C[w] (a - zp) + bias),
 *    the reference's linear_lut / conv2d_lut on the dequantized codes,
 *    activation in {none, relu, gelu}; with out_act_scale > 0, y (fp16) is
 *    the next layer's codes q' - zp' of that result (same rounding as
 *    dimq_quantize_activation_f16), else y holds it in y_dtype.
 * The codebook is the 16-entry fp16 codebook of the packed export.  For the
 * conv, prepared_w (nullable) is dimq_conv2d_prepare_weight's layout at 4
 * bits, prepared once per layer; the output layout is NCHW. */
int dimq_quantize_activation_f16(const void* x, int x_dtype, int64_t numel, double act_scale, int64_t act_zp,
                                 uint16_t* out, void* stream);
int dimq_linear_lut_q(const uint16_t* xq, int64_t M, const uint8_t* packed_w, int64_t packed_numel,
                      const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale, const void* bias,
                      int bias_dtype, int64_t bias_numel, int64_t out_features, int64_t in_features, int activation,
                      double out_act_scale, int64_t out_act_zp, void* y, int y_dtype, void* stream);
int dimq_conv2d_lut_q(const uint16_t* xq, int64_t B, int64_t C, int64_t H, int64_t W, const uint8_t* packed_w,
                      int64_t packed_numel, const uint32_t* prepared_w, int64_t prepared_words,
                      const void* codebook, int cb_dtype, int64_t cb_numel, double act_scale, const void* bias,
                      int bias_dtype, int64_t bias_numel, int64_t out_channels, int64_t in_channels_per_group,
                      int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                      int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, int activation,
                      double out_act_scale, int64_t out_act_zp, void* y, int y_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * 2. Generalised ops for the BASELINE configurations: b in {2,3,4,8} bits,
 *    per-layer or per-output-channel codebooks, weight-only GEMM/conv.
 *    The reference has no kernel for these (it is W4A4-only); their
 *    semantics are those of dequantize-then-F.linear / F.conv2d
 *    (dimq_backend/reference.py:47-56,91-144; quant/dimq_wrapper.py:189-197,237-240).
 * ------------------------------------------------------------------------- */

/* LSB-first b-bit packing, generalising pack_u4_indices
 * (dimq_backend/export.py:38-55): index i occupies bits [b*i, b*i+b).
 * packed receives ceil(numel*bits/8) bytes; values are masked to b bits. */
int dimq_pack_bits(const uint8_t* indices, int64_t numel, int bits, uint8_t* packed, void* stream);

/* Inverse of dimq_pack_bits, generalising unpack_u4_indices (export.py:58-78). */
int dimq_unpack_bits(const uint8_t* packed, int64_t packed_numel, int64_t numel, int bits,
                     uint8_t* indices, void* stream);

/* Nearest-centre assignment, quant/dimq.py:197-221 (hard_quantize_weight) and
 * dimq_backend/export.py:24-35: idx = argmin_j (w - c_j)^2 in fp32, first
 * minimum wins; a NaN distance wins (first NaN), as torch.argmin.
 * w [rows, row_len] (w_dtype F32/F16/BF16); centers fp32 [rows, n_centers]
 * when per_channel, else [n_centers] shared by every row; n_centers <= 256.
 * values (nullable) receives centers[idx] in w_dtype. */
int dimq_hard_quantize(const void* w, int w_dtype, int64_t rows, int64_t row_len, const float* centers,
                       int64_t n_centers, int per_channel, uint8_t* indices, void* values, void* stream);

/* Per-channel product table, generalising build_product_table
 * (dimq_backend/reference.py:32-44): table [G, Kc, 16] fp32,
 * table[g][w][a] = C[g][w] * (s * (a - zp)). */
int dimq_build_product_table_grouped(const void* codebook, int cb_dtype, int64_t groups, int64_t kc,
                                     double act_scale, int64_t act_zp, float* table, void* stream);

/* Weight-only codebook Linear: y[M,N] = x[M,K] . W_hat[N,K]^T + bias.
 * packed_w: LSB-first b-bit stream of the row-major [N,K] index matrix;
 * codebook [cb_rows, cb_size] with cb_rows in {1 (per layer), N (per output
 * channel)} and cb_size <= 2^bits; x_dtype/y_dtype in {F32, F16, BF16};
 * bias (nullable, any float dtype) [N]; fp32 accumulation.
 * Activations are rounded to nearest fp16 for the matrix cores (exact for
 * fp16, and for bf16 values within the fp16 range); the codebook is scaled
 * per row by a power of two before rounding to fp16.  Range guard: a tile
 * whose fp32/bf16 activations hold a value beyond the fp16 range (any
 * accumulator inf or NaN), or none of magnitude >= 2^-7, is recomputed in
 * fp32 from the activations and centres in their own dtypes, so results stay
 * within fp32 rounding of the reference for every input range (such tiles
 * run far slower than the matrix path). */
int dimq_linear_codebook(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                         int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                         int64_t cb_size, const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                         int variant, void* stream);

/* Words of the kernel-layout weight of a conv (0 when the shape has no
 * kernel layout).  The prepared weight holds, one after the other, the
 * LDS-halo layout (C in {64, 128}, 3x3 or 1x1, bits in {2,3,4}; padded to a
 * multiple of 4 words) and the tap-major layout (C % 64 == 0, bits in
 * {2,3,4}), each when the shape has it. */
int64_t dimq_conv2d_prepared_words(int64_t out_channels, int64_t in_channels, int64_t kernel_h, int64_t kernel_w,
                                   int bits);

/* One-time repack of a conv_kcrs b-bit index stream into the kernel
 * layouts: the LDS-halo layout (per output channel and lane group, the
 * indices of each (kh, kw, 32-channel) step in decode order) and the
 * tap-major layout read by the implicit-GEMM kernel (index (oc, kh, kw, c)
 * at k = (kh*KW + kw)*C + c, LSB-first).  Same bits, no expansion; done when
 * a layer is loaded, not per call. */
int dimq_conv2d_prepare_weight(const uint8_t* packed_w, int64_t packed_numel, int bits, int64_t out_channels,
                               int64_t in_channels, int64_t kernel_h, int64_t kernel_w, uint32_t* prepared_w,
                               int64_t prepared_words, void* stream);

/* Weight-only codebook Conv2d (zero padding, stride, dilation, groups).
 * x [B,C,H,W] in x_layout (NCHW or NHWC memory order); y [B,OC,OH,OW] in
 * y_layout; packed_w: b-bit stream of the conv_kcrs index tensor
 * [OC, C/groups, KH, KW] (dimq_backend/export.py:232).  prepared_w
 * (nullable): the same weights in kernel layouts (dimq_conv2d_prepare_weight);
 * with it, NHWC 16-bit calls take the large-tile implicit GEMM or the LDS-halo
 * kernel by shape.  Stride-2 convs of C <= 4 channels (network stems) take a
 * dedicated kernel; everything else the generic implicit-GEMM kernel. */
int dimq_conv2d_codebook(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                         const uint8_t* packed_w, int64_t packed_numel, int bits, const uint32_t* prepared_w,
                         int64_t prepared_words, const void* codebook,
                         int cb_dtype, int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype,
                         int64_t out_channels, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                         int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w,
                         int64_t groups, void* y, int y_dtype, int y_layout, int variant, void* stream);

/* Fused-epilogue forms of the two weight-only ops (no counterpart in the
 * reference, whose models run bias, residual add and activation as separate
 * torch ops after the DIMQ layer: modules.py:36-47,104-122 feed F.relu / the
 * residual sum of the calling model).  Each output element becomes
 *   y = act(acc * scale + bias + residual)
 * in fp32 before the one rounding to y_dtype.  residual (nullable, any float
 * dtype in residual_dtype) has y's shape and memory order ([M, N] row-major
 * for Linear; y_layout for Conv2d) and may alias y.  activation: enum
 * dimq_activation.  The plain entry points above are these with residual
 * NULL and DIMQ_ACT_NONE. */
int dimq_linear_codebook_ex(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                            int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                            int64_t cb_size, const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                            const void* residual, int residual_dtype, int activation, int variant, void* stream);

/* Workspace form of dimq_linear_codebook_ex (same arguments, checks and
 * results, plus a caller-owned device workspace; the library allocates
 * nothing).  With a 16-byte aligned workspace of at least
 * dimq_linear_codebook_workspace_bytes, decode shapes (M <= 16, bits 2-4;
 * 4 < M with N % 64 == 0 and K % 1024 == 0, or K % 4096 == 0) split the k
 * range over work-groups and keep the fp32 partial sums there (a second,
 * small kernel adds them): more work-groups stream the weights, and for
 * M > 4 the activations are read by 64 columns per work-group instead of 16.
 * bf16 activations with 4 < M <= 16 and K in {1024, 2048, 4096} need no
 * workspace: one launch multiplies them as they are with bf16 hi + lo
 * weights.
 * Large-M shapes (M >= 2048, bits 2-4, K % 32 == 0, fp16 / bf16 / fp32 x,
 * 256-byte aligned workspace) decode the weights once per call into the
 * workspace as fp16 (and convert bf16 / fp32 activations to fp16 there with
 * per-row range flags), then run an fp16 GEMM on them.  Otherwise it is
 * dimq_linear_codebook_ex.  The query returns 0 for shapes that use no
 * workspace.  The workspace is written on `stream`; calls sharing one must
 * be ordered on it. */
int64_t dimq_linear_codebook_workspace_bytes(int64_t M, int64_t K, int64_t N, int bits, int x_dtype);
int dimq_linear_codebook_ex_ws(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                               int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                               int64_t cb_size, const void* bias, int bias_dtype, int64_t N, void* y, int y_dtype,
                               const void* residual, int residual_dtype, int activation, int variant, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* Batched weight pre-decode (no counterpart in the reference, whose LUT
 * kernels decode the packed indices inside every call,
 * csrc/dimq_gemm_lut.cu): the large-M path of dimq_linear_codebook_ex_ws
 * decodes one layer's weights per call in a launch of its own; a model
 * forward can instead decode all its layers' weights in one launch per bit
 * width and pass each layer its decode.  Job j reads packed_w / codebook as
 * dimq_linear_codebook_ex (bits 2-4, in_features % 32 == 0) and writes
 * dimq_codebook_predecode_bytes(out_features, in_features, bits) bytes at
 * `decoded` (256-byte aligned): W_hat as fp16 rows scaled by a power of two
 * per row, then the rows' fp32 factors.  The bytes are this library's
 * private layout, valid for dimq_linear_codebook_predecoded with the same
 * packed_w and codebook, until either changes. */
typedef struct {
  const uint8_t* packed_w;
  int64_t packed_numel;
  int bits;
  const void* codebook;
  int cb_dtype;
  int64_t cb_rows;
  int64_t cb_size;
  int64_t out_features;
  int64_t in_features;
  void* decoded;
} DimqPredecodeJob;
int64_t dimq_codebook_predecode_bytes(int64_t out_features, int64_t in_features, int bits);
int dimq_codebook_predecode_batch(const DimqPredecodeJob* jobs, int count, void* stream);

/* dimq_linear_codebook_ex_ws on weights decoded by
 * dimq_codebook_predecode_batch (no counterpart in the reference; same
 * arguments, checks and results as dimq_linear_codebook_ex_ws plus
 * `decoded`).  When the call takes the large-M path the weights come from
 * `decoded` and only bf16 / fp32 activations use the workspace (fp16 ones
 * none); other shapes ignore `decoded` and run as dimq_linear_codebook_ex_ws.
 * A workspace of dimq_linear_codebook_workspace_bytes always suffices. */
int dimq_linear_codebook_predecoded(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                                    int64_t packed_numel, int bits, const void* codebook, int cb_dtype,
                                    int64_t cb_rows, int64_t cb_size, const void* bias, int bias_dtype, int64_t N,
                                    void* y, int y_dtype, const void* residual, int residual_dtype, int activation,
                                    int variant, const void* decoded, void* workspace, int64_t workspace_bytes,
                                    void* stream);

/* Weight x activation codebook Linear (no kernel counterpart in the
 * reference: its QAT wrapper quantizes activations to activation_centers with
 * hard_quantize_weight before F.linear, quant/dimq_wrapper.py:80-85,
 * quant/dimq.py:197-221): y = Q(x) W_hat^T + b with
 * Q(x) = C_a[argmin_c (x - C_a[c])^2] (torch argmin semantics: first minimum,
 * NaN distances win).  act_centers: n_act <= 256 fp32 centres on the device.
 * The quantized activations go to the caller's workspace in x's dtype, as
 * the reference's centers[idx].to(x.dtype) (at least
 * dimq_linear_codebook_act_workspace_bytes, 16-byte aligned), then the
 * weight-codebook tiles run on them (fp16 matrix path with the fp32 recompute
 * of tiles outside the fp16 range, as dimq_linear_codebook).  With
 * DIMQ_VARIANT_SMALL_M and a shape dimq_linear_lut_act runs, the workspace
 * takes the activation indices instead and the index x index LUT gather
 * computes y. */
int64_t dimq_linear_codebook_act_workspace_bytes(int64_t M, int64_t K);
int dimq_linear_codebook_act(const void* x, int x_dtype, int64_t M, int64_t K, const uint8_t* packed_w,
                             int64_t packed_numel, int bits, const void* codebook, int cb_dtype, int64_t cb_rows,
                             int64_t cb_size, const float* act_centers, int64_t n_act, const void* bias, int bias_dtype,
                             int64_t N, void* y, int y_dtype, int variant, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* Weight x activation codebook product table (no kernel counterpart in the
 * reference; the LUT GEMM of its activation codebooks, quant/dimq_wrapper.py
 * :80-85 with quant/dimq.py:197-221): table[g][w][a] = w_codebook[g][w] *
 * act_centers[a] in fp32 (one rounding), g < rows, w < Kw, a < Ka <= 256.
 * act_centers are the values the activations take (the centres in the
 * activations' dtype, widened to fp32). */
int dimq_build_codebook_product_table(const void* w_codebook, int cw_dtype, int64_t rows, int64_t Kw,
                                      const float* act_centers, int64_t Ka, float* table, void* stream);

/* Index x index LUT GEMM of the weight x activation codebook Linear (decode
 * shapes; dimq_linear_codebook_act uses it with DIMQ_VARIANT_SMALL_M for
 * M <= 16, its default being the faster dequantize-then-GEMM form): y[m, n] = sum_k T[n or 0][w[n,k]][a[m,k]]
 * + bias[n] with T = codebook x act_centers rounded to x_dtype, formed per
 * work-group in LDS.  act_idx [M, K] uint8 activation-centre indices
 * (entries >= n_act read centre n_act - 1); M <= 16, K % 32 == 0, bits 1-4,
 * n_act <= 256; act_idx 16-byte and packed_w 4-byte aligned. */
int dimq_linear_lut_act(const uint8_t* act_idx, int64_t M, int64_t K, const uint8_t* packed_w, int64_t packed_numel,
                        int bits, const void* codebook, int cb_dtype, int64_t cb_rows, int64_t cb_size,
                        const float* act_centers, int64_t n_act, int x_dtype, const void* bias, int bias_dtype,
                        int64_t N, void* y, int y_dtype, void* stream);

/* Weight x activation codebook Conv2d (the Conv2d form of
 * dimq_linear_codebook_act): x replaced by its nearest activation centre in
 * x's dtype, written to the caller's workspace (at least
 * dimq_conv2d_codebook_act_workspace_bytes, 16-byte aligned, x's layout),
 * then dimq_conv2d_codebook_ex on it (no residual / activation). */
int64_t dimq_conv2d_codebook_act_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W);
int dimq_conv2d_codebook_act(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                             const uint8_t* packed_w, int64_t packed_numel, int bits, const uint32_t* prepared_w,
                             int64_t prepared_words, const void* codebook, int cb_dtype, int64_t cb_rows,
                             int64_t cb_size, const float* act_centers, int64_t n_act, const void* bias,
                             int bias_dtype, int64_t out_channels, int64_t kernel_h, int64_t kernel_w,
                             int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h,
                             int64_t dilation_w, int64_t groups, void* y, int y_dtype, int y_layout, int variant,
                             void* workspace, int64_t workspace_bytes, void* stream);

int dimq_conv2d_codebook_ex(const void* x, int x_dtype, int x_layout, int64_t B, int64_t C, int64_t H, int64_t W,
                            const uint8_t* packed_w, int64_t packed_numel, int bits, const uint32_t* prepared_w,
                            int64_t prepared_words, const void* codebook, int cb_dtype, int64_t cb_rows,
                            int64_t cb_size, const void* bias, int bias_dtype, int64_t out_channels,
                            int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                            int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t groups, void* y,
                            int y_dtype, int y_layout, const void* residual, int residual_dtype, int activation,
                            int variant, void* stream);

/* ---------------------------------------------------------------------------
 * 3. Support ops of the end-to-end workloads (not DIMQ ops: the reference
 *    runs torch's LayerNorm and max pooling between its quantized layers,
 *    train_dimq_vit.py / train_dimq_resnet.py via torchvision's models).
 * ------------------------------------------------------------------------- */

/* LayerNorm over the last dimension: y = (x - mean) * rstd * weight + bias,
 * mean and biased variance in fp32 per row, as torch.nn.functional.layer_norm.
 * x [rows, dim] fp16/bf16 with row stride ldx (elements), y [rows, dim]
 * contiguous in x's dtype; weight/bias [dim] (nullable) in wb_dtype.
 * dim % 8 == 0, dim <= 2048, 16-byte aligned x and y. */
int dimq_layer_norm(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx, const void* weight,
                    const void* bias, int wb_dtype, double eps, void* y, void* stream);
/* dimq_layer_norm with the output in y_dtype (fp16 or bf16) instead of x's
 * dtype: one rounding of the fp32 result to y_dtype (the ViT workload feeds
 * fp16 to its codebook GEMMs). */
int dimq_layer_norm_ex(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx, const void* weight,
                       const void* bias, int wb_dtype, double eps, void* y, int y_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * QAT kernels (the training step before the packed path; quant/dimq.py).
 * fp32 arithmetic on w.float() and centers (K <= 256 fp32 values on the
 * device), as the reference; d_ij = (w_i - c_j)^2, p_ij = softmax_j(-d_ij/tau).
 * Sums over elements go through per-work-group partials in the caller's
 * workspace (dimq_qat_workspace_bytes) and a fixed-order final pass.
 * aux: 2 floats per element, (min_j d_ij, log sum_j exp(-(d_ij - min d)/tau)),
 * written by a forward and read by its backward.
 * ------------------------------------------------------------------------- */
int64_t dimq_qat_workspace_bytes(int64_t n, int64_t n_centers);

/* dimq_softmin_loss (quant/dimq.py:244-273): loss = sum_i -tau (logsumexp_j(
 * -d_ij/tau) - log K), divided by n when mean_reduction ("mean_per_layer");
 * fp32 scalar into *loss (device). */
int dimq_softmin_loss_forward(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                              double tau, int mean_reduction, float* aux, float* loss, void* workspace,
                              int64_t workspace_bytes, void* stream);
/* Gradients of the sum reduction for the upstream scalar *grad_loss (device):
 * grad_w = g sum_j p_ij 2 (w_i - c_j) (nullable, grad_w_dtype),
 * grad_centers = -2 g sum_i p_ij (w_i - c_j) (fp32).  mean_reduction must be 0:
 * the mean's gradient is the sum's with g / n. */
int dimq_softmin_loss_backward(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                               double tau, int mean_reduction, const float* aux, const float* grad_loss, void* grad_w,
                               int grad_w_dtype, float* grad_centers, void* workspace, int64_t workspace_bytes,
                               void* stream);

/* soft_dequantize_weight (quant/dimq.py:224-241): out_i = sum_j p_ij c_j in
 * w's dtype; and its backward for the upstream grad_out:
 * grad_w_i = g_i sum_j p_ij (c_j - out_i)(-2 (w_i - c_j)/tau),
 * grad_c_j = sum_i g_i p_ij (1 + (c_j - out_i) 2 (w_i - c_j)/tau). */
int dimq_soft_dequantize_forward(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                                 double tau, void* out, float* aux, void* stream);
int dimq_soft_dequantize_backward(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers,
                                  double tau, const float* aux, const void* grad_out, int grad_out_dtype, void* grad_w,
                                  int grad_w_dtype, float* grad_centers, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/* separation_loss (quant/dimq.py:276-296): delta = eta * 6 * max(std(w), 1e-12)
 * / K (population std of w, n >= 1), loss = sum_{a<b} relu(delta -
 * sqrt((c_a - c_b)^2 + eps))^2 into *loss, and d loss / d centers (nullable;
 * the margin carries no gradient to w, as the reference's w.detach()). */
int dimq_separation_loss(const void* w, int w_dtype, int64_t n, const float* centers, int64_t n_centers, double eta,
                         double eps, float* loss, float* grad_centers, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* 2-D max pooling over channels-last activations (the ResNet-18 workload's
 * stem pool; the reference's ResNet runs torch's max_pool2d, torchvision
 * resnet18): y[b,oh,ow,c] = max over the window's in-image taps, NaN
 * propagating, as torch.nn.functional.max_pool2d (dilation 1, floor mode).
 * x [B,H,W,C] and y [B,OH,OW,C] contiguous NHWC in fp16/bf16, C % 8 == 0,
 * 16-byte aligned; OH = (H + 2 pad_h - kernel_h) / stride_h + 1. */
int dimq_max_pool2d_nhwc(const void* x, int x_dtype, int64_t B, int64_t C, int64_t H, int64_t W, int64_t kernel_h,
                         int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                         void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DIMQ_HIP_H_ */
