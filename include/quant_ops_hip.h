/*
 * quant_ops_hip.h — C ABI of the MI355X (gfx950) FlatQuant W4A4 hot path.
 *
 * libquant_ops_hip.so exports these entry points. They take plain device
 * pointers, sizes and strides (in elements), a dtype code and a HIP stream
 * (as void*, NULL = the null stream). They never allocate, never synchronise
 * the host, and return a status code (QO_OK = 0). Outputs are caller-owned.
 *
 * The reference binds the same work through pybind11 / TORCH_LIBRARY inside its
 * CUDA translation units; each entry point names the reference function it
 * replaces. The torch binding in quant_ops_amd/csrc/torch_ops.cpp registers
 * the reference's operator schemas on top of these calls.
 */
#ifndef QUANT_OPS_HIP_H
#define QUANT_OPS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types understood by the entry points. */
enum qo_dtype {
  QO_DTYPE_F32 = 0,
  QO_DTYPE_F16 = 1,
  QO_DTYPE_BF16 = 2,
  QO_DTYPE_I8 = 3,
  QO_DTYPE_I32 = 4
};

/* Status codes. The torch binding turns every non-zero code into a
 * RuntimeError carrying qo_status_string(code) and the failing condition. */
enum qo_status {
  QO_OK = 0,
  QO_ERR_NULL_POINTER = 1,  /* a required pointer is NULL */
  QO_ERR_SHAPE = 2,         /* inconsistent or out-of-range sizes */
  QO_ERR_DTYPE = 3,         /* dtype code not supported for that operand */
  QO_ERR_ALIGNMENT = 4,     /* pointer / stride not aligned as required */
  QO_ERR_UNSUPPORTED = 5,   /* valid request this build does not implement */
  QO_ERR_LAUNCH = 6         /* hipLaunchKernel of this call failed */
};

/* Human-readable name of a status code (static storage). */
const char* qo_status_string(int status);

/* Library version string, e.g. "0.1.0". */
const char* qo_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* qo_last_error(void);

/*
 * Kernel routing overrides, process-wide. Each QO_ROUTE_* bit takes one kernel
 * family out of the dispatch so that the fallback kernel for the same shape
 * runs instead; results are the same to the parity bars. Returns the previous
 * mask. Meant for cross-checking kernels against each other (the test suite)
 * and for diagnosis; production callers leave it at 0. No counterpart in the
 * reference (its dispatch has one kernel per operator). Calls racing with
 * quantize / GEMM calls on other threads see either mask.
 */
enum qo_route {
  QO_ROUTE_FQ_GENERIC = 1u << 0,     /* quantize: every shape on the generic kernel */
  QO_ROUTE_FQ_NO_WAVE = 1u << 1,     /* quantize: no one-wave-per-token kernel */
  QO_ROUTE_FQ_NO_DUO = 1u << 2,      /* quantize: no two-waves-per-token kernel */
  QO_ROUTE_FQ_NO_FEW = 1u << 3,      /* quantize: no few-token routing to the workgroup kernel */
  QO_ROUTE_GEMM_GENERIC = 1u << 4,   /* GEMM: every shape on the generic kernel */
  QO_ROUTE_GEMM_NO_DMA = 1u << 5,    /* GEMM: no LDS-DMA tiled kernel */
  QO_ROUTE_GEMM_NO_SKINNY = 1u << 6, /* GEMM: no small-M kernels */
  QO_ROUTE_LINEAR_NO_READ_AHEAD = 1u << 7, /* linear: no weight read-ahead in the quantize launch */
  QO_ROUTE_GEMM_NO_F6 = 1u << 8,     /* GEMM: no FP6 matrix-core route (qo_int4_gemm_ws) */
  QO_ROUTE_ALL = (1u << 9) - 1u
};
unsigned qo_set_kernel_routing(unsigned mask);

/*
 * Fused FlatQuant dynamic int4 quantization, one pass over X.
 *
 * Replaces cuda_kronecker_quant_int8 (flatquant/kernels/cuda_quant_kernel.cu:316-390),
 * the CUDA implementation behind quant_ops::flatquant_dynamic_quantize
 * (cuda_quant_kernel.cu:395-413). For every token t (row of X, viewed as an
 * M x N matrix, feature f = m*N + n) it computes Y = L^T (X R) with the
 * rounding points of the reference's PyTorch fallback (flatquant/ops.py:99-117),
 * the per-token scale s = max(|rnd(min Y * c)|, rnd(max Y * c)) / 7 (floored at
 * rnd(1e-8)), and codes clamp(round_half_even(rnd(Y / s)), -8, 7).
 *
 *   x           [tokens, M*N] of x_dtype (F32, F16 or BF16), row stride x_ld
 *               elements, unit inner stride
 *   left, right [M, M] and [N, N] row-major, same dtype as x
 *   clip_ratio  the reference's clip_ratio (applied as a float32 product)
 *   pack_int32  0: out_codes is int8 [tokens, M*N] (row stride M*N)
 *               1: out_codes is int32 [tokens, M*N/8]; word p holds features
 *                  8p..8p+7, code i in bits 4i..4i+3 as (q + 8)
 *   out_scales  float32 [tokens]: the scale rounded to x_dtype, as float32
 *
 * Any M and N up to M = 2559 are accepted; shapes outside the MFMA kernels'
 * tables run a VALU kernel with the same rounding points (slower), and those
 * whose X and Z rows exceed the LDS (fp32 above 20480 features, fp16 / bf16
 * above 40960) compute Y by column blocks.
 *
 * Errors: QO_ERR_SHAPE if M*N % 8 != 0 while pack_int32, tokens < 0, M or N < 1;
 * QO_ERR_DTYPE for other x_dtype codes; QO_ERR_UNSUPPORTED for M > 2559 on
 * the column-block path.
 */
int qo_flatquant_quantize(const void* x, int x_dtype, int64_t tokens, int64_t x_ld,
                          const void* left, const void* right, int M, int N,
                          float clip_ratio, int pack_int32,
                          void* out_codes, float* out_scales, void* stream);

/*
 * W4A4 GEMM: out[m, n] = rnd_out((float(acc[m, n]) * scale_a[m]) * scale_b[n]),
 * acc[m, n] = sum_k qa[m, k] * qb[k, n] exactly in int32.
 *
 * Replaces cuda_int4_matmul (int4_matmul/kernels/cuda_int4_matmul_kernel.cu:130-189),
 * the CUDA implementation behind quant_ops::int4_matmul
 * (cuda_int4_matmul_kernel.cu:194-214); numerics follow the fallback
 * int4_matmul_pytorch (int4_matmul/ops.py:69-103).
 *
 *   a        int32 [M, K/8], word (m, p) holds k = 8p..8p+7; row stride lda words
 *   b        int32 words, word (p, n) holds k = 8p..8p+7 of column n, located at
 *            b[p * b_stride_p + n * b_stride_n]. Either stride may be 1:
 *            b_stride_n == 1 is the reference's row-major [K/8, N] tensor,
 *            b_stride_p == 1 is the transposed view W.t() of a [N, K/8] weight.
 *   scale_a  [M] of scale_a_dtype (F32, F16, BF16)
 *   scale_b  [N] of scale_b_dtype (F32, F16, BF16)
 *   out      [M, N] of out_dtype (F16 as the reference, or BF16 / F32), row stride ldc
 *   K        multiple of 8, K < 2^21
 */
int qo_int4_gemm(const int32_t* a, int64_t lda,
                 const int32_t* b, int64_t b_stride_p, int64_t b_stride_n,
                 const void* scale_a, int scale_a_dtype,
                 const void* scale_b, int scale_b_dtype,
                 void* out, int out_dtype, int64_t ldc,
                 int64_t M, int64_t N, int64_t K, void* stream);

/*
 * qo_int4_gemm followed by the bias of the W4A4 linear layer, fused into the
 * epilogue: out[m, n] = rnd(rnd((acc * sa[m]) * sb[n]) + bias[n]), with bias
 * in out_dtype (N elements, not NULL). The two roundings are those of the
 * reference's `output + bias.to(dtype)` after the GEMM
 * (w4a4_flatquant_dynamic.py:262-264 on int4_matmul's output).
 */
int qo_int4_gemm_bias(const int32_t* a, int64_t lda,
                      const int32_t* b, int64_t b_stride_p, int64_t b_stride_n,
                      const void* scale_a, int scale_a_dtype,
                      const void* scale_b, int scale_b_dtype,
                      const void* bias,
                      void* out, int out_dtype, int64_t ldc,
                      int64_t M, int64_t N, int64_t K, void* stream);

/*
 * qo_int4_gemm (bias may be NULL, else as qo_int4_gemm_bias) with a caller
 * workspace, which lets large products take the FP6 matrix-core route: the
 * int4 codes of A and B are rewritten into the workspace as FP6 e2m3 values
 * q / 8 (exact), then multiplied on v_mfma_scale_f32_16x16x128_f8f6f4 with
 * block scales 2^3, whose float32 sums equal the exact int32 sums; the
 * outputs are bit for bit those of qo_int4_gemm. The same entry point as
 * cuda_int4_matmul (cuda_int4_matmul_kernel.cu:130-189), which needs no
 * workspace; the torch operator int4_matmul allocates it.
 *
 *   workspace        device memory, 256-byte aligned, workspace_bytes long;
 *                    only read and written by this call's kernels on stream
 *                    (calls sharing a workspace must be ordered)
 *   workspace_bytes  at least qo_int4_gemm_workspace_size(M, N, K, out_dtype)
 *                    for the FP6 route; a smaller (or NULL) workspace takes
 *                    qo_int4_gemm's kernels
 *
 * Errors: those of qo_int4_gemm.
 */
int qo_int4_gemm_ws(const int32_t* a, int64_t lda,
                    const int32_t* b, int64_t b_stride_p, int64_t b_stride_n,
                    const void* scale_a, int scale_a_dtype,
                    const void* scale_b, int scale_b_dtype,
                    const void* bias,
                    void* out, int out_dtype, int64_t ldc,
                    int64_t M, int64_t N, int64_t K,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes qo_int4_gemm_ws uses for an M x N x K product with outputs
 * of out_dtype: 0 when the shape does not take the FP6 route (M <= 256, float32
 * outputs, K > 65536, or QO_ROUTE_GEMM_NO_F6 or QO_ROUTE_GEMM_GENERIC set), else
 * qo_int4_gemm_f6_workspace_bytes(M, N, K): 0.75 (M + N) K bytes plus padding
 * (M and N up to multiples of 32, K up to a multiple of 128).
 */
int64_t qo_int4_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype);

/*
 * The two launches of qo_int4_gemm_ws's FP6 route, for callers that keep one
 * operand converted (a weight converted once and multiplied many times) or
 * time the kernels apart. No counterpart in the reference.
 *
 * qo_int4_gemm_f6_prepare converts A (a, lda as qo_int4_gemm) and / or B (b
 * and its strides as qo_int4_gemm, one of them 1) into the workspace; a NULL
 * a or b leaves that operand's part of the workspace as it is.
 * qo_int4_gemm_f6_run multiplies the two operands held in the workspace:
 * out = rnd((acc * sa[m]) * sb[n]) (+ bias as qo_int4_gemm_bias, bias may be
 * NULL), out_dtype F16 or BF16; bit for bit qo_int4_gemm's result for the
 * same codes. Both take any M, N >= 1 and K (multiple of 8) <= 65536, and
 * a workspace of qo_int4_gemm_f6_workspace_bytes(M, N, K) bytes, 256-byte
 * aligned; the workspace layout is internal and depends on (M, N, K) only.
 *
 * Errors: QO_ERR_SHAPE for sizes outside those bounds, a small or misaligned
 * workspace, lda or ldc too small, or B with no unit stride;
 * QO_ERR_NULL_POINTER; QO_ERR_DTYPE (run: other out_dtype codes).
 */
int64_t qo_int4_gemm_f6_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * The FP6 route with each operand in a buffer of its own, for a weight
 * converted once: qo_int4_gemm_f6_convert writes one operand of `rows` rows
 * (A's rows, or B's columns: word p of row r at src[r * row_stride +
 * p * word_stride], one stride 1) into dst (256-byte aligned,
 * qo_int4_gemm_f6_operand_bytes(rows, K) bytes); qo_int4_gemm_f6_run2
 * multiplies A (M rows) and B (N rows) held that way (both buffers 256-byte
 * aligned, QO_ERR_SHAPE otherwise), with the arguments and results of
 * qo_int4_gemm_f6_run. No counterpart in the reference.
 */
int64_t qo_int4_gemm_f6_operand_bytes(int64_t rows, int64_t K);
int qo_int4_gemm_f6_convert(const int32_t* src, int64_t row_stride, int64_t word_stride, int64_t rows,
                            int64_t K, void* dst, int64_t dst_bytes, void* stream);
int qo_int4_gemm_f6_run2(const void* a6, int64_t a6_bytes, const void* b6, int64_t b6_bytes,
                         const void* scale_a, int scale_a_dtype, const void* scale_b, int scale_b_dtype,
                         const void* bias, void* out, int out_dtype, int64_t ldc,
                         int64_t M, int64_t N, int64_t K, void* stream);
int qo_int4_gemm_f6_prepare(const int32_t* a, int64_t lda,
                            const int32_t* b, int64_t b_stride_p, int64_t b_stride_n,
                            int64_t M, int64_t N, int64_t K,
                            void* workspace, int64_t workspace_bytes, void* stream);
int qo_int4_gemm_f6_run(const void* scale_a, int scale_a_dtype,
                        const void* scale_b, int scale_b_dtype,
                        const void* bias, void* out, int out_dtype, int64_t ldc,
                        int64_t M, int64_t N, int64_t K,
                        const void* workspace, int64_t workspace_bytes, void* stream);

/*
 * W4A4 FlatQuant linear layer: per-token dynamic quantization of x with the
 * Kronecker transform (as qo_flatquant_quantize, packed codes), then the int4
 * GEMM against the packed weight with per-token x per-channel scales, output
 * in x's dtype, then + bias (as qo_int4_gemm_bias): those two calls on one
 * stream, so the output equals theirs bit for bit. At up to 64 tokens the
 * quantize launch also reads the weight ahead with the workgroup slots its
 * tokens leave idle (reads only; QO_ROUTE_LINEAR_NO_READ_AHEAD switches it
 * off), so that the GEMM finds the weight in L2.
 *
 * Replaces the GPU path of AscendW4A4FlatQuantDynamicLinearMethod.apply
 * (w4a4_flatquant_dynamic.py:168-266), which runs the quantize operator and
 * then the GEMM against weight.t().
 *
 *   x             [tokens, M*N] of x_dtype (F32, F16, BF16), row stride x_ld
 *   left, right   [M, M], [N, N] of x_dtype, contiguous
 *   weight        int32 [out_features, M*N/8] (packed codes, one row per
 *                 output channel), row stride weight_ld words
 *   weight_scale  [out_features] of weight_scale_dtype (F32, F16, BF16)
 *   bias          NULL or [out_features] of x_dtype
 *   codes         int32 [tokens, M*N/8], contiguous: the activation codes
 *   act_scales    float32 [tokens]: the activation scales
 *   out           [tokens, out_features] of x_dtype, row stride out_ld
 *
 * Errors: those of qo_flatquant_quantize and qo_int4_gemm; QO_ERR_SHAPE if
 * M*N % 8 != 0, out_features < 1 or a stride is below its row length.
 */
int qo_w4a4_linear(const void* x, int x_dtype, int64_t tokens, int64_t x_ld,
                   const void* left, const void* right, int M, int N, float clip_ratio,
                   const int32_t* weight, int64_t weight_ld, int64_t out_features,
                   const void* weight_scale, int weight_scale_dtype, const void* bias,
                   int32_t* codes, float* act_scales,
                   void* out, int64_t out_ld, void* stream);

/*
 * qo_w4a4_linear with a caller workspace for its GEMM, which then runs as
 * qo_int4_gemm_ws: at more than 256 tokens (with qo_int4_gemm_workspace_size(
 * tokens, out_features, M*N, x_dtype) bytes or more) on the FP6 route, the
 * codes and the weight converted into the workspace first. Same results as
 * qo_w4a4_linear bit for bit; the torch operator w4a4_linear passes one.
 * workspace may be NULL (then exactly qo_w4a4_linear).
 *
 * Errors: those of qo_w4a4_linear.
 */
/*
 * qo_w4a4_linear against a weight already converted to the FP6 operand layout
 * (qo_int4_gemm_f6_convert(weight, weight_ld, 1, out_features, M*N, ...),
 * once, weight_f6_bytes long): the codes of each call are converted into
 * a_workspace (qo_int4_gemm_f6_operand_bytes(tokens, M*N) bytes) and
 * multiplied on the FP6 route. Same outputs, codes and scales as
 * qo_w4a4_linear bit for bit; x_dtype F16 or BF16, M*N <= 65536. For the
 * serving step of a static weight (the per-call weight conversion of
 * qo_w4a4_linear_ws is skipped); no counterpart in the reference.
 *
 * Errors: those of qo_w4a4_linear and qo_int4_gemm_f6_run2.
 */
int qo_w4a4_linear_f6w(const void* x, int x_dtype, int64_t tokens, int64_t x_ld,
                       const void* left, const void* right, int M, int N, float clip_ratio,
                       const void* weight_f6, int64_t weight_f6_bytes, int64_t out_features,
                       const void* weight_scale, int weight_scale_dtype, const void* bias,
                       int32_t* codes, float* act_scales, void* out, int64_t out_ld,
                       void* a_workspace, int64_t a_workspace_bytes, void* stream);

int qo_w4a4_linear_ws(const void* x, int x_dtype, int64_t tokens, int64_t x_ld,
                      const void* left, const void* right, int M, int N, float clip_ratio,
                      const int32_t* weight, int64_t weight_ld, int64_t out_features,
                      const void* weight_scale, int weight_scale_dtype, const void* bias,
                      int32_t* codes, float* act_scales, void* out, int64_t out_ld,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * qo_w4a4_linear without caller buffers for the activation codes and scales,
 * for callers that cannot allocate device memory (HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference, whose apply allocates those intermediates. The codes and scales
 * go to one staging array per GPU, held from the first call on that GPU until
 * the process ends, of QO_LINEAR_NOALLOC_MAX_BYTES: tokens * M*N/2 bytes of
 * codes (rounded up to 256) plus tokens * 4 bytes of scales must fit. Nothing
 * is allocated per call. Calls that overlap on one GPU (other streams or host
 * threads) share the array and race. The output equals qo_w4a4_linear's bit
 * for bit.
 *
 * The array's device address is looked up (hipGetSymbolAddress) on the
 * first call on each GPU and kept for the life of the process, so a device
 * reset (hipDeviceReset) between calls is not supported.
 *
 * Arguments as qo_w4a4_linear, without codes and act_scales; stream must
 * belong to the current device.
 *
 * Errors: those of qo_w4a4_linear; QO_ERR_SHAPE when the staging does not
 * fit; QO_ERR_UNSUPPORTED when stream is on another device; QO_ERR_LAUNCH
 * when the array's address cannot be looked up.
 */
#define QO_LINEAR_NOALLOC_MAX_BYTES (32LL * 1024 * 1024)
int qo_w4a4_linear_noalloc(const void* x, int x_dtype, int64_t tokens, int64_t x_ld,
                           const void* left, const void* right, int M, int N, float clip_ratio,
                           const int32_t* weight, int64_t weight_ld, int64_t out_features,
                           const void* weight_scale, int weight_scale_dtype, const void* bias,
                           void* out, int64_t out_ld, void* stream);

/*
 * Dequantize int4 codes: out[t, f] = float(q[t, f]) * float(scales[t]) (float32).
 *
 * Replaces dequantize_int4 (flatquant/ops.py:156-178), which the reference runs
 * as torch element-wise operations.
 *
 *   codes        int8 [tokens, features] (pack_int32 = 0) or int32
 *                [tokens, features/8] (pack_int32 = 1), contiguous rows
 *   scales       [tokens] of scale_dtype (F32, F16, BF16)
 *   out          float32 [tokens, features], contiguous
 */
int qo_dequantize_int4(const void* codes, int pack_int32, const void* scales, int scale_dtype,
                       int64_t tokens, int64_t features, float* out, void* stream);

/*
 * Pack int8 codes into int32 words: word p of a row =
 * sum_i ((codes[8p + i] + 8) mod 256) << 4i (mod 2^32), i.e. code + 8 in
 * nibble i for codes in [-8, 7]; other int8 values wrap exactly as the
 * reference's int8 add / uint8 cast / int32 sum do.
 *
 * Replaces pack_int4_to_int32 (int4_matmul/ops.py:23-45) and the activation /
 * weight packing of pack_int4_to_int32_manual
 * (w4a4_flatquant_dynamic.py:43-67, after its clamp).
 *
 *   codes   int8 [rows, features], row stride codes_ld (elements)
 *   out     int32 [rows, features / 8], row stride out_ld; features % 8 == 0
 */
int qo_pack_int4_to_int32(const int8_t* codes, int64_t codes_ld, int64_t rows, int64_t features,
                          int32_t* out, int64_t out_ld, void* stream);

/*
 * Unpack int32 words into int8 codes: out[8p + i] = ((word_p >> 4i) & 0xF) - 8.
 *
 * Replaces unpack_int32_to_int4 (int4_matmul/ops.py:48-66).
 *
 *   words   int32 [rows, nwords], row stride words_ld (elements)
 *   out     int8 [rows, 8 * nwords], row stride out_ld
 */
int qo_unpack_int32_to_int4(const int32_t* words, int64_t words_ld, int64_t rows, int64_t nwords,
                            int8_t* out, int64_t out_ld, void* stream);

/*
 * Transpose a matrix of 32-bit words: out[c, r] = in[r, c].
 *
 * Converts a packed int4 weight between the GEMM's two B layouts, [K/8, N]
 * (word [p, n] holds k = 8p .. 8p+7 of column n) and [N, K/8] (row-major
 * W packed along K), which hold the same words. Replaces the
 * pack(b.T).T / .t().contiguous() round trips of
 * examples/int4_matmul_benchmark.py:21-22 and
 * w4a4_flatquant_dynamic.py:290-292.
 *
 *   in      int32 [rows, cols], row stride in_ld
 *   out     int32 [cols, rows], row stride out_ld
 */
int qo_transpose_int32(const int32_t* in, int64_t in_ld, int64_t rows, int64_t cols, int32_t* out,
                       int64_t out_ld, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QUANT_OPS_HIP_H */
