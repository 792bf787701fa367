// C ABI of the W4A4 FlatQuant linear layer: quantize (packed codes) then the
// GEMM against the weight's transposed view, bias in the GEMM epilogue, as the
// kernels of qo_flatquant_quantize and qo_int4_gemm(_bias) on one stream.
#include "common.h"

// Largest token count whose linear call reads the weight ahead: the small-M
// GEMM's range. Measured on 112 x 128 -> 4096 x 14336 bf16 (step, same
// process): 1 token 15.68 -> 15.41 us, 16 tokens 16.70 -> 16.02, 32 tokens
// 17.95 -> 17.34, 64 tokens 21.44 -> 20.69.
constexpr int64_t kReadAheadTokens = 64;

extern "C" int qo_w4a4_linear(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                              const void* right, int M, int N, float clip_ratio, const int32_t* weight,
                              int64_t weight_ld, int64_t out_features, const void* weight_scale,
                              int weight_scale_dtype, const void* bias, int32_t* codes, float* act_scales, void* out,
                              int64_t out_ld, void* stream) {
  using namespace qo;
  if (tokens < 0 || M < 1 || N < 1 || out_features < 1) {
    qo_set_error("qo_w4a4_linear: invalid sizes tokens=%lld M=%d N=%d out_features=%lld", (long long)tokens, M, N,
                 (long long)out_features);
    return QO_ERR_SHAPE;
  }
  const int64_t features = (int64_t)M * N;
  if (features % 8 != 0) {
    qo_set_error("qo_w4a4_linear: features (%lld) must be divisible by 8 for int32 packing", (long long)features);
    return QO_ERR_SHAPE;
  }
  if (x_ld < features || weight_ld < features / 8 || out_ld < out_features) {
    qo_set_error("qo_w4a4_linear: row stride below row length (x %lld < %lld, weight %lld < %lld, out %lld < %lld)",
                 (long long)x_ld, (long long)features, (long long)weight_ld, (long long)(features / 8),
                 (long long)out_ld, (long long)out_features);
    return QO_ERR_SHAPE;
  }
  if (x_dtype != QO_DTYPE_F32 && x_dtype != QO_DTYPE_F16 && x_dtype != QO_DTYPE_BF16) {
    qo_set_error("qo_w4a4_linear: unsupported input dtype code %d", x_dtype);
    return QO_ERR_DTYPE;
  }
  if (weight_scale_dtype != QO_DTYPE_F32 && weight_scale_dtype != QO_DTYPE_F16 &&
      weight_scale_dtype != QO_DTYPE_BF16) {
    qo_set_error("qo_w4a4_linear: unsupported weight scale dtype code %d", weight_scale_dtype);
    return QO_ERR_DTYPE;
  }
  if (tokens == 0) return QO_OK;
  if (!x || !left || !right || !weight || !weight_scale || !codes || !act_scales || !out) {
    qo_set_error("qo_w4a4_linear: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  // Packed codes, then the GEMM against the weight's transposed view. At
  // decode token counts the quantize launch reads the weight ahead with the
  // workgroup slots its tokens leave idle, into the L2 of the XCD that will
  // stream each row block (kernels that leave no CU idle ignore the request).
  ReadAhead ahead;
  if (tokens <= kReadAheadTokens && !route_off(QO_ROUTE_LINEAR_NO_READ_AHEAD)) {
    ahead.p = weight;
    ahead.rows = out_features;
    ahead.row_bytes = weight_ld * (int64_t)sizeof(int32_t);
    ahead.row_len = features / 2;
  }
  const int q = flatquant_quantize(x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, 1, codes, act_scales,
                                   stream, ahead);
  if (q != QO_OK) return q;
  return bias ? qo_int4_gemm_bias(codes, features / 8, weight, 1, weight_ld, act_scales, QO_DTYPE_F32, weight_scale,
                                  weight_scale_dtype, bias, out, x_dtype, out_ld, tokens, out_features, features,
                                  stream)
              : qo_int4_gemm(codes, features / 8, weight, 1, weight_ld, act_scales, QO_DTYPE_F32, weight_scale,
                             weight_scale_dtype, out, x_dtype, out_ld, tokens, out_features, features, stream);
}
