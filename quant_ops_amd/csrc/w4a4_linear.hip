// C ABI of the W4A4 FlatQuant linear layer: quantize (packed codes) then the
// GEMM against the weight's transposed view, bias in the GEMM epilogue, as the
// kernels of qo_flatquant_quantize and qo_int4_gemm(_bias) on one stream.
#include <stdio.h>

#include <mutex>

#include "common.h"

// Largest token count whose linear call reads the weight ahead: the small-M
// GEMM's range. Measured on 112 x 128 -> 4096 x 14336 bf16 (step, same
// process): 1 token 15.68 -> 15.41 us, 16 tokens 16.70 -> 16.02, 32 tokens
// 17.95 -> 17.34, 64 tokens 21.44 -> 20.69; at 96 and 128 tokens (the GEMM
// no longer waits on the weight) 26.7 and 29.7 us either way.
constexpr int64_t kReadAheadTokens = 64;

// A failure of the quantize or GEMM stage of a linear call: the stage's
// message, prefixed with the entry point the caller called, and its status.
static int inner_failed(const char* fn, int status) {
  char inner[512];
  snprintf(inner, sizeof(inner), "%s", qo_last_error());
  qo_set_error("%s: %s", fn, inner);
  return status;
}

static int linear_run(const char* fn, const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                      const void* right, int M, int N, float clip_ratio, const int32_t* weight, int64_t weight_ld,
                      int64_t out_features, const void* weight_scale, int weight_scale_dtype, const void* bias,
                      int32_t* codes, float* act_scales, void* out, int64_t out_ld, void* stream,
                      void* workspace = nullptr, int64_t workspace_bytes = 0) {
  using namespace qo;
  if (tokens < 0 || M < 1 || N < 1 || out_features < 1) {
    qo_set_error("%s: invalid sizes tokens=%lld M=%d N=%d out_features=%lld", fn, (long long)tokens, M, N,
                 (long long)out_features);
    return QO_ERR_SHAPE;
  }
  const int64_t features = (int64_t)M * N;
  if (features % 8 != 0) {
    qo_set_error("%s: features (%lld) must be divisible by 8 for int32 packing", fn, (long long)features);
    return QO_ERR_SHAPE;
  }
  if (x_ld < features || weight_ld < features / 8 || out_ld < out_features) {
    qo_set_error("%s: row stride below row length (x %lld < %lld, weight %lld < %lld, out %lld < %lld)", fn,
                 (long long)x_ld, (long long)features, (long long)weight_ld, (long long)(features / 8),
                 (long long)out_ld, (long long)out_features);
    return QO_ERR_SHAPE;
  }
  if (x_dtype != QO_DTYPE_F32 && x_dtype != QO_DTYPE_F16 && x_dtype != QO_DTYPE_BF16) {
    qo_set_error("%s: unsupported input dtype code %d", fn, x_dtype);
    return QO_ERR_DTYPE;
  }
  if (weight_scale_dtype != QO_DTYPE_F32 && weight_scale_dtype != QO_DTYPE_F16 &&
      weight_scale_dtype != QO_DTYPE_BF16) {
    qo_set_error("%s: unsupported weight scale dtype code %d", fn, weight_scale_dtype);
    return QO_ERR_DTYPE;
  }
  if (tokens == 0) return QO_OK;
  if (!x || !left || !right || !weight || !weight_scale || !codes || !act_scales || !out) {
    qo_set_error("%s: NULL pointer argument", fn);
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
  if (q != QO_OK) return inner_failed(fn, q);
  int g;
  if (workspace)   // the FP6 route where the workspace and the shape allow it
    g = qo_int4_gemm_ws(codes, features / 8, weight, 1, weight_ld, act_scales, QO_DTYPE_F32, weight_scale,
                        weight_scale_dtype, bias, out, x_dtype, out_ld, tokens, out_features, features, workspace,
                        workspace_bytes, stream);
  else if (bias)
    g = qo_int4_gemm_bias(codes, features / 8, weight, 1, weight_ld, act_scales, QO_DTYPE_F32, weight_scale,
                          weight_scale_dtype, bias, out, x_dtype, out_ld, tokens, out_features, features, stream);
  else
    g = qo_int4_gemm(codes, features / 8, weight, 1, weight_ld, act_scales, QO_DTYPE_F32, weight_scale,
                     weight_scale_dtype, out, x_dtype, out_ld, tokens, out_features, features, stream);
  return g == QO_OK ? g : inner_failed(fn, g);
}

extern "C" int qo_w4a4_linear(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                              const void* right, int M, int N, float clip_ratio, const int32_t* weight,
                              int64_t weight_ld, int64_t out_features, const void* weight_scale,
                              int weight_scale_dtype, const void* bias, int32_t* codes, float* act_scales, void* out,
                              int64_t out_ld, void* stream) {
  return linear_run("qo_w4a4_linear", x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, weight, weight_ld,
                    out_features, weight_scale, weight_scale_dtype, bias, codes, act_scales, out, out_ld, stream);
}

extern "C" int qo_w4a4_linear_ws(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                                 const void* right, int M, int N, float clip_ratio, const int32_t* weight,
                                 int64_t weight_ld, int64_t out_features, const void* weight_scale,
                                 int weight_scale_dtype, const void* bias, int32_t* codes, float* act_scales,
                                 void* out, int64_t out_ld, void* workspace, int64_t workspace_bytes, void* stream) {
  return linear_run("qo_w4a4_linear_ws", x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, weight, weight_ld,
                    out_features, weight_scale, weight_scale_dtype, bias, codes, act_scales, out, out_ld, stream,
                    workspace, workspace_bytes);
}

// The linear layer against a weight already in the FP6 operand layout
// (qo_int4_gemm_f6_convert of its [out, in/8] rows, done once): quantize, the
// codes converted into a_workspace, then the FP6 GEMM.
extern "C" int qo_w4a4_linear_f6w(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                                  const void* right, int M, int N, float clip_ratio, const void* weight_f6,
                                  int64_t weight_f6_bytes, int64_t out_features, const void* weight_scale,
                                  int weight_scale_dtype, const void* bias, int32_t* codes, float* act_scales,
                                  void* out, int64_t out_ld, void* a_workspace, int64_t a_workspace_bytes,
                                  void* stream) {
  using namespace qo;
  const char* fn = "qo_w4a4_linear_f6w";
  const int64_t features = (int64_t)M * N;
  if (tokens < 0 || M < 1 || N < 1 || out_features < 1 || features % 8 != 0 || x_ld < features ||
      out_ld < out_features || features > 65536) {
    qo_set_error("%s: invalid sizes or strides (tokens=%lld M=%d N=%d out_features=%lld)", fn, (long long)tokens, M, N,
                 (long long)out_features);
    return QO_ERR_SHAPE;
  }
  if (x_dtype != QO_DTYPE_F16 && x_dtype != QO_DTYPE_BF16) {
    qo_set_error("%s: input dtype code %d (the FP6 GEMM writes 16-bit outputs: F16 or BF16)", fn, x_dtype);
    return QO_ERR_DTYPE;
  }
  if (tokens == 0) return QO_OK;
  if (!weight_f6 || !a_workspace || !codes || !act_scales) {
    qo_set_error("%s: NULL pointer argument", fn);
    return QO_ERR_NULL_POINTER;
  }
  const int q = flatquant_quantize(x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, 1, codes, act_scales,
                                   stream, ReadAhead{});
  if (q != QO_OK) return inner_failed(fn, q);
  const int c = qo_int4_gemm_f6_convert(codes, features / 8, 1, tokens, features, a_workspace, a_workspace_bytes,
                                        stream);
  if (c != QO_OK) return inner_failed(fn, c);
  const int g = qo_int4_gemm_f6_run2(a_workspace, a_workspace_bytes, weight_f6, weight_f6_bytes, act_scales,
                                     QO_DTYPE_F32, weight_scale, weight_scale_dtype, bias, out, x_dtype, out_ld, tokens,
                                     out_features, features, stream);
  return g == QO_OK ? g : inner_failed(fn, g);
}

// ---------------------------------------------------------------------------
// The linear layer without caller buffers for the activation codes and
// scales: they are staged in `scratch`, one array per GPU that lives as long
// as the process. Every call on a GPU reuses that GPU's array (the quantize
// writes every code word and scale of the call before the GEMM reads them, so
// nothing needs clearing); calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
static constexpr int64_t kStagingBytes = QO_LINEAR_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kStagingBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_staging_mu;
static unsigned char* g_staging[kMaxDevices] = {};

// The array's device address on the current device, looked up once per device
// (the array's name in host code is only a handle for the lookup).
static int staging_on_current_device(void* stream, unsigned char** p) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    qo_set_error("qo_w4a4_linear_noalloc: no usable current device (hipGetDevice gave %d)", dev);
    return QO_ERR_LAUNCH;
  }
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev) != hipSuccess || sdev != dev) {
      qo_set_error("qo_w4a4_linear_noalloc: the stream belongs to device %d, not the current device %d", sdev, dev);
      return QO_ERR_UNSUPPORTED;
    }
  }
  std::lock_guard<std::mutex> lock(g_staging_mu);
  if (!g_staging[dev]) {
    void* q = nullptr;
    const hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !q) {
      qo_set_error("qo_w4a4_linear_noalloc: hipGetSymbolAddress of the staging array failed on device %d: %s", dev,
                   hipGetErrorString(e));
      return QO_ERR_LAUNCH;
    }
    g_staging[dev] = static_cast<unsigned char*>(q);
  }
  *p = g_staging[dev];
  return QO_OK;
}

extern "C" int qo_w4a4_linear_noalloc(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                                      const void* right, int M, int N, float clip_ratio, const int32_t* weight,
                                      int64_t weight_ld, int64_t out_features, const void* weight_scale,
                                      int weight_scale_dtype, const void* bias, void* out, int64_t out_ld,
                                      void* stream) {
  static const char* fn = "qo_w4a4_linear_noalloc";
  if (tokens <= 0 || M < 1 || N < 1 || ((int64_t)M * N) % 8 != 0)   // the checks (or nothing to do) of the run
    return linear_run(fn, x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, weight, weight_ld, out_features,
                      weight_scale, weight_scale_dtype, bias, nullptr, nullptr, out, out_ld, stream);
  // codes [tokens, M*N/8] int32 at offset 0, then the float32 scales at the
  // next 256-byte boundary
  const int64_t row_bytes = (int64_t)M * N / 2;
  if (tokens > kStagingBytes / 4 || row_bytes > kStagingBytes) {
    qo_set_error("%s: %lld tokens of %lld features exceed the %lld-byte staging array", fn, (long long)tokens,
                 (long long)M * N, (long long)kStagingBytes);
    return QO_ERR_SHAPE;
  }
  const int64_t codes_bytes = (tokens * row_bytes + 255) / 256 * 256;
  const int64_t need = codes_bytes + tokens * (int64_t)sizeof(float);
  if (need > kStagingBytes) {
    qo_set_error("%s: %lld tokens of %lld features need %lld bytes of staging, above the %lld-byte limit", fn,
                 (long long)tokens, (long long)M * N, (long long)need, (long long)kStagingBytes);
    return QO_ERR_SHAPE;
  }
  unsigned char* base = nullptr;
  const int st = staging_on_current_device(stream, &base);
  if (st != QO_OK) return st;
  return linear_run(fn, x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, weight, weight_ld, out_features,
                    weight_scale, weight_scale_dtype, bias, reinterpret_cast<int32_t*>(base),
                    reinterpret_cast<float*>(base + codes_bytes), out, out_ld, stream);
}
