// torch operator registration for the quant_ops namespace, backed by the C ABI
// of libquant_ops_hip.so.
//
// Schemas are those of the reference (flatquant/kernels/cuda_quant_kernel.cu:407-409,
// int4_matmul/kernels/cuda_int4_matmul_kernel.cu:207-209), so callers of
// torch.ops.quant_ops.* and graph captures see the same operators. The others
// are additions of this build: int4_matmul_ex (output dtype choice),
// int4_matmul_bias (bias in the epilogue), w4a4_linear (the linear layer's
// quantize + GEMM as one operator) and dequantize_int4 (a device kernel
// for the reference's Python function).
//
// Unlike the reference, kernels go to the caller's current HIP stream and the
// host is never synchronised (cuda_quant_kernel.cu:379-385 synchronised the
// stream after launching on the legacy default stream).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "quant_ops_hip.h"

namespace {

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return QO_DTYPE_F32;
    case at::kHalf: return QO_DTYPE_F16;
    case at::kBFloat16: return QO_DTYPE_BF16;
    default: return -1;
  }
}

void check_status(int st, const char* op) {
  TORCH_CHECK(st == QO_OK, op, " failed: ", qo_status_string(st), ": ", qo_last_error());
}

void* current_stream(const at::Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// Same checks as cuda_kronecker_quant_int8 (cuda_quant_kernel.cu:324-329), plus
// the dtype agreement torch::matmul enforces there.
std::tuple<at::Tensor, at::Tensor> flatquant_dynamic_quantize(const at::Tensor& input, const at::Tensor& left_trans,
                                                              const at::Tensor& right_trans, double clip_ratio,
                                                              bool pack_int32) {
  TORCH_CHECK(input.dim() == 2, "flatquant_dynamic_quantize: input must be 2-D [tokens, features], got ",
              input.sizes());
  TORCH_CHECK(left_trans.dim() == 2 && left_trans.size(0) == left_trans.size(1),
              "flatquant_dynamic_quantize: left_trans must be square [M, M]");
  TORCH_CHECK(right_trans.dim() == 2 && right_trans.size(0) == right_trans.size(1),
              "flatquant_dynamic_quantize: right_trans must be square [N, N]");
  const int64_t T = input.size(0);
  const int64_t M = left_trans.size(0), N = right_trans.size(0), F = M * N;
  TORCH_CHECK(input.size(-1) == F, "Input last dimension must equal M*N");
  TORCH_CHECK(F % 8 == 0 || !pack_int32, "Features must be divisible by 8 for int32 packing");
  const int code = dtype_code(input.scalar_type());
  TORCH_CHECK(code >= 0, "flatquant_dynamic_quantize: input dtype must be float32, float16 or bfloat16, got ",
              input.scalar_type());
  TORCH_CHECK(left_trans.scalar_type() == input.scalar_type() && right_trans.scalar_type() == input.scalar_type(),
              "flatquant_dynamic_quantize: left_trans / right_trans must have the input dtype ",
              input.scalar_type());
  TORCH_CHECK(input.is_cuda(), "flatquant_dynamic_quantize: input must be a GPU tensor");
  c10::DeviceGuard guard(input.device());

  at::Tensor x = input.stride(1) == 1 && input.stride(0) >= F ? input : input.contiguous();
  at::Tensor L = left_trans.to(input.device()).contiguous();
  at::Tensor R = right_trans.to(input.device()).contiguous();
  at::Tensor scales = at::empty({T}, input.options().dtype(at::kFloat));
  at::Tensor codes = pack_int32 ? at::empty({T, F / 8}, input.options().dtype(at::kInt))
                                : at::empty({T, F}, input.options().dtype(at::kChar));
  const int64_t ld = T > 0 ? x.stride(0) : F;
  check_status(qo_flatquant_quantize(x.data_ptr(), code, T, ld, L.data_ptr(), R.data_ptr(), (int)M, (int)N,
                                     (float)clip_ratio, pack_int32 ? 1 : 0, codes.data_ptr(),
                                     scales.data_ptr<float>(), current_stream(input)),
               "flatquant_dynamic_quantize");
  return {codes, scales};
}

// Same checks as cuda_int4_matmul (cuda_int4_matmul_kernel.cu:136-153); scales
// may also be float16 / bfloat16 (the fallback promotes them), and b may be the
// transposed view of a [N, K/8] weight.
at::Tensor int4_matmul_impl(const at::Tensor& a, const at::Tensor& b, const at::Tensor& scale_a,
                            const at::Tensor& scale_b, at::ScalarType out_dtype,
                            const std::optional<at::Tensor>& bias = std::nullopt) {
  TORCH_CHECK(a.is_cuda(), "a_packed must be on CUDA");
  TORCH_CHECK(b.is_cuda(), "b_packed must be on CUDA");
  TORCH_CHECK(scale_a.is_cuda(), "scale_a must be on CUDA");
  TORCH_CHECK(scale_b.is_cuda(), "scale_b must be on CUDA");
  TORCH_CHECK(a.scalar_type() == at::kInt, "a_packed must be int32");
  TORCH_CHECK(b.scalar_type() == at::kInt, "b_packed must be int32");
  const int sad = dtype_code(scale_a.scalar_type()), sbd = dtype_code(scale_b.scalar_type());
  TORCH_CHECK(sad >= 0, "scale_a must be float32, float16 or bfloat16");
  TORCH_CHECK(sbd >= 0, "scale_b must be float32, float16 or bfloat16");
  const int od = dtype_code(out_dtype);
  TORCH_CHECK(od >= 0, "out_dtype must be float16, bfloat16 or float32");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2, "a_packed and b_packed must be 2-D");
  const int64_t M = a.size(0), KP = a.size(1), N = b.size(1), K = KP * 8;
  TORCH_CHECK(b.size(0) == KP, "Matrix dimensions mismatch");
  TORCH_CHECK(scale_a.size(0) == M && scale_a.numel() == M, "scale_a dimension mismatch");
  TORCH_CHECK(scale_b.size(0) == N && scale_b.numel() == N, "scale_b dimension mismatch");
  c10::DeviceGuard guard(a.device());

  at::Tensor A = (a.stride(1) == 1 && (M <= 1 || a.stride(0) >= KP)) ? a : a.contiguous();
  at::Tensor B = b;
  if (!(b.stride(0) == 1 || b.stride(1) == 1)) B = b.contiguous();
  at::Tensor sa = scale_a.contiguous(), sb = scale_b.contiguous();
  at::Tensor out = at::empty({M, N}, a.options().dtype(out_dtype));
  int64_t bsp = B.stride(0), bsn = B.stride(1);
  if (KP == 1) bsp = 1;     // a single packed row: either stride works
  if (N == 1) bsn = 1;
  const int64_t lda = M > 0 ? A.stride(0) : KP;
  at::Tensor bv;
  if (bias.has_value()) {
    TORCH_CHECK(bias->is_cuda() && bias->numel() == N, "bias must be a GPU tensor of N elements");
    // the reference adds bias.to(output dtype) to the output
    bv = bias->to(out_dtype).contiguous();
  }
  // workspace of the FP6 route for the large shapes (the caching allocator's
  // blocks are 512-byte aligned)
  const int64_t ws_bytes = qo_int4_gemm_workspace_size(M, N, K, od);
  at::Tensor ws = ws_bytes > 0 ? at::empty({ws_bytes}, a.options().dtype(at::kByte)) : at::Tensor();
  check_status(qo_int4_gemm_ws(A.data_ptr<int32_t>(), lda, B.data_ptr<int32_t>(), bsp, bsn, sa.data_ptr(), sad,
                               sb.data_ptr(), sbd, bv.defined() ? bv.data_ptr() : nullptr, out.data_ptr(), od, N, M,
                               N, K, ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(a)),
               bias.has_value() ? "int4_matmul_bias" : "int4_matmul");
  return out;
}

at::Tensor int4_matmul(const at::Tensor& a, const at::Tensor& b, const at::Tensor& scale_a,
                       const at::Tensor& scale_b) {
  return int4_matmul_impl(a, b, scale_a, scale_b, at::kHalf);
}

at::Tensor int4_matmul_ex(const at::Tensor& a, const at::Tensor& b, const at::Tensor& scale_a,
                          const at::Tensor& scale_b, std::optional<at::ScalarType> out_dtype) {
  return int4_matmul_impl(a, b, scale_a, scale_b, out_dtype.value_or(at::kHalf));
}

at::Tensor int4_matmul_bias(const at::Tensor& a, const at::Tensor& b, const at::Tensor& scale_a,
                            const at::Tensor& scale_b, const at::Tensor& bias,
                            std::optional<at::ScalarType> out_dtype) {
  return int4_matmul_impl(a, b, scale_a, scale_b, out_dtype.value_or(at::kHalf), bias);
}

// The W4A4 linear layer (w4a4_flatquant_dynamic.py:168-266 on the GPU path):
// x [T, M*N], weight_packed int32 [out, M*N/8] (the GEMM uses its W.t() view),
// weight_scale [out] (float32 / float16 / bfloat16), optional bias; output in
// x's dtype.
at::Tensor w4a4_linear(const at::Tensor& x, const at::Tensor& left_trans, const at::Tensor& right_trans,
                       const at::Tensor& weight_packed, const at::Tensor& weight_scale, double clip_ratio,
                       const std::optional<at::Tensor>& bias) {
  TORCH_CHECK(x.dim() == 2, "w4a4_linear: x must be 2-D [tokens, features], got ", x.sizes());
  TORCH_CHECK(left_trans.dim() == 2 && left_trans.size(0) == left_trans.size(1),
              "w4a4_linear: left_trans must be square [M, M]");
  TORCH_CHECK(right_trans.dim() == 2 && right_trans.size(0) == right_trans.size(1),
              "w4a4_linear: right_trans must be square [N, N]");
  const int64_t T = x.size(0), M = left_trans.size(0), N = right_trans.size(0), F = M * N;
  TORCH_CHECK(x.size(1) == F, "Input last dimension must equal M*N");
  TORCH_CHECK(F % 8 == 0, "Features must be divisible by 8 for int32 packing");
  const int code = dtype_code(x.scalar_type());
  TORCH_CHECK(code >= 0, "w4a4_linear: x dtype must be float32, float16 or bfloat16, got ", x.scalar_type());
  TORCH_CHECK(left_trans.scalar_type() == x.scalar_type() && right_trans.scalar_type() == x.scalar_type(),
              "w4a4_linear: left_trans / right_trans must have x's dtype ", x.scalar_type());
  TORCH_CHECK(weight_packed.scalar_type() == at::kInt && weight_packed.dim() == 2 && weight_packed.size(1) * 8 == F,
              "w4a4_linear: weight_packed must be int32 [out_features, M*N/8]");
  const int64_t NO = weight_packed.size(0);
  const int swd = dtype_code(weight_scale.scalar_type());
  TORCH_CHECK(swd >= 0, "w4a4_linear: weight_scale must be float32, float16 or bfloat16");
  TORCH_CHECK(weight_scale.numel() == NO, "w4a4_linear: weight_scale must hold one value per output channel");
  TORCH_CHECK(x.is_cuda() && weight_packed.is_cuda() && weight_scale.is_cuda(),
              "w4a4_linear: x, weight_packed and weight_scale must be GPU tensors");
  c10::DeviceGuard guard(x.device());

  at::Tensor X = x.stride(1) == 1 && x.stride(0) >= F ? x : x.contiguous();
  at::Tensor L = left_trans.to(x.device()).contiguous();
  at::Tensor R = right_trans.to(x.device()).contiguous();
  at::Tensor W = weight_packed.stride(1) == 1 && weight_packed.stride(0) >= F / 8 ? weight_packed
                                                                                  : weight_packed.contiguous();
  at::Tensor sw = weight_scale.reshape({NO}).contiguous();
  at::Tensor bv;
  if (bias.has_value()) {
    TORCH_CHECK(bias->is_cuda() && bias->numel() == NO, "bias must be a GPU tensor of out_features elements");
    bv = bias->to(x.scalar_type()).reshape({NO}).contiguous();   // the reference adds bias.to(dtype)
  }
  at::Tensor codes = at::empty({T, F / 8}, x.options().dtype(at::kInt));
  at::Tensor scales = at::empty({T}, x.options().dtype(at::kFloat));
  at::Tensor out = at::empty({T, NO}, x.options());
  // the GEMM's FP6 route at large token counts (0 bytes: not taken)
  const int64_t ws_bytes = qo_int4_gemm_workspace_size(T, NO, F, code);
  at::Tensor ws = ws_bytes > 0 ? at::empty({ws_bytes}, x.options().dtype(at::kByte)) : at::Tensor();
  check_status(qo_w4a4_linear_ws(X.data_ptr(), code, T, T > 0 ? X.stride(0) : F, L.data_ptr(), R.data_ptr(), (int)M,
                                 (int)N, (float)clip_ratio, W.data_ptr<int32_t>(), NO > 0 ? W.stride(0) : F / 8, NO,
                                 sw.data_ptr(), swd, bv.defined() ? bv.data_ptr() : nullptr,
                                 codes.data_ptr<int32_t>(), scales.data_ptr<float>(), out.data_ptr(), NO,
                                 ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(x)),
               "w4a4_linear");
  return out;
}

at::Tensor dequantize_int4(const at::Tensor& quantized, const at::Tensor& scales, bool packed_int32) {
  TORCH_CHECK(quantized.is_cuda() && scales.is_cuda(), "dequantize_int4: tensors must be on the GPU");
  TORCH_CHECK(quantized.dim() == 2, "dequantize_int4: quantized must be 2-D");
  TORCH_CHECK(quantized.scalar_type() == (packed_int32 ? at::kInt : at::kChar),
              "dequantize_int4: quantized must be ", packed_int32 ? "int32" : "int8");
  const int sd = dtype_code(scales.scalar_type());
  TORCH_CHECK(sd >= 0, "dequantize_int4: scales must be float32, float16 or bfloat16");
  const int64_t T = quantized.size(0);
  const int64_t F = packed_int32 ? quantized.size(1) * 8 : quantized.size(1);
  TORCH_CHECK(scales.numel() == T, "dequantize_int4: scales must hold one value per token");
  c10::DeviceGuard guard(quantized.device());
  at::Tensor q = quantized.contiguous();
  at::Tensor s = scales.contiguous();
  at::Tensor out = at::empty({T, F}, quantized.options().dtype(at::kFloat));
  check_status(qo_dequantize_int4(q.data_ptr(), packed_int32 ? 1 : 0, s.data_ptr(), sd, T, F,
                                  out.data_ptr<float>(), current_stream(quantized)),
               "dequantize_int4");
  return out;
}

}  // namespace

TORCH_LIBRARY(quant_ops, m) {
  m.def(
      "flatquant_dynamic_quantize(Tensor input, Tensor left_trans, Tensor right_trans, float clip_ratio=1, "
      "bool pack_int32=False) -> (Tensor, Tensor)");
  m.def("int4_matmul(Tensor a, Tensor b, Tensor scale_a, Tensor scale_b) -> Tensor");
  m.def("int4_matmul_ex(Tensor a, Tensor b, Tensor scale_a, Tensor scale_b, ScalarType? out_dtype=None) -> Tensor");
  m.def("dequantize_int4(Tensor quantized, Tensor scales, bool packed_int32=False) -> Tensor");
  m.def(
      "int4_matmul_bias(Tensor a, Tensor b, Tensor scale_a, Tensor scale_b, Tensor bias, "
      "ScalarType? out_dtype=None) -> Tensor");
  m.def(
      "w4a4_linear(Tensor x, Tensor left_trans, Tensor right_trans, Tensor weight_packed, Tensor weight_scale, "
      "float clip_ratio=1, Tensor? bias=None) -> Tensor");
}

TORCH_LIBRARY_IMPL(quant_ops, CUDA, m) {
  m.impl("flatquant_dynamic_quantize", &flatquant_dynamic_quantize);
  m.impl("int4_matmul", &int4_matmul);
  m.impl("int4_matmul_ex", &int4_matmul_ex);
  m.impl("dequantize_int4", &dequantize_int4);
  m.impl("int4_matmul_bias", &int4_matmul_bias);
  m.impl("w4a4_linear", &w4a4_linear);
}
