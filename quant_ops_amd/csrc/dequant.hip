// Dequantize int4 codes to float32: out[t, f] = float(q[t, f]) * float(scale[t]).
//
// Replaces dequantize_int4 (flatquant/ops.py:156-178), which the reference runs
// as eight strided torch passes for the packed layout. HBM-bound: 4 bytes of
// packed codes (or 8 int8 codes) in, 32 bytes of float32 out per 8 features.
// The vector kernels write with non-temporal stores (whole 16-byte pieces,
// each store instruction 1 KiB of a row): the float32 output streams to memory
// instead of waiting in L2 for the write-back at the kernel's end (config 2's
// codes: 11.6 -> 7.6 us, same process, outputs equal).
#include "common.h"

namespace qo {

// int8 codes, 8 per thread (features % 8 == 0, aligned).
__global__ void __launch_bounds__(256)
dequant_i8_kernel(const void* __restrict__ codes, const void* __restrict__ scales, int sd, int64_t tokens,
                  int64_t words_per_row, float* __restrict__ out) {
  const int64_t total = tokens * words_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / words_per_row;
    const float s = load_scale(scales, sd, t);
    float v[8];
    const v2i c = reinterpret_cast<const v2i*>(codes)[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = (float)(int8_t)((uint32_t)c[0] >> (8 * j)) * s;
      v[4 + j] = (float)(int8_t)((uint32_t)c[1] >> (8 * j)) * s;
    }
    v4f* o = reinterpret_cast<v4f*>(out + i * 8);
    __builtin_nontemporal_store(v4f{v[0], v[1], v[2], v[3]}, o);
    __builtin_nontemporal_store(v4f{v[4], v[5], v[6], v[7]}, o + 1);
  }
}

// Packed codes, one token row per blockIdx.y (rows past gridDim.y loop), 256
// words per block along the row. Each store instruction of a wave writes 1 KiB
// of contiguous float32: lane l writes outputs 4l .. 4l+3 of a 32-word group,
// i.e. nibbles 4(l%2) .. 4(l%2)+3 of word l/2 (two lanes share a word, read
// twice from cache), and the token's scale is read once per thread.
__global__ void __launch_bounds__(256)
dequant_rows_kernel(const int32_t* __restrict__ codes, const void* __restrict__ scales, int sd, int64_t tokens,
                    int64_t words_per_row, float* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 1, half = lane >> 1;
  for (int64_t t = blockIdx.y; t < tokens; t += gridDim.y) {
    const float s = load_scale(scales, sd, t);
    const int32_t* row = codes + t * words_per_row;
    float* orow = out + t * words_per_row * 8;
    // this wave's two 32-word groups of the block's 128 words
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int64_t w = (int64_t)blockIdx.x * 256 + wave * 64 + g * 32 + half;
      if (w >= words_per_row) continue;
      const uint32_t bits = (uint32_t)row[w] >> (16 * sub);
      v4f v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (float)((int)((bits >> (4 * j)) & 0xF) - 8) * s;
      __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(orow + w * 8 + 4 * sub));
    }
  }
}

// Any alignment of the output, packed codes: one output per thread.
__global__ void __launch_bounds__(256)
dequant_packed_any(const int32_t* __restrict__ codes, const void* __restrict__ scales, int sd, int64_t tokens,
                   int64_t features, float* __restrict__ out) {
  const int64_t total = tokens * features;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const uint32_t w = (uint32_t)codes[i / 8];   // rows are whole words (features % 8 == 0)
    out[i] = (float)((int)((w >> (4 * (i % 8))) & 0xF) - 8) * load_scale(scales, sd, i / features);
  }
}

// Tail-safe variant for features % 8 != 0 (int8 codes only).
__global__ void __launch_bounds__(256)
dequant_i8_any(const int8_t* __restrict__ codes, const void* __restrict__ scales, int sd, int64_t tokens,
               int64_t features, float* __restrict__ out) {
  const int64_t total = tokens * features;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256)
    out[i] = (float)codes[i] * load_scale(scales, sd, i / features);
}

}  // namespace qo

extern "C" int qo_dequantize_int4(const void* codes, int pack_int32, const void* scales, int scale_dtype,
                                  int64_t tokens, int64_t features, float* out, void* stream) {
  using namespace qo;
  if (tokens < 0 || features < 0 || (pack_int32 && features % 8 != 0)) {
    qo_set_error("qo_dequantize_int4: invalid sizes tokens=%lld features=%lld", (long long)tokens,
                 (long long)features);
    return QO_ERR_SHAPE;
  }
  if (scale_dtype != QO_DTYPE_F32 && scale_dtype != QO_DTYPE_F16 && scale_dtype != QO_DTYPE_BF16) {
    qo_set_error("qo_dequantize_int4: unsupported scale dtype code %d", scale_dtype);
    return QO_ERR_DTYPE;
  }
  if (tokens == 0 || features == 0) return QO_OK;
  if (!codes || !scales || !out) {
    qo_set_error("qo_dequantize_int4: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_begin();
  const bool vec = (features % 8 == 0) && ((uintptr_t)out % 16 == 0) && (pack_int32 || (uintptr_t)codes % 8 == 0);
  if (vec) {
    const int64_t wpr = features / 8;
    int64_t blocks = (tokens * wpr + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (pack_int32) {
      const int64_t bx = (wpr + 255) / 256;
      const unsigned by = (unsigned)std::min<int64_t>(tokens, 65535);
      launch(dequant_rows_kernel, dim3((unsigned)bx, by), dim3(256), 0, s,
                         reinterpret_cast<const int32_t*>(codes), scales, scale_dtype, tokens, wpr, out);
    }
    else
      launch(dequant_i8_kernel, dim3((unsigned)blocks), dim3(256), 0, s, codes, scales, scale_dtype,
                         tokens, wpr, out);
  } else {
    int64_t blocks = (tokens * features + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (pack_int32)
      launch(dequant_packed_any, dim3((unsigned)blocks), dim3(256), 0, s,
                         reinterpret_cast<const int32_t*>(codes), scales, scale_dtype, tokens, features, out);
    else
      launch(dequant_i8_any, dim3((unsigned)blocks), dim3(256), 0, s,
                         reinterpret_cast<const int8_t*>(codes), scales, scale_dtype, tokens, features, out);
  }
  return launch_result("qo_dequantize_int4");
}
