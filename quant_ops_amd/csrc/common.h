// Shared device helpers for the gfx950 kernels of libquant_ops_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_ops_hip.h"

namespace qo {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));

// Hides a value's provenance from the optimizer. The reference rounds every
// float32 result to the input dtype as a separate step; without this barrier
// the backend folds (half)(a * b) and (half)fma(a, b, c) into v_fma_mix*_f16
// (one rounding of the exact result) and narrows (half)(a / b) of widened
// halves into a half-precision divide, both of which can round differently.
__device__ inline float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Element traits: storage type, conversion to float and round-to-nearest-even
// from float. `round` returns the D-rounded value as a float, which is what
// the reference fallback holds after every torch op on a D tensor.
struct F32T {
  using T = float;
  static constexpr int code = QO_DTYPE_F32;
  __device__ static inline float to_f(T v) { return v; }
  __device__ static inline T from_f(float v) { return v; }
  __device__ static inline float round(float v) { return v; }
};

struct F16T {
  using T = _Float16;
  static constexpr int code = QO_DTYPE_F16;
  __device__ static inline float to_f(T v) { return (float)v; }
  __device__ static inline T from_f(float v) { return (T)opaque(v); }
  __device__ static inline float round(float v) { return (float)(_Float16)opaque(v); }
};

struct BF16T {
  using T = __bf16;
  static constexpr int code = QO_DTYPE_BF16;
  __device__ static inline float to_f(T v) { return (float)v; }
  __device__ static inline T from_f(float v) { return (T)opaque(v); }
  __device__ static inline float round(float v) { return (float)(__bf16)opaque(v); }
};

// Load a scalar of a runtime dtype code (F32/F16/BF16) as float.
__device__ inline float load_scale(const void* p, int dtype, int64_t i) {
  if (dtype == QO_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == QO_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  return (float)reinterpret_cast<const __bf16*>(p)[i];
}

// Wave-wide (64 lanes) float max / min.
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace qo

// Thread-local error message used by qo_last_error().
void qo_set_error(const char* fmt, ...);
