// Shared device helpers for the gfx950 kernels of libquant_ops_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <tuple>
#include <type_traits>
#include <utility>

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

// Running maximum of |v| over pairs of 16-bit floats (fp16 or bf16) packed in
// a dword: with the sign bits cleared, their bit patterns order like the
// values, so one packed unsigned 16-bit max handles both halves.
__device__ inline uint32_t pk_absmax16(uint32_t m, uint32_t pair) {
  typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
  const v2u16 a = __builtin_bit_cast(v2u16, pair & 0x7FFF7FFFu);
  const v2u16 b = __builtin_bit_cast(v2u16, m);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}

// Wave-wide (64 lanes) maximum of unsigned values: DPP within each row of 16
// lanes, then the four row results through scalar reads. Every lane receives
// the result.
__device__ inline uint32_t wave_max_u32(uint32_t u) {
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x141, 0xF, 0xF, false));  // row_half_mirror
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x140, 0xF, 0xF, false));  // row_mirror
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)u, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)u, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)u, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)u, 48);
  return max(max(r0, r1), max(r2, r3));
}

// float(low / high half of p as fp16) * r: the exact product rounded once to
// float32, which is what converting and then multiplying gives, in one
// v_fma_mix_f32 (with a zero addend; only the sign of a zero product can
// differ, and no caller distinguishes it). p must not come straight from an
// MFMA: the wait states an MFMA result needs before a VALU read are not
// relied on around inline assembly.
__device__ inline float mul_f16lo(uint32_t p, float r) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(p), "v"(r));
  return d;
}
__device__ inline float mul_f16hi(uint32_t p, float r) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(p), "v"(r));
  return d;
}

// LDS-DMA of 16 bytes per lane: lane l's bytes land at LDS address lds + 16 l
// (lds is wave-uniform, passed in M0). Issued as inline assembly so the
// compiler's wait insertion does not see an LDS write it cannot order: with
// the builtin it falls back to waiting for every outstanding load before LDS
// reads at control-flow joins. The kernel orders these copies itself with
// explicit vmcnt waits and barriers; every other load stays visible to the
// compiler, and its own vmcnt waits remain correct (extra outstanding loads
// only make them stricter).
__device__ inline void dma16(const void* src, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// The same copy addressed as a wave-uniform 64-bit base (SGPRs) plus the
// lane's 32-bit byte offset.
__device__ inline void dma16_s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// LDS byte address of a __shared__ object (the value M0 takes for LDS-DMA).
template <class P>
__device__ inline uint32_t lds_addr(P* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Compute units of the current device (host side), for grid sizing; queried
// once per device and cached (thread-safe). 256 (MI355X) if the query fails.
inline int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < kMaxDevices) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Workgroup barriers without the release/acquire fences of __syncthreads():
// those fences wait for every outstanding vector-memory operation (vmcnt(0)),
// which would also wait for loads still in flight for later stages or tokens.
// The "memory" clobber keeps the compiler from moving memory accesses across
// the barrier; lds_barrier first waits for this wave's LDS accesses.
__device__ inline void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace qo

// Thread-local error message used by qo_last_error().
void qo_set_error(const char* fmt, ...);

namespace qo {

// Kernel routing overrides set through qo_set_kernel_routing (QO_ROUTE_* bits):
// one relaxed atomic load per dispatch decision.
extern std::atomic<unsigned> g_route_mask;
inline bool route_off(unsigned bit) { return (g_route_mask.load(std::memory_order_relaxed) & bit) != 0u; }

// Kernel launches of one C-ABI call. launch() starts a kernel with
// hipLaunchKernel (arguments converted to the kernel's parameter types) and
// keeps the first failure of the current call; launch_result() reports it.
// Errors that earlier, unrelated work left on the thread are neither reported
// as this call's nor consumed; an error of a launch made here is taken off the
// thread (hipGetLastError) so that the caller's next check does not see it
// again.
extern thread_local hipError_t g_launch_error;

inline void launch_begin() { g_launch_error = hipSuccess; }

template <class K, class Tup, size_t... I>
inline hipError_t launch_tuple(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Tup& args,
                               std::index_sequence<I...>) {
  void* ptrs[] = {static_cast<void*>(&std::get<I>(args))...};
  return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, lds, stream);
}

template <class... P, class... A>
inline void launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t stream, A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  std::tuple<std::decay_t<P>...> vals(std::forward<A>(args)...);
  const hipError_t e = launch_tuple(kernel, grid, block, lds, stream, vals, std::index_sequence_for<P...>{});
  if (e != hipSuccess) {
    if (g_launch_error == hipSuccess) g_launch_error = e;
    (void)hipGetLastError();
  }
}

// A read-ahead request carried by a quantize launch (the linear layer's decode
// path): the workgroup slots that a few tokens leave idle read the weight rows
// that the following small-M GEMM streams, each on the XCD whose L2 that
// GEMM's workgroup will read them through (GEMM workgroup j streams rows
// 16 j .. 16 j + 15 and runs on XCD j % 8). Results do not depend on it.
struct ReadAhead {
  const void* p = nullptr;   // weight rows, 16-byte aligned
  int64_t rows = 0;
  int64_t row_bytes = 0;     // row stride in bytes (a multiple of 16)
  int64_t row_len = 0;       // bytes read from the start of each row (a multiple of 16)
};

// qo_flatquant_quantize with a read-ahead request (honoured by the kernels
// that leave CUs idle; ignored by the others). Same arguments and results.
int flatquant_quantize(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left, const void* right,
                       int M, int N, float clip_ratio, int pack_int32, void* out_codes, float* out_scales,
                       void* stream, const ReadAhead& ahead);

inline int launch_result(const char* who) {
  const hipError_t e = g_launch_error;
  g_launch_error = hipSuccess;
  if (e == hipSuccess) return QO_OK;
  qo_set_error("%s: launch failed: %s", who, hipGetErrorString(e));
  return QO_ERR_LAUNCH;
}

}  // namespace qo
