// Device helpers of the W4A4 GEMM shared by every kernel that multiplies
// packed int4 codes on the i8 MFMA (the GEMM kernels and the fused decode
// linear kernel): output conversions, the epilogue arithmetic, nibble
// widening and scale loads.
//
// Widening: XOR with 0x8 turns the offset code (q + 8) into q's 4-bit
// two's-complement pattern; placing it in the high half of a byte gives the
// int8 value 16 q. Both operands carry the factor 16, so an accumulator holds
// 256 acc, exact while 256 * 64 * K < 2^31 (K <= 65536); epilogues shift it
// back. Each packed word gives a "low" dword (nibbles 0, 2, 4, 6) and a "high"
// dword (nibbles 1, 3, 5, 7); both operands use the same k order.
#pragma once

#include <type_traits>

#include "common.h"

namespace qo {

// Conversions start from a materialised float32 (see opaque()).
struct OutF16 {
  using T = _Float16;
  __device__ static inline T cvt(float v) { return (T)opaque(v); }
};
struct OutBF16 {
  using T = __bf16;
  __device__ static inline T cvt(float v) { return (T)opaque(v); }
};
struct OutF32 {
  using T = float;
  __device__ static inline T cvt(float v) { return v; }
};

// Unpacked signed value of nibble i of a packed word.
__device__ inline int nib(uint32_t w, int i) { return (int)((w >> (4 * i)) & 0xF) - 8; }

// Epilogue value: (float(acc) * sa) * sb, two separately rounded float32 products.
__device__ inline float scale_out(int acc, float sa, float sb) {
  float v = (float)acc * sa;
  v = v * sb;
  return v;
}

// Optional bias in the output type, added to the rounded output as the
// reference's `output + bias.to(dtype)` does (one float32 add of the two
// output-type values, one rounding back).
template <class OT>
__device__ inline typename OT::T add_bias(typename OT::T v, const typename OT::T* bias, int64_t n) {
  return bias ? OT::cvt((float)v + (float)bias[n]) : v;
}

// widen16 in the form gfx950's three-input v_bitop3_b32 takes in one
// instruction per dword (plus the shift): (w << 4) ^ (0x88888888 << 4) and
// w ^ 0x88888888, each masked to the high nibbles.
__device__ inline void widen16_b3(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = ((w << 4) ^ 0x88888880u) & 0xF0F0F0F0u;
  hi = (w ^ 0x88888888u) & 0xF0F0F0F0u;
}

// Two packed words -> one 16-byte MFMA operand (low, high dword of each).
__device__ inline v4i widen_pair(int w0, int w1) {
  uint32_t l0, h0, l1, h1;
  widen16_b3((uint32_t)w0, l0, h0);
  widen16_b3((uint32_t)w1, l1, h1);
  return v4i{(int)l0, (int)h0, (int)l1, (int)h1};
}

// widen_pair of words 2h and 2h + 1 of a 16-byte register group: both words'
// shifts by one v_lshlrev_b64 (the bits crossing between the two words land
// in nibbles the mask drops; as C the compiler splits it into two 32-bit
// shifts). Same values as widen_pair.
__device__ inline v4i widen_pair64(const v4i& w, int h) {
  typedef unsigned long long u64;
  const uint32_t w0 = (uint32_t)w[2 * h], w1 = (uint32_t)w[2 * h + 1];
  u64 sh;
  asm("v_lshlrev_b64 %0, 4, %1" : "=v"(sh) : "v"(((u64)w1 << 32) | w0));
  return v4i{(int)(((uint32_t)sh ^ 0x88888880u) & 0xF0F0F0F0u), (int)((w0 ^ 0x88888888u) & 0xF0F0F0F0u),
             (int)(((uint32_t)(sh >> 32) ^ 0x88888880u) & 0xF0F0F0F0u), (int)((w1 ^ 0x88888888u) & 0xF0F0F0F0u)};
}

// Scale element i of a float32 / float16 / bfloat16 vector (dtype fixed at
// compile time).
template <int DT>
__device__ inline float scale_at(const void* p, int64_t i) {
  if constexpr (DT == QO_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == QO_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  else return (float)reinterpret_cast<const __bf16*>(p)[i];
}

// Raw bits of scale element i of a float32 / float16 / bfloat16 vector,
// loaded without a branch on the dtype: two 16-bit loads at selected
// addresses (both halves of a float32, or the 16-bit value twice). A kernel
// can request it before its main loop; nothing waits for it until the
// epilogue converts it (scale_from_bits).
__device__ inline uint32_t scale_bits(const void* p, int dtype, int64_t i) {
  const unsigned short* h = reinterpret_cast<const unsigned short*>(p);
  const int64_t w = dtype == QO_DTYPE_F32 ? 2 : 1;
  return (uint32_t)h[w * i] | ((uint32_t)h[w * i + (w - 1)] << 16);
}

__device__ inline float scale_from_bits(uint32_t bits, int dtype) {
  return dtype == QO_DTYPE_F32   ? __builtin_bit_cast(float, bits)
         : dtype == QO_DTYPE_F16 ? (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xFFFFu))
                                 : __builtin_bit_cast(float, bits << 16);
}

// Calls f(std::integral_constant<int, dtype>) for a runtime scale dtype code.
template <class F>
__device__ inline void with_scale_dtype(int code, F&& f) {
  if (code == QO_DTYPE_F32) f(std::integral_constant<int, QO_DTYPE_F32>{});
  else if (code == QO_DTYPE_F16) f(std::integral_constant<int, QO_DTYPE_F16>{});
  else f(std::integral_constant<int, QO_DTYPE_BF16>{});
}

// vmcnt waits of the pipelined kernels' LDS-DMA rings.
template <int N>
__device__ inline void gemm_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Wait until at most n groups of G copies are in flight, n a workgroup-uniform
// runtime count clamped to 0 .. MAXN (the counter takes only constants).
template <int G, int MAXN>
__device__ inline void gemm_wait_groups(int n) {
  if constexpr (MAXN <= 0) {
    gemm_wait_vmcnt<0>();
  } else {
    if (n >= MAXN) gemm_wait_vmcnt<G * MAXN>();
    else gemm_wait_groups<G, MAXN - 1>(n);
  }
}

// Output value of a 16-bit type as its bit pattern.
template <class OT>
__device__ inline uint32_t out_bits(typename OT::T v) {
  return (uint32_t)(uint16_t)__builtin_bit_cast(uint16_t, v);
}

// Second half of the staged epilogue of the tiled kernels: the workgroup copies the BM x BN tile of 16-bit values from LDS
// to C in 16-byte pieces, consecutive threads taking consecutive pieces of a
// row (rows and columns past the matrix edge are skipped; C rows that are not
// 16-byte aligned take element stores).
// NT: the 16-byte pieces as non-temporal stores (streamed to memory instead of
// kept dirty in L2).
template <int BM, int BN, int THREADS, class OT, bool NT = false>
__device__ __attribute__((always_inline)) inline void copy_out_c(const unsigned char* c_tile, int pitch, typename OT::T* out, int64_t ldc, int M,
                                  int N, int m0, int n0, int tid) {
  using T = typename OT::T;
  constexpr int PPR = BN * 2 / 16;   // 16-byte pieces per row
  static_assert(BN % 8 == 0 && (BM * PPR) % THREADS == 0, "pieces");
  const bool vec = ((uintptr_t)out % 16 == 0) && (ldc % 8 == 0);
#pragma unroll
  for (int it = 0; it < BM * PPR / THREADS; ++it) {
    const int p = tid + THREADS * it;
    const int row = p / PPR, q = p % PPR;
    const int m = m0 + row, n = n0 + 8 * q;
    if (m >= M || n >= N) continue;
    const v4i d = *reinterpret_cast<const v4i*>(c_tile + row * pitch + 16 * q);
    T* o = out + (int64_t)m * ldc + n;
    if (vec && n + 7 < N) {
      if constexpr (NT) __builtin_nontemporal_store(d, reinterpret_cast<v4i*>(o));
      else *reinterpret_cast<v4i*>(o) = d;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N) o[e] = __builtin_bit_cast(T, (uint16_t)((uint32_t)d[e / 2] >> (16 * (e % 2))));
    }
  }
}

// The FP6 route of the tiled GEMM (int4_gemm_f6.hip): workspace bytes for an
// M x N x K product, and the two launches (operand conversion into the
// workspace, then the FP6 GEMM) for 16-bit outputs, M >= 1, N >= 1,
// K <= 65536 and any strides of A and B.
int64_t f6_workspace_bytes(int64_t M, int64_t N, int64_t K);
template <class OT>
void f6_gemm_launch(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, const void* sa,
                    int sad, const void* sb, int sbd, typename OT::T* out, int64_t ldc, const typename OT::T* bias,
                    int64_t M, int64_t N, int64_t K, void* workspace, hipStream_t stream);
// The two halves of f6_gemm_launch: the conversion of A and / or B (either
// pointer null: that operand is left as it is in the workspace), and the GEMM
// on a workspace holding both.
void f6_prepare(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, int64_t M, int64_t N,
                int64_t K, void* workspace, hipStream_t stream);
template <class OT>
void f6_run(const void* sa, int sad, const void* sb, int sbd, typename OT::T* out, int64_t ldc,
            const typename OT::T* bias, int64_t M, int64_t N, int64_t K, const void* workspace, hipStream_t stream);
// One operand (rows R: word p of row r at src[r * s_r + p * s_p], s_p or s_r
// 1) converted into dst (f6_operand_bytes(R, K) bytes), and the GEMM on two
// separately held operands (a prepared weight, converted once).
int64_t f6_operand_bytes(int64_t rows, int64_t K);
void f6_convert_operand(const int32_t* src, int64_t s_r, int64_t s_p, int64_t R, int64_t K, void* dst,
                        hipStream_t stream);
template <class OT>
void f6_run2(const void* a6, const void* b6, const void* sa, int sad, const void* sb, int sbd, typename OT::T* out,
             int64_t ldc, const typename OT::T* bias, int64_t M, int64_t N, int64_t K, hipStream_t stream);

}  // namespace qo
