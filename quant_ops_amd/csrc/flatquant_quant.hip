// Fused FlatQuant dynamic int4 quantization for gfx950 (MI355X).
//
// One pass over X per token: Y = rnd_D(L^T rnd_D(X R)), per-token absmax scale,
// round-half-even codes clamped to [-8, 7], optional 8-nibble int32 packing.
// Replaces the reference's cuBLAS + scale_quant_kernel chain
// (flatquant/kernels/cuda_quant_kernel.cu:231-390) and follows the rounding
// points of its PyTorch fallback (flatquant/ops.py:99-130).
//
// Kernels:
//  * fq_wave_kernel   — one wave per token, M, N <= 64 (fp16 / bf16).
//  * fq_few_kernel    — N = 128, M in {64, 96, 112, 128}: four waves per token
//                       (one or two tokens in flight per workgroup).
//  * fq_few2_kernel   — the same routine in half the registers and LDS, two
//                       workgroups per CU (112 x 128 and 64 x 128).
//  * fq_duo_kernel    — a pair of waves per token, the same shapes (kept for
//                       cross-checks: QO_ROUTE_FQ_NO_FEW routes N = 128 to it).
//  * fq_mfma_kernel   — D in {fp16, bf16}, the listed shapes: M up to 176 zero-padded
//                       to 16 MB, N even up to 256 zero-padded to 32 NP.
//                       Both contractions on v_mfma_f32_16x16x32_{f16,bf16}; X is
//                       streamed into LDS by LDS-DMA one token group ahead (two
//                       stages, one where two do not fit); L is resident in VGPRs
//                       or LDS, R in VGPRs.
//  * fq_generic_kernel — any M, N, D in {fp32, fp16, bf16}; VALU fp32 FMA with the
//                       same rounding points. Used for shapes the MFMA kernels
//                       do not cover (and for fp32 inputs), X and Z in LDS.
//  * fq_generic_big_kernel — the same results where X and Z do not fit in LDS
//                       (fp32 above 20480 features, other shapes above 40960):
//                       Y by blocks of 16 columns, computed twice per token.
//                       M up to 2559.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace qo {

// ---------------------------------------------------------------------------
// Scale and code, shared by both kernels.
// ---------------------------------------------------------------------------

// Per-token scale from the raw (unrounded) fp32 extremes of Y. Rounding to D is
// monotonic, so rnd_D(max y) == max rnd_D(y): this is amax/amin of the D tensor
// (ops.py:108-109), then maximum(|rnd(min*c)|, rnd(max*c)) (ops.py:112), then
// rnd(./7) clamped below by rnd_D(1e-8) (ops.py:113).
template <class DT>
__device__ inline float fq_scale(float ymax_raw, float ymin_raw, float clip) {
  const float hi = DT::round(ymax_raw);
  const float lo = DT::round(ymin_raw);
  const float t_lo = DT::round(lo * clip);
  const float t_hi = DT::round(hi * clip);
  const float bound = fmaxf(fabsf(t_lo), t_hi);
  const float s = DT::round(opaque(bound) / 7.0f);
  return fmaxf(s, DT::round(1e-8f));
}

// The same scale from max |Y| of the D-rounded Y, valid for clip > 0:
// rounding to nearest even is sign-symmetric and monotonic, so
// max(|rnd(rnd(min) c)|, rnd(rnd(max) c)) = rnd(max |rnd(y)| c).
template <class DT>
__device__ inline float fq_scale_abs(float amax, float clip) {
  const float bound = DT::round(amax * clip);
  const float s = DT::round(opaque(bound) / 7.0f);
  return fmaxf(s, DT::round(1e-8f));
}

// Code of one element from its D-rounded quotient t = rnd_D(y / s):
// clamp(round_half_even(t), -8, 7) (ops.py:117). A NaN quotient (0/0 when an
// fp16 token's scale rounds to 0) becomes 0 through the reference's int8 cast
// and nibble 0 (code -8) through its uint8 cast before packing (ops.py:122);
// both are reproduced here.
template <bool PACK>
__device__ inline int fq_code_from_quot(float t) {
  if (t != t) return PACK ? -8 : 0;
  const float c = fminf(fmaxf(t, -8.0f), 7.0f);
  return (int)__builtin_rintf(c);
}

// ---------------------------------------------------------------------------
// Generic kernel: one block of BT threads per token (grid-stride over tokens).
// LDS holds X (as D) and Z (as D); Y overwrites X. With LR_LDS, L and R are
// copied into LDS once per block as well (where they fit beside X and Z):
// the products then read every operand from LDS instead of a global load per
// k step; the arithmetic and its order are the same. Each thread accumulates
// TM x 4 output tiles (TM = 4 with 256 threads; TM = 2 with 512 threads, for
// fewer tokens than CUs: two waves per SIMD, half the products per wave).
// ---------------------------------------------------------------------------

// W consecutive D elements from LDS as float32 (W = 2 or 4; 4 W- or
// 2 W-byte aligned).
template <class DT, int W>
__device__ inline void ldsv(const typename DT::T* p, float (&out)[W]) {
  using T = typename DT::T;
  typedef T vt __attribute__((ext_vector_type(W)));
  const vt v = *reinterpret_cast<const vt*>(p);
#pragma unroll
  for (int i = 0; i < W; ++i) out[i] = DT::to_f(v[i]);
}

// n elements from global memory into LDS by BT threads, eight loads in flight
// per thread (a plain copy loop waits out each load's latency before the
// next).
template <int BT, class T>
__device__ inline void copy_to_lds(T* __restrict__ dst, const T* __restrict__ src, int n, int tid) {
  int f = tid;
  for (; f + 7 * BT < n; f += 8 * BT) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[f + BT * u];
#pragma unroll
    for (int u = 0; u < 8; ++u) dst[f + BT * u] = v[u];
  }
  for (; f < n; f += BT) dst[f] = src[f];
}

template <class DT, bool PACK, bool LR_LDS, int BT, int TM>
__global__ void __launch_bounds__(BT)
fq_generic_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
                  const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right,
                  int M, int N, float clip, void* __restrict__ out_codes,
                  float* __restrict__ out_scales) {
  static_assert(BT % 64 == 0 && (TM == 2 || TM == 4), "block and tile");
  using T = typename DT::T;
  constexpr int NWV = BT / 64;
  extern __shared__ __align__(16) unsigned char smem[];
  const int F = M * N;
  T* xs = reinterpret_cast<T*>(smem);
  T* zs = xs + F;
  T* const ls = zs + F;        // LR_LDS: L [M][M], then R [N][N]
  T* const rs = ls + M * M;
  __shared__ float red_hi[NWV], red_lo[NWV], s_scale;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if constexpr (LR_LDS) {      // ordered before their reads by the token loop's first barrier
    copy_to_lds<BT>(ls, left, M * M, tid);
    copy_to_lds<BT>(rs, right, N * N, tid);
  }
  auto r_at = [&](int i) { return DT::to_f(LR_LDS ? rs[i] : right[i]); };
  auto l_at = [&](int i) { return DT::to_f(LR_LDS ? ls[i] : left[i]); };

  for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
    copy_to_lds<BT>(xs, x + t * x_ld, F, tid);
    __syncthreads();
    // Both contractions in TM x 4 output tiles per thread (rows m0.., columns
    // n0..; consecutive threads take consecutive column groups, so the global
    // reads of R and L coalesce), accumulated in float32 over k in order.
    const int nb = (N + 3) >> 2, tiles = ((M + TM - 1) / TM) * nb;
    // With every operand in LDS and M, N multiples of 4, operands are read as
    // vectors (rows of X by 4 k, rows of R and Z by 4 columns, L by TM
    // columns): same order of float32 products per output.
    const bool vec = LR_LDS && M % 4 == 0 && N % 4 == 0;
    // Z = rnd_D(X R): Z[m][n] = sum_k X[m][k] R[k][n]
    for (int tl = tid; tl < tiles; tl += BT) {
      const int m0 = tl / nb * TM, n0 = (tl % nb) * 4;
      float acc[TM][4] = {};
      if (vec) {
        for (int k = 0; k < N; k += 4) {
          float xv[TM][4], rv[4][4];
#pragma unroll
          for (int i = 0; i < TM; ++i) ldsv<DT, 4>(xs + (m0 + i) * N + k, xv[i]);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) ldsv<DT, 4>(rs + (k + kk) * N + n0, rv[kk]);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i][kk], rv[kk][j], acc[i][j]);
        }
      } else {
#pragma unroll 4
        for (int k = 0; k < N; ++k) {
          float xv[TM], rv[4];
#pragma unroll
          for (int i = 0; i < TM; ++i) xv[i] = m0 + i < M ? DT::to_f(xs[(m0 + i) * N + k]) : 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) rv[j] = n0 + j < N ? r_at(k * N + n0 + j) : 0.f;
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], rv[j], acc[i][j]);
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (m0 + i < M && n0 + j < N) zs[(m0 + i) * N + n0 + j] = DT::from_f(acc[i][j]);
    }
    __syncthreads();
    // Y = rnd_D(L^T Z): Y[m][n] = sum_k L[k][m] Z[k][n]
    float hi = -INFINITY, lo = INFINITY;
    for (int tl = tid; tl < tiles; tl += BT) {
      const int m0 = tl / nb * TM, n0 = (tl % nb) * 4;
      float acc[TM][4] = {};
      if (vec) {
#pragma unroll 4
        for (int k = 0; k < M; ++k) {
          float lv[TM], zv[4];
          ldsv<DT, TM>(ls + k * M + m0, lv);
          ldsv<DT, 4>(zs + k * N + n0, zv);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(lv[i], zv[j], acc[i][j]);
        }
      } else {
#pragma unroll 4
        for (int k = 0; k < M; ++k) {
          float lv[TM], zv[4];
#pragma unroll
          for (int i = 0; i < TM; ++i) lv[i] = m0 + i < M ? l_at(k * M + m0 + i) : 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) zv[j] = n0 + j < N ? DT::to_f(zs[k * N + n0 + j]) : 0.f;
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(lv[i], zv[j], acc[i][j]);
        }
      }
      // Y goes into X's buffer: X was last read before the barrier above
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (m0 + i < M && n0 + j < N) {
            const T y = DT::from_f(acc[i][j]);
            xs[(m0 + i) * N + n0 + j] = y;
            hi = fmaxf(hi, DT::to_f(y));
            lo = fminf(lo, DT::to_f(y));
          }
    }
    hi = wave_max(hi);
    lo = wave_min(lo);
    if (lane == 0) { red_hi[wave] = hi; red_lo[wave] = lo; }
    __syncthreads();
    if (tid == 0) {
      float h = red_hi[0], l = red_lo[0];
      for (int w = 1; w < NWV; ++w) { h = fmaxf(h, red_hi[w]); l = fminf(l, red_lo[w]); }
      const float s = fq_scale<DT>(h, l, clip);
      s_scale = s;
      out_scales[t] = s;
    }
    __syncthreads();
    const float s = s_scale;
    if (PACK) {
      int32_t* o = reinterpret_cast<int32_t*>(out_codes) + t * (F / 8);
      for (int p = tid; p < F / 8; p += BT) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float q = DT::round(opaque(DT::to_f(xs[8 * p + i])) / s);
          word |= (uint32_t)(fq_code_from_quot<true>(q) + 8) << (4 * i);
        }
        o[p] = (int32_t)word;
      }
    } else {
      int8_t* o = reinterpret_cast<int8_t*>(out_codes) + t * F;
      for (int f = tid; f < F; f += BT) {
        const float q = DT::round(opaque(DT::to_f(xs[f])) / s);
        o[f] = (int8_t)fq_code_from_quot<false>(q);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Generic kernel for shapes whose X and Z do not fit in LDS together (fp32
// above 20480 features, fp16 / bf16 shapes outside the MFMA kernels above
// 40960): one 256-thread block per token (grid-stride over tokens). Y is
// computed in blocks of kBigCols columns: Z's block [M, kBigCols] in LDS, X,
// L and R read through the caches. It runs twice per token, once for the
// extremes (the scale) and once more, with the same arithmetic and so the
// same values, for the codes. Rounding points and the sequential float32 sums
// over k are those of fq_generic_kernel, so the results are identical.
// ---------------------------------------------------------------------------
constexpr int kBigCols = 16;

template <class DT, bool PACK>
__global__ void __launch_bounds__(256)
fq_generic_big_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
                      const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, int M,
                      int N, float clip, void* __restrict__ out_codes, float* __restrict__ out_scales) {
  extern __shared__ __align__(16) float zb[];   // [M][kBigCols], D values as float
  __shared__ float red_hi[4], red_lo[4], s_scale;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t F = (int64_t)M * N;
  for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
    const typename DT::T* xt = x + t * x_ld;
    float hi = -INFINITY, lo = INFINITY, s = 0.f;
    for (int pass = 0; pass < 2; ++pass) {
      if (pass == 1 && PACK) {
        // nibbles are ORed in below, a block of columns at a time
        int32_t* o = reinterpret_cast<int32_t*>(out_codes) + t * (F / 8);
        for (int64_t p = tid; p < F / 8; p += 256) o[p] = 0;
        __syncthreads();
      }
      for (int n0 = 0; n0 < N; n0 += kBigCols) {
        const int cb = min(kBigCols, N - n0);
        // Z[:, n0 .. n0 + cb) = rnd_D(X R[:, n0 .. n0 + cb))
        for (int o = tid; o < M * cb; o += 256) {
          const int m = o / cb, j = o % cb;
          float acc = 0.f;
          for (int k = 0; k < N; ++k) acc = fmaf(DT::to_f(xt[(int64_t)m * N + k]), DT::to_f(right[k * N + n0 + j]), acc);
          zb[m * kBigCols + j] = DT::round(acc);
        }
        __syncthreads();
        // Y[:, n0 .. n0 + cb) = rnd_D(L^T Z[:, n0 .. n0 + cb))
        for (int o = tid; o < M * cb; o += 256) {
          const int m = o / cb, j = o % cb;
          float acc = 0.f;
          for (int k = 0; k < M; ++k) acc = fmaf(DT::to_f(left[k * M + m]), zb[k * kBigCols + j], acc);
          const float y = DT::round(acc);
          if (pass == 0) {
            hi = fmaxf(hi, y);
            lo = fminf(lo, y);
          } else {
            const int64_t f = (int64_t)m * N + n0 + j;
            const float q = DT::round(opaque(y) / s);
            if (PACK) {
              const uint32_t nib = (uint32_t)(fq_code_from_quot<true>(q) + 8) << (4 * (f & 7));
              atomicOr(reinterpret_cast<uint32_t*>(out_codes) + t * (F / 8) + (f >> 3), nib);
            } else {
              reinterpret_cast<int8_t*>(out_codes)[t * F + f] = (int8_t)fq_code_from_quot<false>(q);
            }
          }
        }
        __syncthreads();
      }
      if (pass == 0) {
        hi = wave_max(hi);
        lo = wave_min(lo);
        if (lane == 0) { red_hi[wave] = hi; red_lo[wave] = lo; }
        __syncthreads();
        if (tid == 0) {
          float h = red_hi[0], l = red_lo[0];
          for (int w = 1; w < 4; ++w) { h = fmaxf(h, red_hi[w]); l = fminf(l, red_lo[w]); }
          const float sc = fq_scale<DT>(h, l, clip);
          s_scale = sc;
          out_scales[t] = sc;
        }
        __syncthreads();
        s = s_scale;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel.
//
// Shapes: M = 16*MB, N = 32*NP. A "pair" q is the 32 columns n in [32q, 32q+32),
// i.e. output words 4q..4q+3 of each row m. Each wave owns one (token, pair);
// NP waves share a token, TPB = WAVES/NP tokens are in flight per block.
//
// Column permutation: inside pair q, MFMA block h (0/1) lane-column i (0..15)
// is physical column n = 32q + 8*(i/4) + 4h + (i%4). With that choice the
// second product, computed transposed (Y^T = Z^T L with Z's accumulator
// fragment reused as the A operand), leaves lane (g = lane/16) holding
// Y[m][32q + 8g + 0..7] — the eight features of one packed word — so packing
// needs no cross-lane traffic.
//
// MFMA 16x16x32 operand convention used throughout: lane l supplies row/column
// l%16 and the eight k values 8*(l/16) + 0..7 of the current 32-deep slab; the
// accumulator holds rows 4*(l/16) + r, r = 0..3, of column l%16. The k order
// only has to agree between the A and B operands.
// ---------------------------------------------------------------------------

template <class DT>
struct MfmaOps;

// V: 8-element operands of the 16x16x32 MFMA. An odd trailing 16-deep slab of
// the second product (M / 16 odd) is a zero-padded 32-deep slab: elements 0..3
// of lane group g hold k = 4g .. 4g+3 (the rows of Z's accumulator), elements
// 4..7 of both operands are zero, which leaves the MFMA's sum unchanged. (The
// 16x16x16 MFMA gave wrong results in that role on gfx950.)
template <>
struct MfmaOps<F16T> {
  using V = v8h;
  __device__ static inline v4f mfma(V a, V b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct MfmaOps<BF16T> {
  using V = v8bf;
  __device__ static inline v4f mfma(V a, V b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Epilogue on packed pairs. A lane's Y values come in pairs (MFMA block h = 0
// and 1 at the same accumulator row r) that belong in nibbles r and r + 4 of
// one output word, so each pair is kept as two 16-bit D values in one VGPR
// (rounding point 2 for both with one v_cvt_pk). Quantizing a pair:
//   a = clamp(y * rcp, -8, 7) in float32   (clamp commutes with the roundings
//                                           below because -8 and 7 are D values)
//   t = rnd_D(a)                           (one v_cvt_pk for the pair)
//   t + magic                              (round half to even to an integer)
// The magic constant leaves q + 8 in the low bits of each result; shifting the
// pair's bits by 4r and adding puts both codes in place, and the constant bits
// the magic leaves above the codes add up to kJunk, removed once per word.
// y * rcp stands in for the fallback's y / s (IEEE): the two differ only when
// the quotient lies within a few float32 ulps of a rounding boundary of D.
template <class DT>
struct FqEpi;

template <>
struct FqEpi<F16T> {
  __device__ static inline uint32_t pack(float a, float b) {
    const v2h h = {(_Float16)opaque(a), (_Float16)opaque(b)};
    return __builtin_bit_cast(uint32_t, h);
  }
  // The same rounding of two MFMA accumulator values. An MFMA result has no
  // product for the compiler to fuse into the conversion, so no opaque() is
  // needed (which would copy accumulators that are read again for the absmax).
  __device__ static inline uint32_t pack_acc(float a, float b) {
    const v2h h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline float lo(uint32_t p) { return (float)__builtin_bit_cast(v2h, p)[0]; }
  __device__ static inline float hi(uint32_t p) { return (float)__builtin_bit_cast(v2h, p)[1]; }
  // fp16: 1544 = 1536 + 8 has a unit ulp, so t + 1544 is the integer 1536 + q + 8,
  // bits 0x6600 + (q + 8); both halves are handled by one v_pk_add_f16.
  __device__ static inline void accumulate(uint32_t& word, uint32_t p, float rcp, int r) {
    const float a0 = __builtin_amdgcn_fmed3f(mul_f16lo(p, rcp), -8.0f, 7.0f);
    const float a1 = __builtin_amdgcn_fmed3f(mul_f16hi(p, rcp), -8.0f, 7.0f);
    v2h t = __builtin_bit_cast(v2h, pack(a0, a1));
    const v2h magic = {(_Float16)1544.0f, (_Float16)1544.0f};
    t = t + magic;
    word += __builtin_bit_cast(uint32_t, t) << (4 * r);
  }
  static constexpr uint32_t kJunk =
      0x66006600u + (0x66006600u << 4) + (0x66006600u << 8) + (0x66006600u << 12);

  // Packed word of four pairs (nibbles r and r + 4 from pair r), clamping the
  // rounded pair instead of the float32 quotients: rounding is monotonic and
  // -8, 7 are fp16 values, so clamp(rnd(a)) = rnd(clamp(a)). One packed min per
  // pair, plus one packed max when a quotient can round below -8.5 (LOW).
  template <bool LOW>
  __device__ static inline uint32_t word4(const uint32_t (&p)[4], float rcp) {
    const v2h seven = {(_Float16)7.0f, (_Float16)7.0f};
    const v2h minus8 = {(_Float16)-8.0f, (_Float16)-8.0f};
    const v2h magic = {(_Float16)1544.0f, (_Float16)1544.0f};
    uint32_t word = 0u - kJunk;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v2h t = __builtin_bit_cast(v2h, pack(mul_f16lo(p[r], rcp), mul_f16hi(p[r], rcp)));
      t = __builtin_elementwise_min(t, seven);
      if (LOW) t = __builtin_elementwise_max(t, minus8);
      t = t + magic;
      word += __builtin_bit_cast(uint32_t, t) << (4 * r);
    }
    return word;
  }

  // Running extremes of rounded Y pairs, two pairs per step (v_pk_maximum3 /
  // v_pk_minimum3), and max |y| from them as a 16-bit pattern.
  struct Amax {
    v2h hi = {(_Float16)-INFINITY, (_Float16)-INFINITY};
    v2h lo = {(_Float16)INFINITY, (_Float16)INFINITY};
  };
  __device__ static inline void track2(Amax& a, uint32_t p0, uint32_t p1) {
    const v2h y0 = __builtin_bit_cast(v2h, p0), y1 = __builtin_bit_cast(v2h, p1);
    a.hi = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a.hi, y0), y1);
    a.lo = __builtin_elementwise_minimum(__builtin_elementwise_minimum(a.lo, y0), y1);
  }
  __device__ static inline uint32_t amax_bits(const Amax& a) {
    const uint32_t m = pk_absmax16(pk_absmax16(0u, __builtin_bit_cast(uint32_t, a.hi)),
                                   __builtin_bit_cast(uint32_t, a.lo));
    return max(m & 0xFFFFu, m >> 16);
  }
};

template <>
struct FqEpi<BF16T> {
  __device__ static inline uint32_t pack(float a, float b) {
    const v2bf h = {(__bf16)opaque(a), (__bf16)opaque(b)};
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline uint32_t pack_acc(float a, float b) {
    const v2bf h = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline float lo(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
  __device__ static inline float hi(uint32_t p) { return __builtin_bit_cast(float, p & 0xFFFF0000u); }
  // bf16: rounded pair back to float32, then + 12582920 = 1.5 * 2^23 + 8 leaves
  // bits 0x4B400000 + (q + 8). The high element is shifted by 16 + 4r, which
  // drops all of 0x4B400000; the low element's constant part sums to kJunk.
  __device__ static inline void accumulate(uint32_t& word, uint32_t p, float rcp, int r) {
    const float a0 = __builtin_amdgcn_fmed3f(lo(p) * rcp, -8.0f, 7.0f);
    const float a1 = __builtin_amdgcn_fmed3f(hi(p) * rcp, -8.0f, 7.0f);
    const uint32_t t = pack(a0, a1);
    const float f0 = lo(t) + 12582920.0f;
    const float f1 = hi(t) + 12582920.0f;
    word += __builtin_bit_cast(uint32_t, f0) << (4 * r);
    word += __builtin_bit_cast(uint32_t, f1) << (16 + 4 * r);
  }
  static constexpr uint32_t kJunk =
      0x4B400000u + (0x4B400000u << 4) + (0x4B400000u << 8) + (0x4B400000u << 12);

  // Packed word of four pairs (the float32 clamp covers both bounds).
  template <bool LOW>
  __device__ static inline uint32_t word4(const uint32_t (&p)[4], float rcp) {
    uint32_t word = 0u - kJunk;
#pragma unroll
    for (int r = 0; r < 4; ++r) accumulate(word, p[r], rcp, r);
    return word;
  }

  // Code byte B of d from a rounded quotient t (a bf16 value in a float32
  // register, -8.5 <= t < 7.5): one SDWA add of 12582920 = 1.5 * 2^23 + 8,
  // whose float32 sum has a unit ulp, so it rounds t + 8 half to even, which
  // is rint(t) + 8 (8 is even), and leaves that integer (0 .. 15) in the
  // low byte of its bits; dst_sel writes that byte into byte B of d, the
  // other bytes kept (FIRST: cleared). A NaN t (its float32 low half zero)
  // gives byte 0, as v_cvt_pk_u8_f32 of t + 8 does.
  template <int B, bool FIRST>
  __device__ static inline void code_byte(uint32_t& d, float t, float magic) {
    static_assert(!FIRST || B == 0, "the first byte of a word clears the rest");
#define QO_CODE_BYTE(SEL, UNUSED, C)                                                                         \
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:" SEL " dst_unused:" UNUSED " src0_sel:DWORD src1_sel:DWORD"     \
      : C(d)                                                                                                \
      : "v"(t), "v"(magic))
    if constexpr (FIRST) QO_CODE_BYTE("BYTE_0", "UNUSED_PAD", "=v");
    else if constexpr (B == 1) QO_CODE_BYTE("BYTE_1", "UNUSED_PRESERVE", "+v");
    else if constexpr (B == 2) QO_CODE_BYTE("BYTE_2", "UNUSED_PRESERVE", "+v");
    else QO_CODE_BYTE("BYTE_3", "UNUSED_PRESERVE", "+v");
#undef QO_CODE_BYTE
  }

  // The packed word of four pairs from rounded quotients t[i] (code i):
  // even codes in the bytes of ev, odd codes in the bytes of od, and
  // ev | od << 4 puts code i in nibble i.
  __device__ static inline uint32_t word_from_quotients(const float (&t)[8]) {
    const float magic = 12582920.0f;
    uint32_t ev, od;
    code_byte<0, true>(ev, t[0], magic);
    code_byte<0, true>(od, t[1], magic);
    code_byte<1, false>(ev, t[2], magic);
    code_byte<1, false>(od, t[3], magic);
    code_byte<2, false>(ev, t[4], magic);
    code_byte<2, false>(od, t[5], magic);
    code_byte<3, false>(ev, t[6], magic);
    code_byte<3, false>(od, t[7], magic);
    return ev | (od << 4);
  }

  // The same word as word4 through code bytes: per code the quotient
  // y * rcp clamped to [-8, 7] (v_med3; the clamp commutes with the rounding
  // since -8 and 7 are bf16 values), rounded to bf16 straight into a float32
  // register by one v_cvt_pk_bf16_f32 whose low half is the conversion of 0.0
  // (the bf16 value's float32 bits, low half zero), then code_byte: 10 VALU
  // per pair of codes (the two elements unpacked, two products, two clamps,
  // two conversions, two code bytes).
  __device__ static inline uint32_t word_u8(const uint32_t (&p)[4], float rcp) {
    float t[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // operands are VALU results, never MFMA results
      asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(t[r]) : "v"(__builtin_amdgcn_fmed3f(lo(p[r]) * rcp, -8.0f, 7.0f)));
      asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(t[r + 4]) : "v"(__builtin_amdgcn_fmed3f(hi(p[r]) * rcp, -8.0f, 7.0f)));
    }
    return word_from_quotients(t);
  }

  // word_u8 for a token whose largest quotient rounds below 7.5 and whose
  // smallest rounds to -8.5 or above (every code then lies in -8 .. 7 with
  // no clamp; the host picks this form from the clip ratio, kNoClampClip):
  // 8 VALU per pair of codes.
  __device__ static inline uint32_t word_u8_noclamp(const uint32_t (&p)[4], float rcp) {
    float t[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // operands are VALU products, never MFMA results
      asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(t[r]) : "v"(lo(p[r]) * rcp));
      asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(t[r + 4]) : "v"(hi(p[r]) * rcp));
    }
    return word_from_quotients(t);
  }

  // max |y| of rounded Y pairs as a 16-bit pattern (sign-cleared bf16 bits
  // order like the values).
  struct Amax {
    uint32_t m = 0u;
  };
  __device__ static inline void track2(Amax& a, uint32_t p0, uint32_t p1) {
    a.m = pk_absmax16(pk_absmax16(a.m, p0), p1);
  }
  __device__ static inline uint32_t amax_bits(const Amax& a) { return max(a.m & 0xFFFFu, a.m >> 16); }
};

// LDS transpose read of 16-bit elements (gfx950 ds_read_b64_tr_b16): within
// each 16-lane group, lane l supplies the address of 4 consecutive elements
// (8-byte aligned), forming row l of a 16 x 4 matrix A; lane i receives
// A[i/4][i%4], A[4 + i/4][i%4], A[8 + i/4][i%4], A[12 + i/4][i%4] — that is,
// A[4e + i/4][i%4] for e = 0..3 (checked on the device).
typedef short v4s16 __attribute__((ext_vector_type(4)));
__device__ inline v4s16 lds_tr16(const void* p) {
  typedef __attribute__((address_space(3))) v4s16* lds_v4s16;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s16)(__attribute__((address_space(3))) const void*)p);
}
// Two 4-element reads as one 8-element MFMA operand (elements 0..3, 4..7).
template <class V>
__device__ inline V join_tr16(v4s16 lo, v4s16 hi) {
  typedef short v8s16 __attribute__((ext_vector_type(8)));
  const v8s16 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(V, w);
}

// NV, MV: the token's width and height in memory; N = 32 NP and M = 16 MB are
// computed, the rest is zero padding (X's padded columns and rows zeroed in
// registers, R's and L's padded rows and columns zero, padded codes not
// stored; the padded Y values are 0, which leaves max |Y| unchanged).
// NV % 8 != 0 (SPLIT; NV even): rows start off 16-byte boundaries, so X is
// copied in 4-byte pieces, the row's last 8-column chunk is partly padding,
// and codes are stored in pieces as aligned as the row offset allows: 16-bit
// (packed) or 4-byte (int8) for NV % 4 == 0, bytes or 16-bit otherwise.
template <int MB, int NP, int NV = 32 * NP, int MV = 16 * MB>
struct FqShape {
  static constexpr int M = 16 * MB;
  static constexpr int N = 32 * NP;
  static constexpr int F = MV * NV;
  static_assert(NV % 2 == 0 && NV > 32 * (NP - 1) && NV <= N, "valid width");
  static constexpr bool SPLIT = NV % 8 != 0;
  static_assert(MV > 16 * (MB - 1) && MV <= M, "valid height");
  // L's fragments (MB (KS2 + 1) of them, 4 VGPRs each) stay in LDS instead of
  // VGPRs where they would not fit beside R's (2 KS1) and the accumulators.
  static constexpr bool LF_LDS = MB * (MB / 2 + 1) + 2 * NP > 32 || MV != M;
  static constexpr int KS1 = NP;             // 32-deep slabs of the first product (k = n')
  static constexpr int KS2 = MB / 2;         // full 32-deep slabs of the second product (k = m')
  static constexpr bool TAIL = (MB & 1) != 0; // plus one 16-deep slab when M is an odd multiple of 16
  static constexpr int KSL = KS2 + (TAIL ? 1 : 0);   // slabs read, incl. the zero-padded tail
  // L's fragments in LDS at stride KS2 + 1 per row block; for even MB the
  // last one (a zero slab never read) is left out of the allocation
  static constexpr int LF_FRAGS = MB * (KS2 + 1) - (TAIL ? 0 : 1);
  static constexpr int XFRAGS = MB * KS1;    // 1 KiB A fragments per token
  // Four waves per workgroup: one token per group at N = 128, two at N = 64,
  // four at N = 32. Small workgroups (X double buffer only, L in VGPRs) let
  // several run per CU, so one group's MFMA phase overlaps another's epilogue.
  static constexpr int TPB = NP >= 4 ? 1 : 4 / NP;   // tokens per group
  static constexpr int WAVES = NP * TPB;
  static constexpr int STAGE_FRAGS = TPB * XFRAGS;
  static constexpr int FRAGS_PER_WAVE = STAGE_FRAGS / WAVES;   // == MB
  static constexpr int DMA_PER_WAVE = (SPLIT ? 4 : 1) * FRAGS_PER_WAVE;
  static constexpr int STAGE_ELEMS = STAGE_FRAGS * 512;
  // One X stage instead of two where two would not fit in LDS beside L's
  // fragments: the next group's copy is then issued once every wave's first
  // product has read the stage (it still overlaps the second product and the
  // epilogue).
  static constexpr int LF_BYTES = LF_LDS ? LF_FRAGS * 1024 : 16;
  static constexpr bool ONE_STAGE = 2 * STAGE_ELEMS * 2 + LF_BYTES + 8 * TPB * NP > 160 * 1024;
  static_assert(STAGE_FRAGS % WAVES == 0, "X fragments must split evenly over waves");
  static_assert(M * M <= STAGE_ELEMS, "L must fit in one X stage while it is staged");
  static_assert(DMA_PER_WAVE < 64, "vmcnt range");
};

// Wait until at most N vector-memory operations of this wave are outstanding.
// vmcnt is 6 bits on gfx9 (0..63); the encoding keeps lgkmcnt / expcnt at max.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Codes of one lane's 8 columns (rem of them inside the row, rem > 0) where
// the row offset in a SPLIT shape allows only partial alignment. Packed: 8
// nibbles in `word`, at a byte address that is 2-byte aligned when
// NV % 4 == 0. int8: 8 bytes in lo4 / hi4, at an address 4-byte aligned when
// NV % 4 == 0, 2-byte aligned otherwise.
template <int NV>
__device__ inline void fq_store_packed_split(uint8_t* o, uint32_t word, int rem) {
  if constexpr (NV % 4 == 0) {
    reinterpret_cast<uint16_t*>(o)[0] = (uint16_t)word;
    if (rem >= 8) reinterpret_cast<uint16_t*>(o)[1] = (uint16_t)(word >> 16);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (2 * k + 2 <= rem) o[k] = (uint8_t)(word >> (8 * k));
  }
}

template <int NV>
__device__ inline void fq_store_int8_split(int8_t* o, uint32_t lo4, uint32_t hi4, int rem) {
  if constexpr (NV % 4 == 0) {
    *reinterpret_cast<int32_t*>(o) = (int32_t)lo4;
    if (rem >= 8) *reinterpret_cast<int32_t*>(o + 4) = (int32_t)hi4;
  } else {
    const uint32_t h[4] = {lo4 & 0xFFFFu, lo4 >> 16, hi4 & 0xFFFFu, hi4 >> 16};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (2 * k + 2 <= rem) reinterpret_cast<uint16_t*>(o)[k] = (uint16_t)h[k];
  }
}

// One token group (this wave's token slot and pair) from an X stage in LDS:
// both products, the per-token scale and the codes.
// after_x() runs once the first product has read the X stage.
template <class DT, int MB, int NP, bool PACK, int NV, int MV, bool LF_IN_LDS = FqShape<MB, NP, NV, MV>::LF_LDS,
          class AfterX>
__device__ __attribute__((always_inline)) inline void fq_mfma_group(
    const typename DT::T* __restrict__ xs, const typename MfmaOps<DT>::V (&lf)[MB][FqShape<MB, NP>::KS2 + 1],
    const unsigned char* lf_lds,
    const typename MfmaOps<DT>::V (&rf)[2][FqShape<MB, NP>::KS1], float (*red)[NP][2], int64_t t,
    int64_t tokens, float clip, void* __restrict__ out_codes, float* __restrict__ out_scales, int lane,
    int tau, int q, AfterX&& after_x) {
  using S = FqShape<MB, NP, NV, MV>;
  using T = typename DT::T;
  using Ops = MfmaOps<DT>;
  using V = typename Ops::V;
  constexpr int F = S::F, KS1 = S::KS1, KS2 = S::KS2;
  const int li = lane & 15, lg = lane >> 4;
  // this lane's 8 columns of its pair: stored only inside the valid width
  // (with SPLIT the last chunk's first rem columns only)
  const int rem = NV - (32 * q + 8 * lg);
  const bool col_ok = rem > 0;

  // First product, one 16-row block of Z at a time: Z[rb] = X[rb] R[:, pair].
  constexpr int KSL = S::KSL;
  V zp[2][KS2 + 1];   // 32-deep slabs of Z^T
#pragma unroll
  for (int rb = 0; rb < MB; ++rb) {
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) {
      V a = *reinterpret_cast<const V*>(xs + ((rb * KS1 + ks) * 64 + lane) * 8);
      if (NV < S::N && ks == KS1 - 1 && 32 * ks + 8 * lg >= NV) a = V{};   // padded k
      if (S::SPLIT && ks == KS1 - 1) {                                        // partly padded chunk
        const int kv = NV - (32 * ks + 8 * lg);
        if (kv > 0 && kv < 8) {
#pragma unroll
          for (int j = 2; j < 8; ++j)
            if (j >= kv) a[j] = DT::from_f(0.0f);
        }
      }
      if (MV < S::M && rb == MB - 1 && 16 * rb + li >= MV) a = V{};        // padded row
      acc0 = Ops::mfma(a, rf[0][ks], acc0);
      acc1 = Ops::mfma(a, rf[1][ks], acc1);
    }
    // Rounding point 1, and the accumulator -> A-operand hand-off.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      zp[0][rb >> 1][(rb & 1) * 4 + r] = DT::from_f(acc0[r]);
      zp[1][rb >> 1][(rb & 1) * 4 + r] = DT::from_f(acc1[r]);
      if (S::TAIL && rb == MB - 1) {
        zp[0][rb >> 1][4 + r] = DT::from_f(0.0f);
        zp[1][rb >> 1][4 + r] = DT::from_f(0.0f);
      }
    }
    // keep the scheduler from hoisting every row block's fragment loads at once
    // (their VGPRs would not fit next to L's and R's fragments)
    __builtin_amdgcn_sched_barrier(0);
  }
  after_x();

  // Second product, transposed: Y^T[n][m] = sum_m' Z[m'][n] L[m'][m].
  using Epi = FqEpi<DT>;
  uint32_t yp[MB][4];
  float hi = -INFINITY, lo = INFINITY;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      V lfv;
      if constexpr (LF_IN_LDS) lfv = *reinterpret_cast<const V*>(lf_lds + (mb * (KS2 + 1) + s) * 1024 + 16 * lane);
      else lfv = lf[mb][s];
      acc0 = Ops::mfma(zp[0][s], lfv, acc0);
      acc1 = Ops::mfma(zp[1][s], lfv, acc1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // extremes of the raw accumulators: rounding is monotonic, so the D
      // rounding of these equals amax/amin of the rounded Y
      hi = fmaxf(hi, fmaxf(acc0[r], acc1[r]));
      lo = fminf(lo, fminf(acc0[r], acc1[r]));
      yp[mb][r] = Epi::pack(acc0[r], acc1[r]);  // rounding point 2
    }
  }

  hi = wave_max(hi);
  lo = wave_min(lo);
  if (lane == 0) {
    red[tau][q][0] = hi;
    red[tau][q][1] = lo;
  }
  lds_barrier();
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    hi = fmaxf(hi, red[tau][p][0]);
    lo = fminf(lo, red[tau][p][1]);
  }
  const float s = fq_scale<DT>(hi, lo, clip);
  if (t >= tokens) return;
  if (q == 0 && lane == 0) out_scales[t] = s;
  if (PACK && s > 0.f) {
    const float rcp = 1.0f / s;
    int32_t* orow = reinterpret_cast<int32_t*>(out_codes) + t * (F / 8) + 4 * q + lg;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      uint32_t word = 0u - Epi::kJunk;
#pragma unroll
      for (int r = 0; r < 4; ++r) Epi::accumulate(word, yp[mb][r], rcp, r);
      if constexpr (S::SPLIT) {
        // nibble offset t F + m NV + 8 (4q + lg) is even: a byte offset; 16
        // rows further on is 8 NV bytes further on
        uint8_t* ob = reinterpret_cast<uint8_t*>(out_codes) + t * (F / 2) + (li * NV + 32 * q + 8 * lg) / 2 +
                      mb * (8 * NV);
        if (col_ok && 16 * mb + li < MV) fq_store_packed_split<NV>(ob, word, rem);
      } else {
        if (col_ok && 16 * mb + li < MV) orow[(16 * mb + li) * (NV / 8)] = (int32_t)word;
      }
    }
    return;
  }
  // int8 codes, and tokens whose scale rounded to 0 (the fallback's 0/0 codes)
  const float rcp = 1.0f / s;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + li;
    if (m >= MV) continue;
    int code[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float y0 = Epi::lo(yp[mb][r]), y1 = Epi::hi(yp[mb][r]);
      if (s > 0.f) {
        code[r] = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y0 * rcp, -8.0f, 7.0f)));
        code[4 + r] = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y1 * rcp, -8.0f, 7.0f)));
      } else {
        code[r] = fq_code_from_quot<PACK>(DT::round(opaque(y0) / s));
        code[4 + r] = fq_code_from_quot<PACK>(DT::round(opaque(y1) / s));
      }
    }
    if (PACK) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) word |= (uint32_t)(code[j] + 8) << (4 * j);
      if constexpr (S::SPLIT) {
        uint8_t* ob = reinterpret_cast<uint8_t*>(out_codes) + t * (F / 2) + (m * NV + 32 * q + 8 * lg) / 2;
        if (col_ok) fq_store_packed_split<NV>(ob, word, rem);
      } else {
        if (col_ok) reinterpret_cast<int32_t*>(out_codes)[t * (F / 8) + m * (NV / 8) + 4 * q + lg] = (int32_t)word;
      }
    } else {
      uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo4 |= (uint32_t)(code[j] & 0xFF) << (8 * j);
        hi4 |= (uint32_t)(code[4 + j] & 0xFF) << (8 * j);
      }
      int8_t* ob = reinterpret_cast<int8_t*>(out_codes) + t * F + m * NV + 32 * q + 8 * lg;
      if constexpr (S::SPLIT) {
        if (col_ok) fq_store_int8_split<NV>(ob, lo4, hi4, rem);
      } else {
        v2i pair = {(int)lo4, (int)hi4};
        if (col_ok) *reinterpret_cast<v2i*>(ob) = pair;
      }
    }
  }
}

template <class DT, int MB, int NP, bool PACK, int NV, int MV>
__global__ void __launch_bounds__((FqShape<MB, NP, NV, MV>::WAVES * 64)) __attribute__((amdgpu_waves_per_eu(2)))
fq_mfma_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
               const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right,
               float clip, void* __restrict__ out_codes, float* __restrict__ out_scales) {
  using S = FqShape<MB, NP, NV, MV>;
  using T = typename DT::T;
  using V = typename MfmaOps<DT>::V;
  constexpr int KS1 = S::KS1, KS2 = S::KS2;
  constexpr int NT = S::WAVES * 64;

  // Two X stages as distinct objects: the compiler then knows that reading one
  // stage does not depend on the LDS-DMA still writing the other. L is staged
  // through the stage that is free at set-up.
  __shared__ __align__(16) T xbuf0[S::STAGE_ELEMS];
  __shared__ __align__(16) T xbuf1[S::ONE_STAGE ? 8 : S::STAGE_ELEMS];
  T* const lstage = S::ONE_STAGE ? xbuf0 : xbuf1;
  __shared__ __align__(16) unsigned char lf_lds[S::LF_LDS ? S::LF_FRAGS * 1024 : 16];
  __shared__ float red[S::TPB][NP][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform, so in SGPRs: the LDS-DMA destinations (M0 values) derived
  // from it then need no VGPRs across the token loop
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tau = wave / NP;   // token slot of this wave
  const int q = wave % NP;     // column pair of this wave
  const int li = lane & 15;    // lane row / column inside a 16x16 block
  const int lg = lane >> 4;    // lane group: k values 8*lg .. 8*lg+7

  // LDS-DMA of one token group into a stage. Fragment c of the stage is token
  // slot c / XFRAGS, block (rb, ks); lane l fetches X[16rb + l%16][32ks + 8(l/16) .. +7]
  // (16 bytes), which the hardware writes to fragment base + 16*l. With SPLIT
  // each fragment takes four 4-byte copies: copy h, lane l fetches dword l%4 of
  // fragment lane 16h + l/4, i.e. X[16rb + l/4][32ks + 8h + 2(l%4) .. +1], which
  // lands at fragment base + 256h + 4l = base + 16(16h + l/4) + 4(l%4).
  const int64_t ngroups = (tokens + S::TPB - 1) / S::TPB;
  auto issue = [&](int64_t g, T* stage) {
#pragma unroll
    for (int i = 0; i < S::FRAGS_PER_WAVE; ++i) {
      const int c = wave + i * S::WAVES;
      const int ts = c / S::XFRAGS, fr = c % S::XFRAGS;
      const int rb = fr / KS1, ks = fr % KS1;
      int64_t t = g * S::TPB + ts;
      t = t < tokens ? t : tokens - 1;  // tail slots re-read a valid row; never stored
      // padded chunks (columns >= NV) re-read the row's last chunk (last dword
      // with SPLIT); zeroed before use
      // padded rows (>= MV) re-read the last row; zeroed before use
      if constexpr (S::SPLIT) {
        // offsets recomputed at every issue from an opaque lane copy: 4 MB
        // addresses held across the token loop would not fit in VGPRs
        int l = lane;
        asm volatile("" : "+v"(l));
        const int off = min(16 * rb + (l >> 2), MV - 1) * NV + 2 * (l & 3);
        const T* xt = x + t * x_ld;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const T* src = xt + min(off + 32 * ks + 8 * h, min(16 * rb + (l >> 2), MV - 1) * NV + NV - 2);
          __builtin_amdgcn_global_load_lds((const void*)src,
                                           (__attribute__((address_space(3))) void*)(stage + c * 512 + h * 128), 4,
                                           0, 0);
        }
      } else {
        const T* src = x + t * x_ld + min(16 * rb + li, MV - 1) * NV + min(32 * ks + 8 * lg, NV - 8);
        __builtin_amdgcn_global_load_lds((const void*)src,
                                         (__attribute__((address_space(3))) void*)(stage + c * 512), 16, 0, 0);
      }
    }
  };
  // Before reading a stage: issue the next group into the other stage (past
  // the last group the DMA re-reads the last token, so every iteration issues
  // the same number of loads), wait for this wave's DMA of the current group
  // (loads complete in order, so at most DMA_PER_WAVE outstanding means the
  // older group has landed), then a barrier so every wave's part is visible.
  auto prefetch_and_wait = [&](int64_t gn, T* other) {
    issue(gn < ngroups ? gn : ngroups - 1, other);
    wait_vmcnt<S::DMA_PER_WAVE>();
    raw_barrier();
  };

  int64_t g = blockIdx.x;
  // first X group in flight while L and R are set up (grid <= ngroups); with
  // one stage, once L has been staged through it
  if constexpr (!S::ONE_STAGE) issue(g, xbuf0);

  // R as B-operand fragments of the first product for this wave's pair:
  // rf[h][ks][j] = R[32ks + 8lg + j][n], n = 32q + 8(li/4) + 4h + li%4.
  // Gathered straight from global memory; all loads issue before any use.
  V rf[2][KS1];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int n = 32 * q + 8 * (li >> 2) + 4 * h + (li & 3);
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = 32 * ks + 8 * lg + j;
        rf[h][ks][j] = (k < NV && n < NV) ? right[k * NV + n] : DT::from_f(0.0f);
      }
  }

  // L, staged row-major through the free X stage with coalesced 16-byte
  // copies, then gathered into B-operand fragments of the second product held
  // in VGPRs: lf[mb][s][j] = L[m'][m], m = 16mb + li,
  // m' = 32s + 16(j/4) + 4lg + j%4 — the row order of Z's accumulator pairs —
  // and, for odd M/16, the zero-padded slab lf[mb][KS2][j] = L[16(MB-1) + 4lg + j][m]
  // for j < 4.
  {
    constexpr int CHUNKS = MV * MV / 8;   // whole 16-byte chunks of L (MV x MV), then the tail elements
    constexpr int TAILE = MV * MV - 8 * CHUNKS;
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    v4i_t tmp[(CHUNKS + NT - 1) / NT];
#pragma unroll
    for (int i = 0; i < (CHUNKS + NT - 1) / NT; ++i) {
      const int c = tid + i * NT;
      tmp[i] = reinterpret_cast<const v4i_t*>(left)[c < CHUNKS ? c : 0];
    }
#pragma unroll
    for (int i = 0; i < (CHUNKS + NT - 1) / NT; ++i) {
      const int c = tid + i * NT;
      if (c < CHUNKS) reinterpret_cast<v4i_t*>(lstage)[c] = tmp[i];
    }
    if (TAILE > 0 && tid < TAILE) lstage[8 * CHUNKS + tid] = left[8 * CHUNKS + tid];
  }
  lds_barrier();
  // L[m'][m] of the staged MV x MV rows, 0 in the padding
  auto lval = [&](int mp, int m) { return (mp < MV && m < MV) ? lstage[mp * MV + m] : DT::from_f(0.0f); };
  V lf[MB][KS2 + 1];
  auto lfrag = [&](int mb, int s) {   // fragment (mb, s); s = KS2 is the zero-padded trailing slab
    if constexpr (MV == S::M && !S::LF_LDS) {
      // unpadded L held in VGPRs: two LDS transpose reads (lds_tr16) of 4 consecutive rows of
      // column 16mb + li, rows 32s + 4lg .. +3 (elements 0..3) and 16 rows on (4..7);
      // lane li supplies the address of row 32s + 4lg + li/4, columns 16mb + 4(li%4) .. +3
      const T* at = lstage + (32 * s + 4 * lg + (li >> 2)) * MV + 16 * mb + 4 * (li & 3);
      if (s < KS2) return join_tr16<V>(lds_tr16(at), lds_tr16(at + 16 * MV));
      if (S::TAIL) return join_tr16<V>(lds_tr16(at), v4s16{0, 0, 0, 0});
      return V{};
    } else {
      V v;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = s < KS2 ? lval(32 * s + 16 * (j >> 2) + 4 * lg + (j & 3), 16 * mb + li)
                       : (S::TAIL && j < 4) ? lval(16 * (MB - 1) + 4 * lg + j, 16 * mb + li) : DT::from_f(0.0f);
      return v;
    }
  };
  if constexpr (S::LF_LDS) {
    // the waves split the fragments; the barrier below makes them visible
#pragma unroll 1
    for (int fr = wave; fr < S::LF_FRAGS; fr += S::WAVES)
      *reinterpret_cast<V*>(lf_lds + fr * 1024 + 16 * lane) = lfrag(fr / (KS2 + 1), fr % (KS2 + 1));
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s <= KS2; ++s) lf[mb][s] = lfrag(mb, s);
  }
  lds_barrier();   // the staging stage is free again for the first prefetch

  if constexpr (S::ONE_STAGE) {
    issue(g, xbuf0);
    while (g < ngroups) {
      const int64_t gn = g + gridDim.x;
      wait_vmcnt<0>();
      raw_barrier();
      fq_mfma_group<DT, MB, NP, PACK, NV, MV>(xbuf0 + tau * S::XFRAGS * 512, lf, lf_lds, rf, red, g * S::TPB + tau,
                                              tokens, clip, out_codes, out_scales, lane, tau, q, [&] {
                                                lds_barrier();   // every wave's first product has read the stage
                                                if (gn < ngroups) issue(gn, xbuf0);
                                              });
      g = gn;
    }
  } else {
    while (g < ngroups) {
      int64_t gn = g + gridDim.x;
      prefetch_and_wait(gn, xbuf1);
      fq_mfma_group<DT, MB, NP, PACK, NV, MV>(xbuf0 + tau * S::XFRAGS * 512, lf, lf_lds, rf, red, g * S::TPB + tau,
                                              tokens, clip, out_codes, out_scales, lane, tau, q, [] {});
      g = gn;
      if (g >= ngroups) break;
      gn = g + gridDim.x;
      prefetch_and_wait(gn, xbuf0);
      fq_mfma_group<DT, MB, NP, PACK, NV, MV>(xbuf1 + tau * S::XFRAGS * 512, lf, lf_lds, rf, red, g * S::TPB + tau,
                                              tokens, clip, out_codes, out_scales, lane, tau, q, [] {});
      g = gn;
    }
  }
  wait_vmcnt<0>();  // no LDS-DMA may still be writing when the workgroup retires
}

// ---------------------------------------------------------------------------
// Few-token kernel (fq_few_kernel): N = 128, M = 16 MB. The decode shapes: a
// few tokens each take the serial chain of one token, so the chain is split
// over a workgroup of four waves (one 32-column pair each, the workgroup
// kernel's layouts; few_products) and the set-up is
// one round trip: the first token's X (by LDS-DMA, in fragment order) and R
// and L (16-byte loads, stored row-major into LDS at a 288-byte pitch, so
// that four consecutive rows start 8 banks apart) are all requested at entry.
// R's and L's fragments are then gathered with LDS transpose reads into VGPRs
// (one wave per SIMD leaves room for L's too). Further tokens of a workgroup
// have their X copied into the other buffer while the current one is used.
// ---------------------------------------------------------------------------
template <int MB>
struct FewShape {
  static constexpr int M = 16 * MB, N = 128, F = M * N;
  static constexpr int KS1 = 4, KS2 = MB / 2;
  static constexpr bool TAIL = (MB & 1) != 0;
  static constexpr int XFRAGS = MB * KS1;          // 1 KiB X fragments per token
  static constexpr int XF_PER_WAVE = XFRAGS / 4;   // == MB
  static constexpr int P = 144;                    // R and L row pitch in elements (288 bytes)
  static_assert(M <= 128, "L rows fit the staging pitch");
};

// Per-token work of the few-token kernel on this wave's 32-column pair q, with
// the workgroup kernel's layouts (X fragments in LDS, R's and L's fragments in
// VGPRs; see fq_mfma_group) and the pair kernel's epilogue, in three parts:
// the two products (few_products), the scale (few_scale) and the codes
// (few_codes_packed / few_codes_int8).
//
// At one wave per SIMD the MFMAs' result latency is the time, so both products
// run G row blocks at a time: 2G independent accumulator chains instead of
// two, each in the same k order (so the results are those of the other
// kernels, bit for bit). Lane (li, lg) of block mb ends with yp[mb][r], the
// D-rounded pair (h = 0, 1) Y[16mb + li][32q + 8lg + 4h + r]: nibbles r and
// r + 4 of word 4q + lg of that row; amax = max |Y| of the wave's raw
// accumulators.
// lfrag(mb, s) returns L's fragment (mb, s) (from VGPRs or LDS); G row blocks
// per step; after_first() runs between the two products (X is no longer read).
struct NoHook {
  __device__ void operator()() const {}
};
template <class DT, int MB, int G = 4, class LFrag, class Hook = NoHook>
__device__ __attribute__((always_inline)) inline void few_products(
    const typename DT::T* __restrict__ xs, LFrag&& lfrag,
    const typename MfmaOps<DT>::V (&rf)[2][FewShape<MB>::KS1], int lane, uint32_t (&yp)[MB][4], float& amax,
    Hook&& after_first = Hook{}) {
  using S = FewShape<MB>;
  using T = typename DT::T;
  using Ops = MfmaOps<DT>;
  using V = typename Ops::V;
  using Epi = FqEpi<DT>;
  constexpr int KS1 = S::KS1, KS2 = S::KS2;
  constexpr int KSL = KS2 + (S::TAIL ? 1 : 0);

  // First product, rounding point 1: zp[h][s][4e + r] = Z[16(2s + e) + 4lg + r][n(h, li)].
  V zp[2][KS2 + 1];
#pragma unroll
  for (int rb0 = 0; rb0 < MB; rb0 += G) {
    V a[G][KS1];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks)
        if (rb0 + g < MB) a[g][ks] = *reinterpret_cast<const V*>(xs + (((rb0 + g) * KS1 + ks) * 64 + lane) * 8);
    v4f c[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) c[g][0] = c[g][1] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks)
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (rb0 + g < MB) {
          c[g][0] = Ops::mfma(a[g][ks], rf[0][ks], c[g][0]);
          c[g][1] = Ops::mfma(a[g][ks], rf[1][ks], c[g][1]);
        }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int rb = rb0 + g;
      if (rb >= MB) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        zp[0][rb >> 1][(rb & 1) * 4 + r] = (T)c[g][0][r];   // MFMA results: no opaque()
        zp[1][rb >> 1][(rb & 1) * 4 + r] = (T)c[g][1][r];
        if (S::TAIL && rb == MB - 1) {                      // zero-padded tail slab
          zp[0][rb >> 1][4 + r] = __builtin_bit_cast(T, (short)0);
          zp[1][rb >> 1][4 + r] = __builtin_bit_cast(T, (short)0);
        }
      }
    }
  }

  after_first();
  // Second product, transposed, rounding point 2, G row blocks of Y at a time.
  amax = 0.f;
#pragma unroll
  for (int mb0 = 0; mb0 < MB; mb0 += G) {
    v4f c[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) c[g][0] = c[g][1] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < KSL; ++sl)
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (mb0 + g < MB) {
          const V lv = lfrag(mb0 + g, sl);
          c[g][0] = Ops::mfma(zp[0][sl], lv, c[g][0]);
          c[g][1] = Ops::mfma(zp[1][sl], lv, c[g][1]);
        }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (mb0 + g >= MB) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        yp[mb0 + g][r] = Epi::pack_acc(c[g][0][r], c[g][1][r]);
        amax = fmaxf(fmaxf(amax, fabsf(c[g][0][r])), fabsf(c[g][1][r]));
      }
    }
  }
}

// The token's scale from max |Y| (clip > 0): a DPP wave maximum, then one LDS
// exchange across the four waves (red[4]; the barrier also orders every
// wave's earlier reads of the X buffer before its refill).
template <class DT>
__device__ inline float few_scale(float amax, float* red, int q, int lane, float clip, float& amax_d) {
  amax = __builtin_bit_cast(float, wave_max_u32(__builtin_bit_cast(uint32_t, amax)));
  if (lane == 0) red[q] = amax;
  lds_barrier();
  amax_d = DT::round(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  return fq_scale_abs<DT>(amax_d, clip);
}

// Packed codes of one token (this lane's word 4q + lg of rows 16mb + li) from
// rcp = 1 / s, without branches or divisions (either would end the block the
// products are scheduled with): a scale of 0 (an all-zero fp16 token) stores
// wrong words here, which few_codes_zero_scale then replaces.
// NOCLAMP (bf16): the token's largest quotient rounds below 7.5 (see
// FqEpi<BF16T>::word_u8_noclamp).
template <class DT, int MB, bool NOCLAMP = false>
__device__ inline void few_codes_packed(const uint32_t (&yp)[MB][4], float rcp, int32_t* orow, int li) {
  using Epi = FqEpi<DT>;
  constexpr int N = FewShape<MB>::N;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    uint32_t w;
    if constexpr (std::is_same<DT, BF16T>::value && NOCLAMP) w = Epi::word_u8_noclamp(yp[mb], rcp);
    else if constexpr (std::is_same<DT, BF16T>::value) w = Epi::word_u8(yp[mb], rcp);
    else w = Epi::template word4<true>(yp[mb], rcp);   // the lower clamp as well: valid for any amax
    orow[(16 * mb + li) * (N / 8)] = (int32_t)w;
  }
}

// Codes of a token whose scale rounded to 0: the fallback's 0/0 codes.
template <class DT, int MB>
__device__ inline void few_codes_zero_scale(const uint32_t (&yp)[MB][4], float s, int32_t* orow, int li) {
  using Epi = FqEpi<DT>;
  constexpr int N = FewShape<MB>::N;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    uint32_t w = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      w |= (uint32_t)(fq_code_from_quot<true>(DT::round(opaque(Epi::lo(yp[mb][r])) / s)) + 8) << (4 * r);
      w |= (uint32_t)(fq_code_from_quot<true>(DT::round(opaque(Epi::hi(yp[mb][r])) / s)) + 8) << (4 * r + 16);
    }
    orow[(16 * mb + li) * (N / 8)] = (int32_t)w;
  }
}

// int8 codes of one token: 8 bytes per row block (columns 32q + 8lg .. + 7).
template <class DT, int MB>
__device__ inline void few_codes_int8(const uint32_t (&yp)[MB][4], float s, int8_t* orow, int li) {
  using Epi = FqEpi<DT>;
  constexpr int N = FewShape<MB>::N;
  const float rcp = 1.0f / s;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float y0 = Epi::lo(yp[mb][r]), y1 = Epi::hi(yp[mb][r]);
      int c0, c1;
      if (s > 0.f) {
        c0 = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y0 * rcp, -8.0f, 7.0f)));
        c1 = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y1 * rcp, -8.0f, 7.0f)));
      } else {
        c0 = fq_code_from_quot<false>(DT::round(opaque(y0) / s));
        c1 = fq_code_from_quot<false>(DT::round(opaque(y1) / s));
      }
      lo4 |= (uint32_t)(c0 & 0xFF) << (8 * r);
      hi4 |= (uint32_t)(c1 & 0xFF) << (8 * r);
    }
    *reinterpret_cast<v2i*>(orow + (16 * mb + li) * N) = v2i{(int)lo4, (int)hi4};
  }
}

// LDS of the few-token routine, carved from one byte array: the X buffers
// (buffer b of slot p at (b SLOTS + p) XE elements), R's and L's staging rows
// (one slot; with two, R and then L go through the two slots' second buffers,
// free at set-up), L's fragments (two slots) and the scale exchange.
template <int MB, int SLOTS>
struct FewLds {
  using S = FewShape<MB>;
  static constexpr int XE = S::XFRAGS * 512;             // elements of one token's X buffer
  static constexpr int LF_FRAGS = MB * (S::KS2 + 1);
  static constexpr int STAGE_E = SLOTS == 1 ? (S::N + S::M) * S::P : 8;
  static constexpr int XB_OFF = 0;
  static constexpr int STAGE_OFF = XB_OFF + 2 * SLOTS * XE * 2;
  static constexpr int LF_OFF = STAGE_OFF + STAGE_E * 2;
  static constexpr int RED_OFF = LF_OFF + (SLOTS == 1 ? 16 : LF_FRAGS * 1024);
  static constexpr int BYTES = RED_OFF + SLOTS * 16;
  static_assert(SLOTS == 1 || (S::N * S::P <= 2 * XE && S::M * S::P <= 2 * XE), "staging fits two X buffers");
  static_assert(STAGE_OFF % 16 == 0 && LF_OFF % 16 == 0, "16-byte aligned parts");
};

// The few-token routine of workgroup `group` of `groups`, on the 256 SLOTS
// threads of the workgroup and LDS of FewLds<MB, SLOTS>::BYTES at `lds`.
// SLOTS = 1: one token at a time per workgroup, L's fragments in VGPRs (one
// wave per SIMD). SLOTS = 2 (many tokens): two tokens at a time, four waves
// each (two waves per SIMD, so one token's MFMA or VALU work can run while the
// other waits), L's fragments in LDS, shared by all eight waves.
template <class DT, int MB, bool PACK, int SLOTS>
__device__ __attribute__((always_inline)) inline void few_quantize(
    unsigned char* lds, const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
    const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
    void* __restrict__ out_codes, float* __restrict__ out_scales, int64_t group, int64_t groups) {
  using S = FewShape<MB>;
  using LD = FewLds<MB, SLOTS>;
  using T = typename DT::T;
  using V = typename MfmaOps<DT>::V;
  static_assert(sizeof(T) == 2, "16-bit inputs");
  constexpr int M = S::M, N = S::N, KS1 = S::KS1, KS2 = S::KS2, P = S::P;
  constexpr int XE = LD::XE;
  constexpr int LF_FRAGS = LD::LF_FRAGS;
  T* const xb = reinterpret_cast<T*>(lds + LD::XB_OFF);
  T* const stage_arr = reinterpret_cast<T*>(lds + LD::STAGE_OFF);
  unsigned char* const lfs = lds + LD::LF_OFF;
  float* const red = reinterpret_cast<float*>(lds + LD::RED_OFF);

  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = wave & 3;                 // this wave's 32-column pair
  const int p = SLOTS == 1 ? 0 : wave >> 2;   // its token slot
  T* const rst = SLOTS == 1 ? stage_arr : xb + SLOTS * XE;   // the second buffers
  T* const lst = SLOTS == 1 ? stage_arr + N * P : xb + SLOTS * XE;

  // LDS-DMA of token tt's X: this wave copies fragments q, q + 4, ...; lane l
  // of fragment (rb, ks) fetches X[16rb + l%16][32ks + 8(l/16) .. +7]. The
  // copies are issued as inline assembly (dma16): the compiler then adds no
  // wait of its own for them (with the builtin it waits for every outstanding
  // load before the next LDS read, which would also wait for the next token's
  // copy); the loop below waits for them explicitly.
  auto issue = [&](int64_t tt, T* stage) {
    tt = tt < tokens ? tt : tokens - 1;   // past the last token: a valid row, never stored
    const T* base = x + tt * x_ld + li * N + 8 * lg;
    const uint32_t lbase = lds_addr(stage);
#pragma unroll
    for (int i = 0; i < S::XF_PER_WAVE; ++i) {
      const int f = q + 4 * i;
      dma16(base + (f / KS1) * 16 * N + 32 * (f % KS1), lbase + f * 1024);
    }
  };

  // tokens of slot p: blockIdx SLOTS + p, then every SLOTS grid further on
  const int64_t stride = groups * SLOTS;
  int64_t t = group * SLOTS + p;
  const int64_t t_slot0 = group * SLOTS;   // slot 0 has at least as many tokens as slot 1
  T* cur = xb + p * XE;
  T* nxt = xb + (SLOTS + p) * XE;
  issue(t, cur);
  // R (N x N) and L (M x M) as 16-byte chunks, all loads before any store
  constexpr int NT = 256 * SLOTS;
  constexpr int RCH = N * N / 8, LCH = M * M / 8;
  constexpr int RPT = (RCH + NT - 1) / NT, LPT = (LCH + NT - 1) / NT;
  v4i rtmp[RPT], ltmp[LPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + NT * i;
    rtmp[i] = reinterpret_cast<const v4i*>(right)[c < RCH ? c : 0];
  }
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int c = tid + NT * i;
    ltmp[i] = reinterpret_cast<const v4i*>(left)[c < LCH ? c : 0];
  }
  auto store_l = [&]() {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + NT * i;   // row c / (M / 8)
      if (c < LCH) *reinterpret_cast<v4i*>(lst + (c / (M / 8)) * P + 8 * (c % (M / 8))) = ltmp[i];
    }
  };
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + NT * i;   // row c / 16, 8 elements from column 8 (c % 16)
    if (c < RCH) *reinterpret_cast<v4i*>(rst + (c >> 4) * P + 8 * (c & 15)) = rtmp[i];
  }
  if constexpr (SLOTS == 1) store_l();
  lds_barrier();
  // R fragments of this pair, rf[h][ks][j] = R[32ks + 8lg + j][n],
  // n = 32q + 8(li/4) + 4h + li%4: lane l supplies row 32ks + 8lg + l/4 (+4),
  // columns 32q + 8(l%4) + 4h .. +3, and receives column 32q + 8(l/4) + 4h + l%4.
  V rf[2][KS1];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) {
      const T* at = rst + (32 * ks + 8 * lg + (li >> 2)) * P + 32 * q + 8 * (li & 3) + 4 * h;
      rf[h][ks] = join_tr16<V>(lds_tr16(at), lds_tr16(at + 4 * P));
    }
  // L fragments, lf[mb][s][j] = L[32s + 16(j/4) + 4lg + j%4][16mb + li]; the
  // zero-padded tail slab (s = KS2, M / 16 odd) has elements 4..7 zero.
  auto lgather = [&](int mb, int sl) -> V {
    const T* at = lst + (32 * sl + 4 * lg + (li >> 2)) * P + 16 * mb + 4 * (li & 3);
    if (sl < KS2) return join_tr16<V>(lds_tr16(at), lds_tr16(at + 16 * P));
    if (S::TAIL) return join_tr16<V>(lds_tr16(at), v4s16{0, 0, 0, 0});
    return V{};
  };
  V lf[SLOTS == 1 ? MB : 1][KS2 + 1];
  if constexpr (SLOTS == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int sl = 0; sl <= KS2; ++sl) lf[mb][sl] = lgather(mb, sl);
  } else {
    lds_barrier();   // every wave holds R's fragments: L may overwrite R's staged rows
    store_l();
    lds_barrier();
#pragma unroll 1
    for (int fr = wave; fr < LF_FRAGS; fr += 4 * SLOTS)
      *reinterpret_cast<V*>(lfs + fr * 1024 + 16 * lane) = lgather(fr / (KS2 + 1), fr % (KS2 + 1));
    lds_barrier();   // L's fragments written; the staging buffers are free for X
  }
  auto lfrag = [&](int mb, int sl) -> V {
    if constexpr (SLOTS == 1) return lf[mb][sl];
    else return *reinterpret_cast<const V*>(lfs + (mb * (KS2 + 1) + sl) * 1024 + 16 * lane);
  };

  // One token per slot and iteration: the next token's X goes into the other
  // buffer, then this wave's copies of the current one are waited for (copies
  // retire in order; stores issued in between only make the count stricter)
  // and a barrier makes every wave's share visible. The barrier inside
  // few_scale comes after every wave's reads of the current buffer, so the
  // buffer can be refilled in the next iteration. Both slots run the same
  // number of iterations (slot 1's past the last token compute on the last
  // token and store nothing), so they meet at every barrier.
  //
  // Packed codes are software-pipelined: token i's codes (VALU work) are
  // computed in the iteration of token i + 1's products (MFMA work).
  // stored: this wave issued a token's MB code stores after the current
  // buffer's copies (the pipelined packed loop below): then those stores may
  // stay outstanding too, since copies and stores retire in order.
  auto next_x = [&](int64_t tn, bool stored = false) {
    if (tn < tokens + (SLOTS - 1)) {   // slot 1 copies (a valid row) as long as slot 0 has a token
      issue(tn, nxt);
      if (stored) wait_vmcnt<S::XF_PER_WAVE + MB>();
      else wait_vmcnt<S::XF_PER_WAVE>();
    } else {
      if (stored) wait_vmcnt<MB>();
      else wait_vmcnt<0>();
    }
    raw_barrier();
  };
  float* const red_p = red + 4 * p;
  if constexpr (PACK) {
    uint32_t ypp[MB][4];
    float sp, rcpp, amax_d;
    int64_t tp = t;
    {
      const int64_t tn = t + stride;
      next_x(tn);
      float amax;
      few_products<DT, MB>(cur, lfrag, rf, lane, ypp, amax);
      sp = few_scale<DT>(amax, red_p, q, lane, clip, amax_d);
      rcpp = 1.0f / sp;
      if (q == 0 && lane == 0 && t < tokens) out_scales[t] = sp;
      T* tmp = cur;
      cur = nxt;
      nxt = tmp;
      t = tn;
    }
    bool stored = false;   // the previous iteration stored token tp's codes
    for (int64_t t0 = t_slot0 + stride; t0 < tokens; t0 += stride) {
      const int64_t tn = t + stride;
      next_x(tn, stored);
      uint32_t yp[MB][4];
      float amax;
      few_products<DT, MB>(cur, lfrag, rf, lane, yp, amax);
      int32_t* orowp = reinterpret_cast<int32_t*>(out_codes) + tp * (S::F / 8) + 4 * q + lg;
      stored = tp < tokens;
      if (stored) few_codes_packed<DT, MB>(ypp, rcpp, orowp, li);
      const float s = few_scale<DT>(amax, red_p, q, lane, clip, amax_d);
      if (q == 0 && lane == 0 && t < tokens) out_scales[t] = s;
      if (tp < tokens && !(sp > 0.f)) few_codes_zero_scale<DT, MB>(ypp, sp, orowp, li);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) ypp[mb][r] = yp[mb][r];
      sp = s;
      rcpp = 1.0f / s;
      tp = t;
      T* tmp = cur;
      cur = nxt;
      nxt = tmp;
      t = tn;
    }
    int32_t* orowp = reinterpret_cast<int32_t*>(out_codes) + tp * (S::F / 8) + 4 * q + lg;
    if (tp < tokens) {
      few_codes_packed<DT, MB>(ypp, rcpp, orowp, li);
      if (!(sp > 0.f)) few_codes_zero_scale<DT, MB>(ypp, sp, orowp, li);
    }
  } else {
    for (int64_t t0 = t_slot0; t0 < tokens; t0 += stride) {
      const int64_t tn = t + stride;
      next_x(tn);
      uint32_t yp[MB][4];
      float amax, amax_d;
      few_products<DT, MB>(cur, lfrag, rf, lane, yp, amax);
      const float s = few_scale<DT>(amax, red_p, q, lane, clip, amax_d);
      if (t < tokens) {
        if (q == 0 && lane == 0) out_scales[t] = s;
        few_codes_int8<DT, MB>(yp, s, reinterpret_cast<int8_t*>(out_codes) + t * S::F + 32 * q + 8 * lg, li);
      }
      T* tmp = cur;
      cur = nxt;
      nxt = tmp;
      t = tn;
    }
  }
  wait_vmcnt<0>();  // no LDS-DMA may still be writing when the workgroup retires
}

template <class DT, int MB, bool PACK, int SLOTS>
__global__ void __launch_bounds__(256 * SLOTS) __attribute__((amdgpu_waves_per_eu(SLOTS, SLOTS)))
fq_few_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
              const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
              void* __restrict__ out_codes, float* __restrict__ out_scales) {
  __shared__ __align__(16) unsigned char lds[FewLds<MB, SLOTS>::BYTES];
  few_quantize<DT, MB, PACK, SLOTS>(lds, x, tokens, x_ld, left, right, clip, out_codes, out_scales, blockIdx.x,
                                    gridDim.x);
}

// ---------------------------------------------------------------------------
// Compact few-token routine (fq_few2_kernel): the same per-token work as
// few_quantize with one slot, in at most 256 registers and about 64 KB of LDS,
// so that two workgroups share a CU (two waves per SIMD: one workgroup's MFMA
// or VALU work runs while the other waits). Against the one-slot routine:
// one X buffer (the next token's X is requested once every wave has read the
// current one: after the first product, or after the scale's barrier); R and
// then L staged through one area; one or two row blocks per product step;
// the codes right after the scale (no cross-token pipelining).
// ---------------------------------------------------------------------------
template <int MB>
struct FewLdsCompact {
  using S = FewShape<MB>;
  static constexpr int XE = S::XFRAGS * 512;
  static constexpr int STAGE_OFF = XE * 2;
  static constexpr int STAGE_E = (S::N > S::M ? S::N : S::M) * S::P;
  static constexpr int RED_OFF = STAGE_OFF + STAGE_E * 2;
  static constexpr int BYTES = RED_OFF + 16;
  static_assert(STAGE_OFF % 16 == 0 && BYTES <= 80 * 1024, "two workgroups per CU");
};

template <class DT, int MB, bool PACK, bool NOCLAMP, bool STAGE>
__device__ __attribute__((always_inline)) inline void few_quantize_compact(
    unsigned char* lds, const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
    const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
    void* __restrict__ out_codes, float* __restrict__ out_scales, int64_t group, int64_t groups) {
  using S = FewShape<MB>;
  using LD = FewLdsCompact<MB>;
  using T = typename DT::T;
  using V = typename MfmaOps<DT>::V;
  static_assert(sizeof(T) == 2, "16-bit inputs");
  constexpr int M = S::M, N = S::N, KS1 = S::KS1, KS2 = S::KS2, P = S::P;
  // Measured (8192 x 112 x 128, same process): bf16 requests the next X
  // between the two products (one more barrier per token; 81.4 -> 77.9 us)
  // with two row blocks per step; fp16 fits its registers only with one row
  // block per step (two spilled: 86.2 -> 74.1 us) and is faster with the
  // request after the scale (76.2 vs 80.6 us).
  constexpr bool kF16 = std::is_same<DT, F16T>::value;
  constexpr int kG = kF16 ? 1 : 2;
  constexpr bool kEarly = !kF16;
  T* const xb = reinterpret_cast<T*>(lds);
  T* const stage = reinterpret_cast<T*>(lds + LD::STAGE_OFF);
  float* const red = reinterpret_cast<float*>(lds + LD::RED_OFF);
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int q = __builtin_amdgcn_readfirstlane(tid >> 6);   // this wave's 32-column pair

  // LDS-DMA of token tt's X in fragment order (as few_quantize)
  auto issue = [&](int64_t tt) {
    const T* base = x + tt * x_ld + li * N + 8 * lg;
    const uint32_t lbase = lds_addr(xb);
#pragma unroll
    for (int i = 0; i < S::XF_PER_WAVE; ++i) {
      const int f = q + 4 * i;
      dma16(base + (f / KS1) * 16 * N + 32 * (f % KS1), lbase + f * 1024);
    }
  };
  int64_t t = group;
  if (t >= tokens) return;
  issue(t);
  // R and L as 16-byte chunks, all loads before any store; R staged first
  constexpr int RCH = N * N / 8, LCH = M * M / 8;
  constexpr int RPT = (RCH + 255) / 256, LPT = (LCH + 255) / 256;
  v4i rtmp[RPT], ltmp[LPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + 256 * i;
    rtmp[i] = reinterpret_cast<const v4i*>(right)[c < RCH ? c : 0];
  }
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int c = tid + 256 * i;
    ltmp[i] = reinterpret_cast<const v4i*>(left)[c < LCH ? c : 0];
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int c = tid + 256 * i;   // row c / 16, 8 elements from column 8 (c % 16)
    if (c < RCH) *reinterpret_cast<v4i*>(stage + (c >> 4) * P + 8 * (c & 15)) = rtmp[i];
  }
  lds_barrier();
  // R's fragments (as few_quantize)
  V rf[2][KS1];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) {
      const T* at = stage + (32 * ks + 8 * lg + (li >> 2)) * P + 32 * q + 8 * (li & 3) + 4 * h;
      rf[h][ks] = join_tr16<V>(lds_tr16(at), lds_tr16(at + 4 * P));
    }
  lds_barrier();   // every wave holds R's fragments: L may overwrite R's rows
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int c = tid + 256 * i;   // row c / (M / 8)
    if (c < LCH) *reinterpret_cast<v4i*>(stage + (c / (M / 8)) * P + 8 * (c % (M / 8))) = ltmp[i];
  }
  lds_barrier();
  V lf[MB][KS2 + 1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int sl = 0; sl <= KS2; ++sl) {
      const T* at = stage + (32 * sl + 4 * lg + (li >> 2)) * P + 16 * mb + 4 * (li & 3);
      if (sl < KS2) lf[mb][sl] = join_tr16<V>(lds_tr16(at), lds_tr16(at + 16 * P));
      else if (S::TAIL) lf[mb][sl] = join_tr16<V>(lds_tr16(at), v4s16{0, 0, 0, 0});
      else lf[mb][sl] = V{};
    }
  auto lfrag = [&](int mb, int sl) -> V { return lf[mb][sl]; };

  // One token per iteration: wait for this wave's copies, a barrier for every
  // wave's (and, from the second token on, for every wave's reads of the
  // scale exchange), the products, the scale, then this token's codes; the
  // next token's copy goes out once every wave's reads of X are done. Vector
  // memory operations retire in order, and after a token's copies every wave
  // issues at least MB code stores of the token before: waiting until at
  // most MB remain waits for the copies, not for those stores.
  //
  // STAGE (bf16 packed codes, 16-byte aligned output): a token's codes go to
  // the staging area (free after the set-up) instead of memory, and the
  // workgroup copies them out as whole 16-byte pieces of the token's
  // contiguous codes during the next token, after its X request (so the wait
  // at the top of a token still waits only for the copies: at least one store
  // of every wave follows them). Without staging, each 64-byte row of codes
  // is written in 16-byte parts by four waves. The last token's codes go out
  // after the loop, non-temporal when the workgroup had more than one token
  // (they would otherwise sit dirty in L2 for the write-back at the kernel's
  // end; with one token per workgroup, the decode sizes, the next GEMM reads
  // them at once and they stay plain). Measured (same process, outputs
  // equal, two boxes): 8192 x 112 x 128 74.3 -> 73.0 / 78.6 -> 76.5 us,
  // 4096 x 112 x 128 at clip 0.9 41.2 -> 39.8 / 42.3 -> 42.3, 8192 x 64 x 128
  // 41.8 -> 39.9 / 44.2 -> 41.8; the linear step at 16 and 4096 tokens within
  // the boxes' spread (15.8 -> 15.9, 195.0 -> 194.9 / 199.0 -> 200.1 us).
  static_assert(!STAGE || (kEarly && PACK), "staging: bf16 packed codes");
  int32_t* const cst = reinterpret_cast<int32_t*>(stage);
  constexpr int PIECES = S::F / 32;   // 16-byte pieces of a token's packed codes
  static_assert(S::F / 8 * 4 <= LD::STAGE_E * 2, "a token's codes fit the staging area");
  auto store_staged = [&](int64_t tt, auto nt) {
    const v4i* src = reinterpret_cast<const v4i*>(cst);
    v4i* dst = reinterpret_cast<v4i*>(reinterpret_cast<int32_t*>(out_codes) + tt * (S::F / 8));
#pragma unroll
    for (int i = 0; i < (PIECES + 255) / 256; ++i) {
      const int pc = tid + 256 * i;
      if (pc < PIECES) {
        if constexpr (decltype(nt)::value) __builtin_nontemporal_store(src[pc], dst + pc);
        else dst[pc] = src[pc];
      }
    }
  };
  static_assert(!STAGE || PIECES > 192, "every wave stores at least one piece per staged token");
  for (; t < tokens; t += groups) {
    if (t == group || (STAGE && t == group + groups)) wait_vmcnt<0>();
    else wait_vmcnt<(STAGE ? 1 : MB)>();
    raw_barrier();
    uint32_t yp[MB][4];
    float amax, amax_d;
    if constexpr (kEarly) {
      few_products<DT, MB, kG>(xb, lfrag, rf, lane, yp, amax, [&]() {
        lds_barrier();   // every wave's reads of X (and of the staged codes' previous readers) are done
        if (t + groups < tokens) issue(t + groups);
        if (STAGE && t != group) store_staged(t - groups, std::false_type{});
      });
    } else {
      few_products<DT, MB, kG>(xb, lfrag, rf, lane, yp, amax);
    }
    const float sc = few_scale<DT>(amax, red, q, lane, clip, amax_d);
    if (!kEarly && t + groups < tokens) issue(t + groups);
    if (q == 0 && lane == 0) out_scales[t] = sc;
    if constexpr (PACK) {
      int32_t* orow = (STAGE ? cst : reinterpret_cast<int32_t*>(out_codes) + t * (S::F / 8)) + 4 * q + lg;
      few_codes_packed<DT, MB, NOCLAMP>(yp, 1.0f / sc, orow, li);
      if (!(sc > 0.f)) few_codes_zero_scale<DT, MB>(yp, sc, orow, li);
    } else {
      few_codes_int8<DT, MB>(yp, sc, reinterpret_cast<int8_t*>(out_codes) + t * S::F + 32 * q + 8 * lg, li);
    }
  }
  if constexpr (STAGE) {
    lds_barrier();   // the last token's codes are staged
    const int64_t last = group + (tokens - 1 - group) / groups * groups;
    if (last != group) {
      // fenced so that the compiler cannot merge these stores with the plain
      // branch's (a merged store loses the non-temporal flag)
      asm volatile("" ::: "memory");
      store_staged(last, std::true_type{});
      asm volatile("" ::: "memory");
    } else {
      store_staged(last, std::false_type{});
    }
  }
  wait_vmcnt<0>();  // no LDS-DMA may still be writing when the workgroup retires
}

// Read-ahead share of workgroup blockIdx (>= qgroups, on XCD blockIdx % 8):
// the rows of the GEMM workgroups j with j % 8 == that XCD, listed unit by
// unit (16 rows, len16 16-byte chunks each; row stride rs16 chunks) and split
// into equal contiguous shares over the read-ahead workgroups of the XCD.
// Eight 16-byte loads per thread in flight, the values dropped (an empty asm
// statement takes each), and a short sleep after each issue: measured at 16
// tokens (112 x 128 -> 4096 x 14336), the weight read in a burst delays the
// quantize's own loads (step 17.0 -> 17.2 us), paced at about 320 cycles per
// load and wave it ends with the quantize (17.0 -> 16.1 us; 1 token 16.2 ->
// 15.6 us). Reads only; every access is inside the rows given.
__device__ inline void read_ahead_rows(const v4i* __restrict__ p, int64_t rows, int64_t rs16, int len16,
                                       int qgroups) {
  const int b = blockIdx.x, x = b % 8, grid = gridDim.x;
  const int first = qgroups + ((x - qgroups % 8) + 8) % 8;   // first read-ahead workgroup on this XCD
  if (first >= grid) return;
  const int k = (b - first) / 8, nx = (grid - 1 - first) / 8 + 1;
  const int units = (int)((rows + 15) / 16);
  const int upx = units > x ? (units - x + 7) / 8 : 0;        // GEMM workgroups on this XCD
  const int per_unit = 16 * len16, total = upx * per_unit;
  const int share = (total + nx - 1) / nx, lo = k * share, hi = min(total, lo + share);
  // element e of the XCD's list: chunk cc of row rr of unit uu (GEMM workgroup x + 8 uu)
  int e = lo + (int)threadIdx.x;
  int uu = e / per_unit, rr = e % per_unit / len16, cc = e % len16;
  while (e < hi) {
    v4i v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t row = min((int64_t)16 * (x + 8 * uu) + rr, rows - 1);
      v[u] = p[e < hi ? row * rs16 + cc : 0];
      __builtin_amdgcn_s_sleep(5);
      e += 256;   // next element of this thread
      cc += 256;
      while (cc >= len16) {
        cc -= len16;
        if (++rr == 16) {
          rr = 0;
          ++uu;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) asm volatile("" ::"v"(v[u]));
  }
}

// Workgroups 0 .. qgroups - 1 quantize; the rest, if any, read ahead.
// NOCLAMP (bf16, packed codes): the host has found from the clip ratio that no
// quotient can round to 7.5 or above (kNoClampClip).
template <class DT, int MB, bool PACK, bool NOCLAMP = false, bool STAGE = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fq_few2_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
               const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
               void* __restrict__ out_codes, float* __restrict__ out_scales, int qgroups,
               const v4i* __restrict__ ahead, int64_t ahead_rows, int64_t ahead_rs16, int ahead_len16) {
  __shared__ __align__(16) unsigned char lds[FewLdsCompact<MB>::BYTES];
  if ((int)blockIdx.x >= qgroups) {
    read_ahead_rows(ahead, ahead_rows, ahead_rs16, ahead_len16, qgroups);
    return;
  }
  few_quantize_compact<DT, MB, PACK, NOCLAMP, STAGE>(lds, x, tokens, x_ld, left, right, clip, out_codes,
                                                     out_scales, blockIdx.x, qgroups);
}

// ---------------------------------------------------------------------------
// Wave-per-token kernel (fq_wave_kernel): M = 16*MB with MB even, N = 32*NQ,
// small enough that one wavefront holds a whole token (M = N = 64 at most).
//
// * X arrives by direct 16-byte loads straight into A-operand fragments: lane
//   (li, lg) loads X[16rb + li][32ks + 8lg .. +7], each element once.
// * L and R fragments are built once per workgroup by the matrix core. The
//   fragments need columns of L and R (8 consecutive rows of one column per
//   lane), while memory holds rows; an MFMA whose B operand is a one-hot
//   selection matrix turns a row-major 16 x 32 tile (coalesced 16-byte loads)
//   into that order: D[4lg + r][li] = A[4lg + r][sel(li)], exact, since every
//   output is one product with 1.0 plus zeros. The waves split the build,
//   exchange the fragments through LDS (one barrier) and keep them in VGPRs.
// * The second product runs transposed as in fq_mfma_kernel, and a column
//   permutation (wave_col) leaves each lane with whole packed words, adjacent
//   ones, so every store instruction writes 16 complete rows of codes.
// * The scale needs only an in-wave reduction.
//
// Waves loop over tokens (stride = all waves of the grid); the next token's X
// is loaded into the fragment registers as soon as the first product has
// consumed them. The scale comes from max |Y| (fq_scale_abs), so the host
// routes clip <= 0 elsewhere.
// ---------------------------------------------------------------------------


template <class DT>
struct DBits;
template <>
struct DBits<F16T> {
  static constexpr uint32_t one = 0x3C00u;
};
template <>
struct DBits<BF16T> {
  static constexpr uint32_t one = 0x3F80u;
};

// B operand of the 16x16x32 MFMA selecting A column src for output column li:
// lane (li, lg) holds B[8lg + j][li] = (8lg + j == src) for j = 0..7.
template <class DT>
__device__ inline typename MfmaOps<DT>::V onehot_b(int src, int lg) {
  const int j = src - 8 * lg;   // the lane's slot holding the one, if 0 <= j < 8
  const uint32_t bits = DBits<DT>::one << (16 * (j & 1));
  v4i w;
#pragma unroll
  for (int d = 0; d < 4; ++d) w[d] = ((unsigned)j < 8u && (j >> 1) == d) ? (int)bits : 0;
  return __builtin_bit_cast(typename MfmaOps<DT>::V, w);
}

// Two selection products of the rows tiles a0 (slots j = 0..3) and a1 (slots
// j = 4..7) assembled into one 8-element fragment (values are exact in D).
template <class DT>
__device__ inline typename MfmaOps<DT>::V pack_frag(v4f d0, v4f d1) {
  const v4i w = {(int)FqEpi<DT>::pack(d0[0], d0[1]), (int)FqEpi<DT>::pack(d0[2], d0[3]),
                 (int)FqEpi<DT>::pack(d1[0], d1[1]), (int)FqEpi<DT>::pack(d1[2], d1[3])};
  return __builtin_bit_cast(typename MfmaOps<DT>::V, w);
}

template <class DT>
__device__ inline typename MfmaOps<DT>::V transpose_frag(typename MfmaOps<DT>::V a0, typename MfmaOps<DT>::V a1,
                                                        typename MfmaOps<DT>::V sel) {
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  return pack_frag<DT>(MfmaOps<DT>::mfma(a0, sel, z), MfmaOps<DT>::mfma(a1, sel, z));
}

template <class DT, int MB, int NQ>
__device__ inline void fq_wave_load_x(const typename DT::T* __restrict__ xt,
                                      typename MfmaOps<DT>::V (&xf)[MB][NQ], int li, int lg) {
  constexpr int N = 32 * NQ;
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks)
      xf[rb][ks] = *reinterpret_cast<const typename MfmaOps<DT>::V*>(xt + (16 * rb + li) * N + 32 * ks + 8 * lg);
}

// Store N adjacent 32-bit words (N = 1, 2 or 4) with one instruction,
// non-temporal if NT.
template <int NW_, bool NT>
__device__ inline void store_words(int32_t* dst, const uint32_t (&w)[NW_]) {
  if constexpr (NW_ == 1) {
    if constexpr (NT) __builtin_nontemporal_store((int32_t)w[0], dst);
    else *dst = (int32_t)w[0];
  } else if constexpr (NW_ == 2) {
    const v2i v = {(int)w[0], (int)w[1]};
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<v2i*>(dst));
    else *reinterpret_cast<v2i*>(dst) = v;
  } else {
    static_assert(NW_ == 4, "1, 2 or 4 words");
    const v4i v = {(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(dst));
    else *reinterpret_cast<v4i*>(dst) = v;
  }
}

// Packed codes of a wave kernel token: lane (li, lg) writes row 16mb + li,
// words NQ lg .. NQ lg + NQ - 1 (orow already offset by NQ lg).
template <class DT, int MB, int NQ, bool LOW, bool NT>
__device__ inline void fq_wave_store_codes(int32_t* orow, const uint32_t (&yp)[MB][NQ][4], float rcp, int li) {
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    uint32_t words[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) words[q] = FqEpi<DT>::template word4<LOW>(yp[mb][q], rcp);
    store_words<NQ, NT>(orow + (16 * mb + li) * (4 * NQ), words);
  }
}

// fq_wave_store_codes, non-temporal when nt (uniform). The empty asm
// statements around the non-temporal branch keep the compiler from hoisting or
// sinking its stores into the plain branch's (merged stores lose the flag).
template <class DT, int MB, int NQ, bool LOW>
__device__ inline void fq_wave_store_codes(int32_t* orow, const uint32_t (&yp)[MB][NQ][4], float rcp, int li,
                                           bool nt) {
  if (nt) {
    asm volatile("" ::: "memory");
    fq_wave_store_codes<DT, MB, NQ, LOW, true>(orow, yp, rcp, li);
    asm volatile("" ::: "memory");
  } else {
    fq_wave_store_codes<DT, MB, NQ, LOW, false>(orow, yp, rcp, li);
  }
}

// Transform fragments of the wave kernel in LDS: R's rf[q][h][ks] at index
// (2q + h) KS1 + ks, then L's lf[mb][s] at 2 NQ KS1 + mb KS2 + s; one 1 KiB
// fragment per index (16 bytes per lane). A build job is one pair of row tiles
// and the two fragments its selection products give: R job (q, ks) ->
// rf[q][0..1][ks], L job (s, p) -> lf[2p..2p+1][s].
template <int MB, int NQ>
struct WaveFrags {
  static constexpr int KS1 = NQ, KS2 = MB / 2;
  static constexpr int NR = 2 * NQ * KS1;
  static constexpr int NF = NR + MB * KS2;
  static constexpr int JR = NQ * KS1;            // R jobs
  static constexpr int NJ = JR + KS2 * (MB / 2); // all jobs
};

constexpr int kWaveKernelWaves = 8;

// Column permutation of the wave kernel: MFMA block (q, h) of the first
// product, lane column i, is physical column n = 8 NQ (i/4) + 8q + 4h + i%4.
// After the transposed second product, lane (li, lg) of block (q, h) holds the
// columns 8 (NQ lg + q) + 4h + r: packed word NQ lg + q, nibbles 4h + r. The
// lane's NQ words of a row are adjacent, so one store per row block writes 16
// whole rows.
template <int NQ>
__device__ inline int wave_col(int q, int h, int i) {
  return 8 * NQ * (i >> 2) + 8 * q + 4 * h + (i & 3);
}

template <class DT, int MB, int NQ, bool PACK>
__global__ void __launch_bounds__(64 * kWaveKernelWaves)
fq_wave_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
               const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
               void* __restrict__ out_codes, float* __restrict__ out_scales) {
  static_assert(MB % 2 == 0 && MB >= 2 && NQ >= 1, "shape");
  using T = typename DT::T;
  using Ops = MfmaOps<DT>;
  using V = typename Ops::V;
  using Epi = FqEpi<DT>;
  using W = WaveFrags<MB, NQ>;
  constexpr int NW = kWaveKernelWaves;
  constexpr int M = 16 * MB, N = 32 * NQ, F = M * N;
  constexpr int KS1 = W::KS1;    // 32-deep slabs of the first product (k = n')
  constexpr int KS2 = W::KS2;    // 32-deep slabs of the second product (k = m')
  static_assert(W::NJ <= NW, "one fragment build job per wave at most");
  __shared__ __align__(16) unsigned char frag_lds[W::NF * 1024];

  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * NW;
  int64_t t = (int64_t)blockIdx.x * NW + wave;

  // Row tiles of this wave's build job first, then the first token's X: the
  // build below waits only for the tiles (loads retire in order) while X is
  // still in flight. No divergent branch precedes the X loads, so the
  // compiler's wait counts stay exact: a wave without a job repeats the last
  // one (same bytes to the same place), a wave without a token loads the last
  // token and stores nothing.
  //   R job (q, ks), tile (c, e): A[i][k] = R[32ks + 8(i/4) + i%4 + 4e][32c + k]
  //   L job (s, p),  tile (0, e): A[i][k] = L[32s + 16e + i][32p + k]
  const int j = min(wave, W::NJ - 1);
  const bool rjob = j < W::JR;
  V ra[NQ][2], la[2];
  if (rjob) {
    const int ks = j % KS1;
#pragma unroll
    for (int c = 0; c < NQ; ++c) {
      const T* base = right + (32 * ks + 8 * (li >> 2) + (li & 3)) * N + 32 * c + 8 * lg;
      ra[c][0] = *reinterpret_cast<const V*>(base);
      ra[c][1] = *reinterpret_cast<const V*>(base + 4 * N);
    }
  } else {
    const int s = (j - W::JR) / (MB / 2), p = (j - W::JR) % (MB / 2);
    const T* base = left + (32 * s + li) * M + 32 * p + 8 * lg;
    la[0] = *reinterpret_cast<const V*>(base);
    la[1] = *reinterpret_cast<const V*>(base + 16 * M);
  }
  // Waves issue their first token's loads about 320 cycles apart, in wave
  // order: the memory system then returns a workgroup's tokens one after
  // another instead of all of them at the end of the stream, so early tokens
  // compute while later ones are still arriving (4-6% at 2048-8192 tokens of
  // 64 x 64). The delay sits in a branch without memory instructions, which
  // leaves the compiler's wait counts exact.
  for (int k = 0; k < wave; ++k) __builtin_amdgcn_s_sleep(5);
  V xf[MB][KS1];
  fq_wave_load_x<DT, MB, NQ>(x + min(t, tokens - 1) * x_ld, xf, li, lg);

  // Build (selection products, exact):
  //   rf[q][h][ks][j] = R[32ks + 8lg + j][wave_col(q, h, li)], summed over the
  //                     column tiles c (only the tile holding the column selects)
  //   lf[mb][s][j]    = L[32s + 16(j/4) + 4lg + j%4][16mb + li], mb = 2p + cc
  {
    int f0, f1;
    V g0, g1;
    if (rjob) {
      const int q = j / KS1, ks = j % KS1;
      f0 = (2 * q) * KS1 + ks;
      f1 = (2 * q + 1) * KS1 + ks;
      v4f d[2][2] = {};
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
          const V sel = onehot_b<DT>(wave_col<NQ>(q, h, li) - 32 * c, lg);
          d[h][0] = Ops::mfma(ra[c][0], sel, d[h][0]);
          d[h][1] = Ops::mfma(ra[c][1], sel, d[h][1]);
        }
      g0 = pack_frag<DT>(d[0][0], d[0][1]);
      g1 = pack_frag<DT>(d[1][0], d[1][1]);
    } else {
      const int s = (j - W::JR) / (MB / 2), p = (j - W::JR) % (MB / 2);
      f0 = W::NR + (2 * p) * KS2 + s;
      f1 = W::NR + (2 * p + 1) * KS2 + s;
      g0 = transpose_frag<DT>(la[0], la[1], onehot_b<DT>(li, lg));
      g1 = transpose_frag<DT>(la[0], la[1], onehot_b<DT>(16 + li, lg));
    }
    *reinterpret_cast<V*>(frag_lds + f0 * 1024 + 16 * lane) = g0;
    *reinterpret_cast<V*>(frag_lds + f1 * 1024 + 16 * lane) = g1;
  }
  lds_barrier();   // LDS only: the X loads stay in flight
  if (t >= tokens) return;
  V rf[NQ][2][KS1];
  V lf[MB][KS2];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks)
        rf[q][h][ks] = *reinterpret_cast<const V*>(frag_lds + ((2 * q + h) * KS1 + ks) * 1024 + 16 * lane);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int s = 0; s < KS2; ++s)
      lf[mb][s] = *reinterpret_cast<const V*>(frag_lds + (W::NR + mb * KS2 + s) * 1024 + 16 * lane);

  while (true) {
    // First product Z = X R, rounding point 1, accumulator -> A operand of the
    // second product: zp[q][h][s][4e + r] = Z[16(2s + e) + 4lg + r][wave_col(q, h, li)].
    V zp[NQ][2][KS2];
#pragma unroll
    for (int s = 0; s < KS2; ++s) {
      v4f acc[2][NQ][2];   // row blocks rb = 2s + e
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            acc[e][q][h] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS1; ++ks)
              acc[e][q][h] = Ops::mfma(xf[2 * s + e][ks], rf[q][h][ks], acc[e][q][h]);
          }
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v4i w = {(int)Epi::pack(acc[0][q][h][0], acc[0][q][h][1]),
                         (int)Epi::pack(acc[0][q][h][2], acc[0][q][h][3]),
                         (int)Epi::pack(acc[1][q][h][0], acc[1][q][h][1]),
                         (int)Epi::pack(acc[1][q][h][2], acc[1][q][h][3])};
          zp[q][h][s] = __builtin_bit_cast(V, w);
        }
    }

    // X is consumed: the next token's loads go into the same registers and
    // arrive while this token's second product and epilogue run.
    const int64_t tn = t + nwaves;
    if (tn < tokens) fq_wave_load_x<DT, MB, NQ>(x + tn * x_ld, xf, li, lg);

    // Second product, transposed (Y^T = Z^T L), rounding point 2. Lane (li, lg)
    // of block (mb, q) holds Y[16mb + li][8(NQ lg + q) + 4h + r]: packed word
    // NQ lg + q of row 16mb + li, nibbles r (h = 0) and r + 4 (h = 1).
    uint32_t yp[MB][NQ][4];
    typename Epi::Amax am;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS2; ++s) {
          acc0 = Ops::mfma(zp[q][0][s], lf[mb][s], acc0);
          acc1 = Ops::mfma(zp[q][1][s], lf[mb][s], acc1);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) yp[mb][q][r] = Epi::pack(acc0[r], acc1[r]);
        Epi::track2(am, yp[mb][q][0], yp[mb][q][1]);
        Epi::track2(am, yp[mb][q][2], yp[mb][q][3]);
      }
    const float amax = Epi::lo(wave_max_u32(Epi::amax_bits(am)));
    const float s = fq_scale_abs<DT>(amax, clip);
    if (lane == 0) out_scales[t] = s;

    if (PACK && s > 0.f) {
      const float rcp = 1.0f / s;
      int32_t* orow = reinterpret_cast<int32_t*>(out_codes) + t * (F / 8) + NQ * lg;
      // This wave's last token: its codes are written in the kernel's last
      // microseconds, where plain stores would leave them dirty in L2 for the
      // write-back at the kernel's end; non-temporal stores send them on
      // (2048 tokens of 64 x 64 fp16, one per wave: 8.82 -> 7.66 us, same
      // process). Earlier tokens keep plain stores, which L2 combines into
      // whole lines (non-temporal for every token: 8192 tokens 22.7 -> 23.9 us).
      const bool nt = tn >= tokens;
      // Quotients are >= -rnd(amax * rcp); below -8.5 they would need the
      // lower clamp (rne(-8.5) = -8). Uniform per token.
      if (DT::round(amax * rcp) > 8.5f)
        fq_wave_store_codes<DT, MB, NQ, true>(orow, yp, rcp, li, nt);
      else
        fq_wave_store_codes<DT, MB, NQ, false>(orow, yp, rcp, li, nt);
    } else {
      // int8 codes, and tokens whose scale rounded to 0 (the fallback's 0/0 codes)
      const float rcp = 1.0f / s;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int m = 16 * mb + li;
          int code[8];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float y0 = Epi::lo(yp[mb][q][r]), y1 = Epi::hi(yp[mb][q][r]);
            if (s > 0.f) {
              code[r] = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y0 * rcp, -8.0f, 7.0f)));
              code[4 + r] = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y1 * rcp, -8.0f, 7.0f)));
            } else {
              code[r] = fq_code_from_quot<PACK>(DT::round(opaque(y0) / s));
              code[4 + r] = fq_code_from_quot<PACK>(DT::round(opaque(y1) / s));
            }
          }
          if (PACK) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) word |= (uint32_t)(code[j] + 8) << (4 * j);
            reinterpret_cast<int32_t*>(out_codes)[t * (F / 8) + m * (N / 8) + NQ * lg + q] = (int32_t)word;
          } else {
            uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              lo4 |= (uint32_t)(code[j] & 0xFF) << (8 * j);
              hi4 |= (uint32_t)(code[4 + j] & 0xFF) << (8 * j);
            }
            v2i pair = {(int)lo4, (int)hi4};
            *reinterpret_cast<v2i*>(reinterpret_cast<int8_t*>(out_codes) + t * F + m * N + 8 * (NQ * lg + q)) =
                pair;
          }
        }
    }

    t = tn;
    if (t >= tokens) break;
  }
}

// ---------------------------------------------------------------------------
// Pair kernel (fq_duo_kernel): N = 128, M = 16*MB (MB <= 8), the wide
// transforms (e.g. 112 x 128 for 14336 features). Two waves share a token,
// one per 64-column half c; the pair is the workgroup, and it walks the
// tokens (persistent). R's fragments, Z and Y of a 64-column half take about
// 180 registers, so the waves run one per SIMD (512 registers each), two
// workgroups per CU.
//
// * X: each token's fragments arrive by LDS-DMA in A-operand order (lane l of
//   fragment (rb, ks) holds X[16rb + l%16][32ks + 8(l/16) .. +7]); the DMA of
//   the next token is issued as soon as both waves of the pair have read the
//   current one, so it overlaps the second product and the epilogue.
// * R: this wave's 64 columns as B-operand fragments in VGPRs (64 registers),
//   in the column order of the wave kernel, so each lane ends up with whole
//   adjacent code words.
// * L: B-operand fragments of the second product in LDS, built once per
//   workgroup and read by both waves of every pair.
// * Products and rounding points as in fq_wave_kernel; the second product runs
//   transposed with Z's accumulators as its A operand. When M / 16 is odd its
//   last 16 rows of k form a zero-padded 32-deep slab (elements 4..7 of both
//   operands zero; the MFMA's sum is unchanged), not a 16x16x16 MFMA, whose
//   results here came out wrong on gfx950. max |Y| of the raw
//   accumulators (rounding is monotonic and symmetric) is combined across the
//   pair through LDS, then the scale, codes and packing of fq_wave_kernel.
// ---------------------------------------------------------------------------
template <int MB>
struct DuoShape {
  static constexpr int M = 16 * MB, N = 128, F = M * N;
  static constexpr int KS1 = N / 32;           // 32-deep slabs of the first product (k = n')
  static constexpr int KS2 = MB / 2;           // full 32-deep slabs of the second (k = m')
  static constexpr bool TAIL = (MB & 1) != 0;  // one 16-deep slab when M / 16 is odd
  static constexpr int XF = MB * KS1;          // 1 KiB X fragments per token
  static constexpr int X_BYTES = XF * 1024;    // one X buffer
  static constexpr int KSL = KS2 + (TAIL ? 1 : 0);   // slabs incl. the zero-padded tail
  static constexpr int LF_BYTES = MB * KSL * 1024;     // L fragments
  static constexpr int SLOTS = 2;              // token pairs per workgroup (four waves)
  // X buffers per slot: two (the next-but-one token's X is copied while this
  // one is processed) where the LDS holds them, else one
  static constexpr int XB = SLOTS * 2 * X_BYTES + LF_BYTES + 64 <= 160 * 1024 ? 2 : 1;
  static constexpr int XAREA = SLOTS * XB * X_BYTES;   // buffer b of slot p at (b SLOTS + p) X_BYTES
  static constexpr int STAGE_BYTES = N * N * 2 + M * M * 2;   // R and L rows during the set-up
  // EARLY: the set-up stages R and L behind the slots' first X buffers, so the
  // first tokens' copies are issued before the set-up instead of after it
  // (worth a global round trip when each slot has one or two tokens), where
  // the LDS holds that layout; otherwise the staging reuses the X area.
  static constexpr int EARLY_LF_OFF =
      (SLOTS * X_BYTES + STAGE_BYTES > XAREA ? SLOTS * X_BYTES + STAGE_BYTES : XAREA);
  static constexpr bool EARLY = EARLY_LF_OFF + LF_BYTES + 64 <= 160 * 1024;
  static constexpr int STAGE_OFF = EARLY ? SLOTS * X_BYTES : 0;
  static constexpr int LF_OFF = EARLY ? EARLY_LF_OFF : XAREA;
  static constexpr int LDS_BYTES = LF_OFF + LF_BYTES;
  static_assert(STAGE_OFF + STAGE_BYTES <= LF_OFF, "R and L staging space");
  static_assert(MB >= 2 && MB <= 8, "M = 32 .. 128");
  static_assert(XF % 2 == 0, "X fragments split over the pair");
};

template <class DT, int MB, bool PACK>
__global__ void __launch_bounds__(128 * DuoShape<MB>::SLOTS) __attribute__((amdgpu_waves_per_eu(1, 1)))
fq_duo_kernel(const typename DT::T* __restrict__ x, int64_t tokens, int64_t x_ld,
              const typename DT::T* __restrict__ left, const typename DT::T* __restrict__ right, float clip,
              void* __restrict__ out_codes, float* __restrict__ out_scales) {
  using S = DuoShape<MB>;
  using T = typename DT::T;
  using Ops = MfmaOps<DT>;
  using V = typename Ops::V;
  using Epi = FqEpi<DT>;
  constexpr int M = S::M, N = S::N, F = S::F, KS1 = S::KS1, KS2 = S::KS2, XB = S::XB, SLOTS = S::SLOTS;
  // one LDS block: the X buffers, then the L fragments (the set-up stages R
  // across both)
  __shared__ __align__(16) unsigned char lds_all[S::LDS_BYTES];
  __shared__ float red[SLOTS][2];
  unsigned char* const lfs = lds_all + S::LF_OFF;

  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = wave >> 1, c = wave & 1;   // token slot, column half
  auto xbuf = [&](int b) { return lds_all + (b * SLOTS + p) * S::X_BYTES; };
  // token of this wave's slot in iteration it
  const int64_t step = (int64_t)gridDim.x * SLOTS;
  const int64_t t0 = (int64_t)blockIdx.x * SLOTS + p;

  // LDS-DMA of token tt's X into buffer b of this slot: this wave copies
  // fragments c, c + 2, c + 4, ... (lane l of fragment (rb, ks) holds
  // X[16rb + l%16][32ks + 8(l/16) .. +7]). Tokens past the last re-read a valid
  // row and store nothing.
  auto issue_x = [&](int64_t tt, int b) {
    tt = tt < tokens ? tt : tokens - 1;
    const T* base = x + tt * x_ld + li * N + 8 * lg;
    const uint32_t lbase = lds_addr(xbuf(b));
#pragma unroll
    for (int i = 0; i < S::XF / 2; ++i) {
      const int f = c + 2 * i;
      dma16(base + (f / KS1) * 16 * N + 32 * (f % KS1), lbase + f * 1024);
    }
  };

  // Set-up, once per workgroup. R and L are copied row-major into LDS by
  // LDS-DMA (coalesced 16-byte chunks; R, then L after it, one round trip for
  // both), then rearranged from LDS: R into this wave's registers, L into the
  // L fragments. With EARLY the first token's X copy of each slot follows the
  // staging copies, and the wait leaves it in flight.
  unsigned char* const stage = lds_all + S::STAGE_OFF;
  {
    const uint32_t lb = lds_addr(stage);
    auto stage_rows = [&](const T* src, int chunks, uint32_t base) {   // chunk c (8 elements) -> base + 16 c
#pragma unroll 1
      for (int c0 = wave * 64; c0 < chunks; c0 += 64 * 2 * SLOTS)
        if (c0 + lane < chunks) dma16(src + 8 * (c0 + lane), base + 16 * c0);
    };
    stage_rows(right, N * N / 8, lb);
    stage_rows(left, M * M / 8, lb + N * N * 2);
    if constexpr (S::EARLY) {
      issue_x(t0, 0);
      wait_vmcnt<S::XF / 2>();   // the staging copies (older) have landed
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
  }
  // Both gathers below read 4 consecutive rows of one column per lane with
  // the LDS transpose read (lds_tr16): lane l of a 16-lane group supplies the
  // address of row k0 + l/4, columns C(l%4) .. C(l%4) + 3, and receives rows
  // k0 .. k0 + 3 of column C(l/4) + l%4.
  // R fragments of this wave's columns: rf[q][h][ks][j] = R[32ks + 8lg + j][n],
  // n = 64c + 16(li/4) + 8q + 4h + li%4, i.e. C(x) = 64c + 16x + 8q + 4h.
  V rf[2][2][KS1];
  {
    const T* rs = reinterpret_cast<const T*>(stage);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < KS1; ++ks) {
          const T* at = rs + (32 * ks + 8 * lg + (li >> 2)) * N + 64 * c + 16 * (li & 3) + 8 * q + 4 * h;
          rf[q][h][ks] = join_tr16<V>(lds_tr16(at), lds_tr16(at + 4 * N));
        }
  }
  // L fragments (16 bytes per lane and slab): slab (mb, s), lane l, element j
  // holds L[32s + 16(j/4) + 4(l/16) + j%4][16mb + l%16] (C(x) = 16mb + 4x); in
  // the zero-padded tail slab (s = KS2, M / 16 odd) elements 4..7 are zero.
  {
    const T* ls = reinterpret_cast<const T*>(stage + N * N * 2);
#pragma unroll 1
    for (int fr = wave; fr < MB * S::KSL; fr += 2 * SLOTS) {
      const int mb = fr / S::KSL, sl = fr % S::KSL;
      const T* at = ls + (32 * sl + 4 * lg + (li >> 2)) * M + 16 * mb + 4 * (li & 3);
      const v4s16 lo = lds_tr16(at);
      const v4s16 hi = sl == KS2 ? v4s16{0, 0, 0, 0} : lds_tr16(at + 16 * M);
      *reinterpret_cast<V*>(lfs + fr * 1024 + 16 * lane) = join_tr16<V>(lo, hi);
    }
  }
  lds_barrier();   // R in registers, L fragments written: the staging space is free
#pragma unroll
  for (int b = S::EARLY ? 1 : 0; b < XB; ++b) issue_x(t0 + b * step, b);

  for (int64_t it = 0; t0 - p + it * step < tokens; ++it) {
    const int64_t t = t0 + it * step;
    const int b = XB == 2 ? (int)(it & 1) : 0;
    unsigned char* const xb = xbuf(b);
    // This iteration's copy is older than the copies issued in the last
    // XB - 1 iterations. The output stores issued in between are not counted:
    // a store may complete out of order with the copies, and counting it
    // could end the wait before this copy landed.
    wait_vmcnt<(XB - 1) * (S::XF / 2)>();
    lds_barrier();   // the slot's X (and, the first time, the L fragments) visible

    // First product Z = X R for this wave's 64 columns, rounding point 1, the
    // accumulators packed as A operands of the second product:
    //   zp[q][h][s][4e + r] = Z[16(2s + e) + 4lg + r][n(q, h, li)].
    V zp[2][2][S::KSL];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
      V a[KS1];
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) a[ks] = *reinterpret_cast<const V*>(xb + (rb * KS1 + ks) * 1024 + 16 * lane);
      v4f acc[2][2];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[q][h] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS1; ++ks) acc[q][h] = Ops::mfma(a[ks], rf[q][h][ks], acc[q][h]);
        }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            zp[q][h][rb >> 1][(rb & 1) * 4 + r] = (T)acc[q][h][r];   // an MFMA result: no opaque()
            if (S::TAIL && rb == MB - 1) zp[q][h][rb >> 1][4 + r] = __builtin_bit_cast(T, (short)0);
          }
    }
    lds_barrier();                     // both waves of each pair are done with buffer b
    issue_x(t + XB * step, b);         // the token XB iterations ahead

    // Second product, transposed, rounding point 2. Lane (li, lg) of block
    // (mb, q) holds Y[16mb + li][64c + 8(2lg + q) + 4h + r]: packed word
    // 8c + 2lg + q of row 16mb + li, nibbles r (h = 0) and r + 4 (h = 1).
    uint32_t yp[MB][2][4];
    float amax = 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      V lf[S::KSL];
#pragma unroll
      for (int sl = 0; sl < S::KSL; ++sl) lf[sl] = *reinterpret_cast<const V*>(lfs + (mb * S::KSL + sl) * 1024 + 16 * lane);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        v4f acc[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[h] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sl = 0; sl < S::KSL; ++sl) acc[h] = Ops::mfma(zp[q][h][sl], lf[sl], acc[h]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          yp[mb][q][r] = Epi::pack_acc(acc[0][r], acc[1][r]);
          amax = fmaxf(fmaxf(amax, fabsf(acc[0][r])), fabsf(acc[1][r]));
        }
      }
    }
    // max |y| over the token: the wave, then the pair (non-negative floats
    // order like their bit patterns)
    amax = __builtin_bit_cast(float, wave_max_u32(__builtin_bit_cast(uint32_t, amax)));
    if (lane == 0) red[p][c] = amax;
    lds_barrier();
    amax = DT::round(fmaxf(red[p][0], red[p][1]));
    const float s = fq_scale_abs<DT>(amax, clip);

    if (t < tokens) {
      if (c == 0 && lane == 0) out_scales[t] = s;
      const float rcp = 1.0f / s;
      if (PACK) {
        int32_t* orow = reinterpret_cast<int32_t*>(out_codes) + t * (F / 8) + 8 * c + 2 * lg;
        if (s > 0.f) {
          if constexpr (std::is_same<DT, BF16T>::value) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              *reinterpret_cast<v2i*>(orow + (16 * mb + li) * (N / 8)) =
                  v2i{(int)Epi::word_u8(yp[mb][0], rcp), (int)Epi::word_u8(yp[mb][1], rcp)};
          } else if (DT::round(amax * rcp) > 8.5f) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              *reinterpret_cast<v2i*>(orow + (16 * mb + li) * (N / 8)) =
                  v2i{(int)Epi::template word4<true>(yp[mb][0], rcp), (int)Epi::template word4<true>(yp[mb][1], rcp)};
          } else {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              *reinterpret_cast<v2i*>(orow + (16 * mb + li) * (N / 8)) =
                  v2i{(int)Epi::template word4<false>(yp[mb][0], rcp), (int)Epi::template word4<false>(yp[mb][1], rcp)};
          }
        } else {
          // scale rounded to 0 (an all-zero fp16 token): the fallback's 0/0 codes
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            uint32_t w[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              w[q] = 0;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                w[q] |= (uint32_t)(fq_code_from_quot<true>(DT::round(opaque(Epi::lo(yp[mb][q][r])) / s)) + 8) << (4 * r);
                w[q] |= (uint32_t)(fq_code_from_quot<true>(DT::round(opaque(Epi::hi(yp[mb][q][r])) / s)) + 8)
                        << (4 * r + 16);
              }
            }
            *reinterpret_cast<v2i*>(orow + (16 * mb + li) * (N / 8)) = v2i{(int)w[0], (int)w[1]};
          }
        }
      } else {
        // int8 codes: 16 bytes per row block (words 8c + 2lg and + 1)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          uint32_t lo4[2], hi4[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            lo4[q] = hi4[q] = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float y0 = Epi::lo(yp[mb][q][r]), y1 = Epi::hi(yp[mb][q][r]);
              int c0, c1;
              if (s > 0.f) {
                c0 = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y0 * rcp, -8.0f, 7.0f)));
                c1 = (int)__builtin_rintf(DT::round(__builtin_amdgcn_fmed3f(y1 * rcp, -8.0f, 7.0f)));
              } else {
                c0 = fq_code_from_quot<false>(DT::round(opaque(y0) / s));
                c1 = fq_code_from_quot<false>(DT::round(opaque(y1) / s));
              }
              lo4[q] |= (uint32_t)(c0 & 0xFF) << (8 * r);
              hi4[q] |= (uint32_t)(c1 & 0xFF) << (8 * r);
            }
          }
          *reinterpret_cast<v4i*>(reinterpret_cast<int8_t*>(out_codes) + t * F + (16 * mb + li) * N +
                                  8 * (8 * c + 2 * lg)) = v4i{(int)lo4[0], (int)hi4[0], (int)lo4[1], (int)hi4[1]};
        }
      }
    }
  }
  wait_vmcnt<0>();   // no LDS-DMA may still be writing when the workgroup retires
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------

template <class DT, int MB, int NP, bool PACK, int NV = 32 * NP, int MV = 16 * MB>
static int launch_mfma(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right,
                       float clip, void* out_codes, float* out_scales, hipStream_t stream) {
  using S = FqShape<MB, NP, NV, MV>;
  using T = typename DT::T;
  // static LDS of the kernel (X stages; L's fragments counted where one stage is used)
  constexpr size_t lds = S::ONE_STAGE ? S::STAGE_ELEMS * sizeof(T) + S::LF_BYTES : 2 * S::STAGE_ELEMS * sizeof(T);
  const int per_cu = (int)std::min<size_t>(4, (160 * 1024) / (lds + 256));
  const int64_t ngroups = (tokens + S::TPB - 1) / S::TPB;
  int64_t grid = (int64_t)device_cu_count() * per_cu;
  if (grid > ngroups) grid = ngroups;
  launch((fq_mfma_kernel<DT, MB, NP, PACK, NV, MV>), dim3((unsigned)grid), dim3(S::WAVES * 64), 0, stream,
                     reinterpret_cast<const T*>(x), tokens, x_ld, reinterpret_cast<const T*>(left),
                     reinterpret_cast<const T*>(right), clip, out_codes, out_scales);
  return QO_OK;
}

template <class DT, int MB, int NQ, bool PACK>
static int launch_wave(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right,
                       float clip, void* out_codes, float* out_scales, hipStream_t stream) {
  using T = typename DT::T;
  // one token per wave, up to two workgroups per CU; beyond that waves loop
  const int64_t grid = std::min<int64_t>((tokens + kWaveKernelWaves - 1) / kWaveKernelWaves,
                                         (int64_t)device_cu_count() * 2);
  launch((fq_wave_kernel<DT, MB, NQ, PACK>), dim3((unsigned)grid), dim3(64 * kWaveKernelWaves), 0,
                     stream,
                     reinterpret_cast<const T*>(x), tokens, x_ld, reinterpret_cast<const T*>(left),
                     reinterpret_cast<const T*>(right), clip, out_codes, out_scales);
  return QO_OK;
}

// N = 128 shapes take the few-token routine at every token count. Measured
// (8192 tokens bf16 unless noted; same process, outputs equal):
// * 112 x 128 and 64 x 128 run fq_few2_kernel (two workgroups per CU):
//   112 x 128 82.8-84.4 us against 89.9-90.2 with fq_few_kernel's one slot
//   (4096 tokens 44.6 vs 48.1, 1024 tokens 16.8 vs 17.3, 16 tokens 6.41 vs
//   6.46; fp16 88.3 vs 89.0); 64 x 128 44.8 us against 49.3 on the pair
//   kernel.
// * 96 x 128 keeps two tokens in flight per workgroup above kFewTwoSlots
//   tokens per CU (72.8 us with two slots vs 75.7 with one, 73.4 compact).
// * 128 x 128 stays on one slot (its compact form spills).
constexpr int64_t kFewTwoSlots = 2;

// bf16 codes need no upper clamp when clip >= kNoClampClip. With c the clip
// ratio and every rounding's relative error bounded (2^-8 for bf16, 2^-24 for
// float32): bound = rnd(amax c) >= amax c (1 - 2^-24)(1 - 2^-8), s = rnd(bound
// / 7) >= bound / 7 (1 - 2^-24)(1 - 2^-8), rcp <= (1 + 2^-24) / s, so the
// largest quotient u = fl(amax rcp) <= 7 (1 + 2^-24)^2 / (c (1 - 2^-24)^2
// (1 - 2^-8)^2), which is below 7.484375 (the least float32 that rounds to
// bf16 7.5 or above) for c > 0.9427. The clamp of the scale at rnd(1e-8)
// only makes s larger. No lower clamp is needed either: |y| <= amax and both
// roundings are sign-symmetric, so the smallest quotient is above -7.5.
constexpr float kNoClampClip = 0.95f;

template <class DT, int MB, bool PACK>
static int launch_few(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right, float clip,
                      void* out_codes, float* out_scales, hipStream_t stream, const ReadAhead& ra) {
  using T = typename DT::T;
  const int64_t cus = device_cu_count();
  if constexpr (MB == 6) {
    if (tokens > kFewTwoSlots * cus) {
      // two tokens at a time per workgroup (eight waves, two per SIMD), one workgroup per CU
      const int64_t grid = std::min<int64_t>((tokens + 1) / 2, cus);
      launch((fq_few_kernel<DT, MB, PACK, 2>), dim3((unsigned)grid), dim3(512), 0, stream,
             reinterpret_cast<const T*>(x), tokens, x_ld, reinterpret_cast<const T*>(left),
             reinterpret_cast<const T*>(right), clip, out_codes, out_scales);
      return QO_OK;
    }
  }
  if constexpr (MB == 7 || MB == 4) {
    // one token at a time per workgroup, two workgroups per CU (two waves per SIMD);
    // a read-ahead request takes the workgroup slots the tokens leave free
    const int64_t grid = std::min<int64_t>(tokens, 2 * cus);
    const bool ahead = ra.p && ra.rows > 0 && ra.row_len >= 16 && (uintptr_t)ra.p % 16 == 0 &&
                       ra.row_bytes % 16 == 0 && ra.row_len % 16 == 0 && ra.row_len <= ra.row_bytes &&
                       (ra.rows + 256) * (ra.row_len / 16) < INT32_MAX / 2 && grid < 2 * cus;
    auto go = [&](auto kernel) {
      launch(kernel, dim3((unsigned)(ahead ? 2 * cus : grid)), dim3(256), 0, stream, reinterpret_cast<const T*>(x),
             tokens, x_ld, reinterpret_cast<const T*>(left), reinterpret_cast<const T*>(right), clip, out_codes,
             out_scales, (int)grid, reinterpret_cast<const v4i*>(ra.p), ahead ? ra.rows : (int64_t)0,
             ra.row_bytes / 16, ahead ? (int)(ra.row_len / 16) : 0);
    };
    if constexpr (std::is_same<DT, BF16T>::value && PACK) {
      // staged code stores need 16-byte pieces of the codes
      const bool stage = (uintptr_t)out_codes % 16 == 0;
      if (clip >= kNoClampClip) {
        if (stage) go(fq_few2_kernel<DT, MB, PACK, true, true>);
        else go(fq_few2_kernel<DT, MB, PACK, true>);
      } else {
        if (stage) go(fq_few2_kernel<DT, MB, PACK, false, true>);
        else go(fq_few2_kernel<DT, MB, PACK>);
      }
      return QO_OK;
    }
    go(fq_few2_kernel<DT, MB, PACK>);
    return QO_OK;
  }
  // one token at a time per workgroup (four waves, one per SIMD); workgroups loop beyond one per CU
  const int64_t grid = std::min<int64_t>(tokens, cus);
  launch((fq_few_kernel<DT, MB, PACK, 1>), dim3((unsigned)grid), dim3(256), 0, stream, reinterpret_cast<const T*>(x),
         tokens, x_ld, reinterpret_cast<const T*>(left), reinterpret_cast<const T*>(right), clip, out_codes,
         out_scales);
  return QO_OK;
}

template <class DT, int MB, bool PACK>
static int launch_duo(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right, float clip,
                      void* out_codes, float* out_scales, hipStream_t stream) {
  using T = typename DT::T;
  constexpr int SLOTS = DuoShape<MB>::SLOTS;
  // one workgroup (four waves, one per SIMD) per CU
  const int64_t grid = std::min<int64_t>((tokens + SLOTS - 1) / SLOTS, (int64_t)device_cu_count());
  launch((fq_duo_kernel<DT, MB, PACK>), dim3((unsigned)grid), dim3(128 * SLOTS), 0, stream,
                     reinterpret_cast<const T*>(x), tokens, x_ld, reinterpret_cast<const T*>(left),
                     reinterpret_cast<const T*>(right), clip, out_codes, out_scales);
  return QO_OK;
}

// QO_ROUTE_FQ_NO_DUO keeps N = 128 shapes on fq_mfma_kernel (tests use it to
// cross-check the two).
static bool fq_allow_duo() {
  return !route_off(QO_ROUTE_FQ_NO_DUO);
}

// QO_ROUTE_FQ_NO_WAVE keeps small shapes on fq_mfma_kernel (tests use it to
// cross-check the two MFMA kernels).
static bool fq_allow_wave() {
  return !route_off(QO_ROUTE_FQ_NO_WAVE);
}

// QO_ROUTE_FQ_NO_FEW keeps the one-wave and pair kernels at any token count
// (tests use it to cross-check them against the workgroup kernel on small
// inputs).

static bool fq_route_few() {
  return !route_off(QO_ROUTE_FQ_NO_FEW);
}

template <class DT, bool PACK>
static int dispatch_mfma(int M, int N, const void* x, int64_t tokens, int64_t x_ld, const void* left,
                         const void* right, float clip, void* out_codes, float* out_scales,
                         hipStream_t stream, bool* handled, const ReadAhead& ra) {
  *handled = true;
  // Up to a few hundred tokens the workgroup kernel (fq_mfma_kernel, one
  // token per group of 2-4 waves) finishes sooner than the one-wave and pair
  // kernels, whose per-token chain is longer; measured crossovers: 64 x 64
  // after 512 tokens (16 tokens bf16: 5.2 vs 6.4 us), 32 x 64 and 64 x 128
  // after 256; 96 x 128 at up to 256 tokens too (1 token bf16: 6.8 vs 7.7 us).
  // 112 x 128 and 128 x 128 keep the pair kernel at any count.
  const bool few = fq_route_few() && tokens <= (M == 64 && N == 64 ? 512 : 256);
  // the wave kernel takes the scale from max |Y|, which needs clip > 0
  if (fq_allow_wave() && clip > 0.f && clip <= 3.4e38f && !few) {
#define QO_FQ_WAVE_CASE(MB_, NQ_)                                                                    \
    if (M == 16 * (MB_) && N == 32 * (NQ_))                                                          \
      return launch_wave<DT, MB_, NQ_, PACK>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, \
                                             stream);
    QO_FQ_WAVE_CASE(4, 2)   // 64 x 64 (hidden 4096)
    QO_FQ_WAVE_CASE(2, 2)   // 32 x 64 (hidden 2048)
    QO_FQ_WAVE_CASE(2, 1)   // 32 x 32 (hidden 1024)
    QO_FQ_WAVE_CASE(4, 1)   // 64 x 32 (hidden 2048)
#undef QO_FQ_WAVE_CASE
  }
  // N = 128 at decode token counts: the few-token kernel (scale from max |Y| as well)
  if (N == 128 && clip > 0.f && clip <= 3.4e38f && fq_route_few()) {
#define QO_FQ_FEW_CASE(MB_)                                                                                  \
    if (M == 16 * (MB_))                                                                                     \
      return launch_few<DT, MB_, PACK>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, stream, ra);
    QO_FQ_FEW_CASE(7)   // 112 x 128 (hidden 14336)
    QO_FQ_FEW_CASE(4)   // 64 x 128  (hidden 8192)
    QO_FQ_FEW_CASE(8)   // 128 x 128 (hidden 16384)
    QO_FQ_FEW_CASE(6)   // 96 x 128  (hidden 12288)
#undef QO_FQ_FEW_CASE
  }
  // the pair kernel takes its scale from max |Y| as well
  if (fq_allow_duo() && clip > 0.f && clip <= 3.4e38f && N == 128 && !(few && (M == 64 || M == 96))) {
#define QO_FQ_DUO_CASE(MB_)                                                                                  \
    if (M == 16 * (MB_))                                                                                     \
      return launch_duo<DT, MB_, PACK>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, stream);
    QO_FQ_DUO_CASE(7)   // 112 x 128 (hidden 14336)
    QO_FQ_DUO_CASE(4)   // 64 x 128  (hidden 8192)
    QO_FQ_DUO_CASE(8)   // 128 x 128 (hidden 16384)
    QO_FQ_DUO_CASE(6)   // 96 x 128  (hidden 12288)
#undef QO_FQ_DUO_CASE
  }
#define QO_FQ_CASE(MB_, NP_)                                                                      \
  if (M == 16 * (MB_) && N == 32 * (NP_))                                                         \
    return launch_mfma<DT, MB_, NP_, PACK>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, \
                                           stream);
  QO_FQ_CASE(4, 2)   // 64 x 64    (hidden 4096)
  QO_FQ_CASE(7, 4)   // 112 x 128  (hidden 14336)
  QO_FQ_CASE(2, 2)   // 32 x 64    (hidden 2048)
  QO_FQ_CASE(4, 4)   // 64 x 128   (hidden 8192)
  QO_FQ_CASE(8, 4)   // 128 x 128  (hidden 16384)
  QO_FQ_CASE(2, 1)   // 32 x 32    (hidden 1024)
  QO_FQ_CASE(3, 2)   // 48 x 64    (hidden 3072)
  QO_FQ_CASE(5, 2)   // 80 x 64
  QO_FQ_CASE(6, 4)   // 96 x 128   (hidden 12288)
  QO_FQ_CASE(4, 3)   // 64 x 96    (hidden 6144)
  QO_FQ_CASE(5, 4)   // 80 x 128   (hidden 10240)
  QO_FQ_CASE(8, 5)   // 128 x 160  (hidden 20480)
  QO_FQ_CASE(8, 6)   // 128 x 192  (hidden 24576)
  QO_FQ_CASE(8, 7)   // 128 x 224  (hidden 28672)
  QO_FQ_CASE(9, 6)   // 144 x 192  (hidden 27648)
  QO_FQ_CASE(10, 5)  // 160 x 160  (hidden 25600)
  QO_FQ_CASE(8, 8)   // 128 x 256  (hidden 32768; one X stage)
#undef QO_FQ_CASE
  // widths that are not a multiple of 32: computed zero-padded to 32 NP
#define QO_FQ_CASE_NV(MB_, NP_, NV_)                                                                     \
  if (M == 16 * (MB_) && N == (NV_))                                                                     \
    return launch_mfma<DT, MB_, NP_, PACK, NV_>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, \
                                                stream);
  QO_FQ_CASE_NV(4, 3, 80)    // 64 x 80   (hidden 5120)
  QO_FQ_CASE_NV(4, 4, 112)   // 64 x 112  (hidden 7168)
  QO_FQ_CASE_NV(8, 5, 144)   // 128 x 144 (hidden 18432)
  QO_FQ_CASE_NV(2, 2, 48)    // 32 x 48   (hidden 1536)
  QO_FQ_CASE_NV(4, 3, 88)    // 64 x 88   (hidden 5632)
  QO_FQ_CASE_NV(5, 4, 112)   // 80 x 112  (hidden 8960)
  QO_FQ_CASE_NV(8, 5, 148)   // 128 x 148 (hidden 18944; 16-bit code halves)
  QO_FQ_CASE_NV(8, 6, 172)   // 128 x 172 (hidden 22016; 16-bit code halves)
  QO_FQ_CASE_NV(4, 7, 214)   // 64 x 214  (hidden 13696; byte code stores)
#undef QO_FQ_CASE_NV
  // heights that are not a multiple of 16: computed zero-padded to 16 MB
#define QO_FQ_CASE_MV(MB_, NP_, MV_)                                                                          \
  if (M == (MV_) && N == 32 * (NP_))                                                                          \
    return launch_mfma<DT, MB_, NP_, PACK, 32 * (NP_), MV_>(x, tokens, x_ld, left, right, clip, out_codes,    \
                                                            out_scales, stream);
  QO_FQ_CASE_MV(4, 2, 56)    // 56 x 64   (hidden 3584)
  QO_FQ_CASE_MV(6, 4, 86)    // 86 x 128  (hidden 11008)
  QO_FQ_CASE_MV(7, 4, 108)   // 108 x 128 (hidden 13824)
  QO_FQ_CASE_MV(3, 2, 40)    // 40 x 64   (hidden 2560)
  QO_FQ_CASE_MV(5, 3, 72)    // 72 x 96   (hidden 6912)
  QO_FQ_CASE_MV(5, 4, 76)    // 76 x 128  (hidden 9728)
  // both padded, one X stage
  if (M == 168 && N == 176)   // 168 x 176 (hidden 29568)
    return launch_mfma<DT, 11, 6, PACK, 176, 168>(x, tokens, x_ld, left, right, clip, out_codes, out_scales, stream);
#undef QO_FQ_CASE_MV
  *handled = false;
  return QO_OK;
}

template <class DT, bool PACK>
static int launch_generic(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right,
                          int M, int N, float clip, void* out_codes, float* out_scales, hipStream_t stream) {
  using T = typename DT::T;
  size_t lds = (size_t)2 * M * N * sizeof(T);
  constexpr size_t kMaxDynLds = 160 * 1024 - 64;   // the static reduction slots take the rest
  if (lds > kMaxDynLds) {
    // X and Z do not fit together: Y by column blocks, twice per token
    const size_t zb = (size_t)M * kBigCols * sizeof(float);
    auto big = fq_generic_big_kernel<DT, PACK>;
    if (zb > kMaxDynLds ||
        (zb > 64 * 1024 &&
         hipFuncSetAttribute((const void*)big, hipFuncAttributeMaxDynamicSharedMemorySize, (int)zb) != hipSuccess)) {
      qo_set_error("qo_flatquant_quantize: M=%d needs %zu bytes of LDS for a Z column block", M, zb);
      return QO_ERR_UNSUPPORTED;
    }
    int64_t grid = (int64_t)device_cu_count() * 4;
    if (grid > tokens) grid = tokens;
    launch(big, dim3((unsigned)grid), dim3(256), zb, stream, reinterpret_cast<const T*>(x), tokens, x_ld,
           reinterpret_cast<const T*>(left), reinterpret_cast<const T*>(right), M, N, clip, out_codes, out_scales);
    return QO_OK;
  }
  // L and R in LDS too where they fit; fewer tokens than CUs: 512 threads per
  // token (two waves per SIMD, half the products each)
  const size_t lds_lr = lds + ((size_t)M * M + (size_t)N * N) * sizeof(T);
  const bool lr = lds_lr <= kMaxDynLds;
  const int cus = device_cu_count();
  const bool wide = tokens < cus;
  auto kern = wide ? (lr ? fq_generic_kernel<DT, PACK, true, 512, 2> : fq_generic_kernel<DT, PACK, false, 512, 2>)
                   : (lr ? fq_generic_kernel<DT, PACK, true, 256, 4> : fq_generic_kernel<DT, PACK, false, 256, 4>);
  if (lr) lds = lds_lr;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
        hipSuccess) {
      qo_set_error("qo_flatquant_quantize: M*N=%d needs %zu bytes of LDS", M * N, lds);
      return QO_ERR_UNSUPPORTED;
    }
  }
  int64_t grid = (int64_t)cus * 4;
  if (grid > tokens) grid = tokens;
  launch(kern, dim3((unsigned)grid), dim3(wide ? 512 : 256), lds, stream, reinterpret_cast<const T*>(x), tokens,
                     x_ld, reinterpret_cast<const T*>(left), reinterpret_cast<const T*>(right), M, N, clip,
                     out_codes, out_scales);
  return QO_OK;
}

template <class DT, bool PACK>
static int run_quantize(const void* x, int64_t tokens, int64_t x_ld, const void* left, const void* right, int M,
                        int N, float clip, void* out_codes, float* out_scales, hipStream_t stream,
                        bool allow_mfma, const ReadAhead& ra) {
  if constexpr (DT::code != QO_DTYPE_F32) {
    // 16-byte vector loads of X rows and of L / R rows, vector stores of codes
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((x_ld * (int64_t)sizeof(typename DT::T)) % 16 == 0) &&
                         ((uintptr_t)left % 16 == 0) && ((uintptr_t)right % 16 == 0) &&
                         ((uintptr_t)out_codes % 16 == 0) && ((uintptr_t)out_scales % 4 == 0);
    if (allow_mfma && aligned) {
      bool handled = false;
      int st = dispatch_mfma<DT, PACK>(M, N, x, tokens, x_ld, left, right, clip, out_codes, out_scales, stream,
                                       &handled, ra);
      if (handled) return st;
    }
  }
  return launch_generic<DT, PACK>(x, tokens, x_ld, left, right, M, N, clip, out_codes, out_scales, stream);
}

}  // namespace qo

// Selects the kernel family; QO_ROUTE_FQ_GENERIC routes every shape through
// the generic kernel (tests use it to cross-check the two).
static bool fq_allow_mfma() {
  return !qo::route_off(QO_ROUTE_FQ_GENERIC);
}

int qo::flatquant_quantize(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                           const void* right, int M, int N, float clip_ratio, int pack_int32, void* out_codes,
                           float* out_scales, void* stream, const ReadAhead& ra) {
  using namespace qo;
  if (tokens < 0 || M < 1 || N < 1) {
    qo_set_error("qo_flatquant_quantize: invalid sizes tokens=%lld M=%d N=%d", (long long)tokens, M, N);
    return QO_ERR_SHAPE;
  }
  if (pack_int32 && ((int64_t)M * N) % 8 != 0) {
    qo_set_error("qo_flatquant_quantize: features (%lld) must be divisible by 8 for int32 packing",
                 (long long)M * N);
    return QO_ERR_SHAPE;
  }
  if (x_ld < (int64_t)M * N) {
    qo_set_error("qo_flatquant_quantize: row stride %lld < features %lld", (long long)x_ld, (long long)M * N);
    return QO_ERR_SHAPE;
  }
  if (tokens == 0) return QO_OK;
  if (!x || !left || !right || !out_codes || !out_scales) {
    qo_set_error("qo_flatquant_quantize: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool mf = fq_allow_mfma();
  launch_begin();
  int st;
  switch (x_dtype) {
    case QO_DTYPE_F32:
      st = pack_int32 ? run_quantize<F32T, true>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                  out_scales, s, mf, ra)
                      : run_quantize<F32T, false>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                   out_scales, s, mf, ra);
      break;
    case QO_DTYPE_F16:
      st = pack_int32 ? run_quantize<F16T, true>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                  out_scales, s, mf, ra)
                      : run_quantize<F16T, false>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                   out_scales, s, mf, ra);
      break;
    case QO_DTYPE_BF16:
      st = pack_int32 ? run_quantize<BF16T, true>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                   out_scales, s, mf, ra)
                      : run_quantize<BF16T, false>(x, tokens, x_ld, left, right, M, N, clip_ratio, out_codes,
                                                    out_scales, s, mf, ra);
      break;
    default:
      qo_set_error("qo_flatquant_quantize: unsupported input dtype code %d", x_dtype);
      return QO_ERR_DTYPE;
  }
  const int lst = launch_result("qo_flatquant_quantize");
  return st != QO_OK ? st : lst;
}

extern "C" int qo_flatquant_quantize(const void* x, int x_dtype, int64_t tokens, int64_t x_ld, const void* left,
                                     const void* right, int M, int N, float clip_ratio, int pack_int32,
                                     void* out_codes, float* out_scales, void* stream) {
  return qo::flatquant_quantize(x, x_dtype, tokens, x_ld, left, right, M, N, clip_ratio, pack_int32, out_codes,
                                out_scales, stream, qo::ReadAhead{});
}
