// W4A4 GEMM for gfx950 (MI355X): packed int4 x packed int4 -> int32 -> scaled fp.
//
// out[m, n] = rnd_out((float(acc) * scale_a[m]) * scale_b[n]), acc = sum_k qa[m,k] qb[k,n]
// exactly. Replaces the reference's dp4a kernel (int4_matmul/kernels/
// cuda_int4_matmul_kernel.cu:49-189); numerics are those of its fallback
// int4_matmul_pytorch (int4_matmul/ops.py:69-103): the float32 matmul of
// integers is exact, then two separate float32 products, then one rounding.
//
// Fast kernel (gemm_i4_mfma): gfx950 has no int4 MFMA, so nibbles are widened
// to int8 on the way from registers into LDS and fed to
// v_mfma_i32_16x16x64_i8. Widening trick: XOR with 0x8 turns the offset code
// (q + 8) into q's 4-bit two's-complement pattern; placing it in the high half
// of a byte gives the int8 value 16*q. Both operands carry the factor 16, so the
// accumulator holds 256*acc, exact while 256 * 64 * K < 2^31 (K <= 65536); the
// epilogue shifts it back. Each packed word gives a "low" dword (nibbles
// 0,2,4,6) and a "high" dword (nibbles 1,3,5,7); A and B use the same k order.
//
// Generic kernel (gemm_i4_generic): one output per thread, any strides and
// sizes (K < 2^21). Used when the fast kernel's layout / alignment
// requirements are not met.
#include "common.h"

#ifndef QO_GEMM_TILE
#define QO_GEMM_TILE 256, 256, 128, 4, 2
#endif

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

// ---------------------------------------------------------------------------
// Generic kernel.
// ---------------------------------------------------------------------------
template <class OT>
__global__ void __launch_bounds__(256)
gemm_i4_generic(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t bsp,
                int64_t bsn, const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
                typename OT::T* __restrict__ out, int64_t ldc, int64_t M, int64_t N, int64_t KP) {
  const int64_t n = (int64_t)blockIdx.x * 16 + (threadIdx.x & 15);
  const int64_t m = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  if (m >= M || n >= N) return;
  const int32_t* ar = a + m * lda;
  const int32_t* bc = b + n * bsn;
  int acc = 0;
  for (int64_t p = 0; p < KP; ++p) {
    const uint32_t wa = (uint32_t)ar[p], wb = (uint32_t)bc[p * bsp];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += nib(wa, i) * nib(wb, i);
  }
  out[m * ldc + n] = OT::cvt(scale_out(acc, load_scale(sa, sad, m), load_scale(sb, sbd, n)));
}

// ---------------------------------------------------------------------------
// MFMA kernel.
// ---------------------------------------------------------------------------

// Widen one packed word to two dwords of 16*q bytes (see file comment).
__device__ inline void widen16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t t = w ^ 0x88888888u;
  lo = (t << 4) & 0xF0F0F0F0u;
  hi = t & 0xF0F0F0F0u;
}

// Block tile BM x BN, BK k per LDS stage, WGM x WGN waves, wave tile
// (BM/WGM) x (BN/WGN) made of 16x16 accumulator blocks. B_NK: B words are
// k-contiguous per column (b_stride_p == 1, the W.t() view); otherwise
// n-contiguous per packed row (b_stride_n == 1, the reference's [K/8, N]).
template <int BM, int BN, int BK, int WGM, int WGN>
struct GemmCfg {
  static constexpr int THREADS = 64 * WGM * WGN;
  static constexpr int BKW = BK / 8;            // packed words per row per stage
  static constexpr int ROW = BK + 16;           // LDS row stride in bytes (padding against bank conflicts)
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int FM = WM / 16, FN = WN / 16;
  static constexpr int A_VEC = BM * BKW / 4 / THREADS;   // dwordx4 loads of A per thread per stage
  static constexpr int B_VEC = BN * BKW / 4 / THREADS;   // dwordx4 loads of B per thread per stage
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile");
  static_assert(A_VEC >= 1 && A_VEC * 4 * THREADS == BM * BKW, "A tile must split into dwordx4 loads");
  static_assert(B_VEC >= 1 && B_VEC * 4 * THREADS == BN * BKW, "B tile must split into dwordx4 loads");
};

template <int BM, int BN, int BK, int WGM, int WGN, bool B_NK, class OT>
__global__ void __launch_bounds__(64 * WGM * WGN, 1)
gemm_i4_mfma(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t ldb,
             const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
             typename OT::T* __restrict__ out, int64_t ldc, int M, int N, int K, int tiles_m, int tiles_n) {
  using C = GemmCfg<BM, BN, BK, WGM, WGN>;
  constexpr int NT = C::THREADS;
  constexpr int BKW = C::BKW, ROW = C::ROW, FM = C::FM, FN = C::FN;
  __shared__ __align__(16) unsigned char As[2][BM * ROW];
  __shared__ __align__(16) unsigned char Bs[2][BN * ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int li = lane & 15, lg = lane >> 4;

  // XCD-aware tile order: consecutive workgroups go round-robin over the 8
  // XCDs; regroup so each XCD gets a contiguous run of tiles (column-major:
  // the tiles of one run share B columns and sweep A), keeping reuse in its L2.
  const int nblk = gridDim.x;
  int pid = blockIdx.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  const int tm = pid % tiles_m, tn = pid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int KP = K >> 3;                       // packed words along k
  const int nk = (KP + BKW - 1) / BKW;         // stages

  // Global -> register staging. A: row r, words c4*4..c4*4+3 of the stage.
  uint32_t ra[C::A_VEC][4], rb[C::B_VEC][4];
  auto load_stage = [&](int ks) {
    const int kw0 = ks * BKW;
#pragma unroll
    for (int i = 0; i < C::A_VEC; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / (BKW / 4), c4 = idx % (BKW / 4);
      const int m = m0 + r, kw = kw0 + c4 * 4;
      if (m < M && kw + 3 < KP) {
        const v4i v = *reinterpret_cast<const v4i*>(a + (int64_t)m * lda + kw);
#pragma unroll
        for (int j = 0; j < 4; ++j) ra[i][j] = (uint32_t)v[j];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ra[i][j] = (m < M && kw + j < KP) ? (uint32_t)a[(int64_t)m * lda + kw + j] : 0x88888888u;
      }
    }
#pragma unroll
    for (int i = 0; i < C::B_VEC; ++i) {
      const int idx = tid + i * NT;
      if (B_NK) {
        const int r = idx / (BKW / 4), c4 = idx % (BKW / 4);
        const int n = n0 + r, kw = kw0 + c4 * 4;
        if (n < N && kw + 3 < KP) {
          const v4i v = *reinterpret_cast<const v4i*>(b + (int64_t)n * ldb + kw);
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[i][j] = (uint32_t)v[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            rb[i][j] = (n < N && kw + j < KP) ? (uint32_t)b[(int64_t)n * ldb + kw + j] : 0x88888888u;
        }
      } else {
        const int p = idx / (BN / 4), c4 = idx % (BN / 4);
        const int kw = kw0 + p, n = n0 + c4 * 4;
        if (kw < KP && n + 3 < N) {
          const v4i v = *reinterpret_cast<const v4i*>(b + (int64_t)kw * ldb + n);
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[i][j] = (uint32_t)v[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            rb[i][j] = (kw < KP && n + j < N) ? (uint32_t)b[(int64_t)kw * ldb + n + j] : 0x88888888u;
        }
      }
    }
  };
  // Register -> LDS, widening nibbles to 16*q bytes. Words outside the matrix
  // were loaded as 0x88888888 (all codes 0) and contribute nothing.
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::A_VEC; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / (BKW / 4), c4 = idx % (BKW / 4);
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) widen16(ra[i][j], w[2 * j], w[2 * j + 1]);
      unsigned char* dst = &As[buf][r * ROW + c4 * 32];
      *reinterpret_cast<v4i*>(dst) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      *reinterpret_cast<v4i*>(dst + 16) = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
    }
#pragma unroll
    for (int i = 0; i < C::B_VEC; ++i) {
      const int idx = tid + i * NT;
      if (B_NK) {
        const int r = idx / (BKW / 4), c4 = idx % (BKW / 4);
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) widen16(rb[i][j], w[2 * j], w[2 * j + 1]);
        unsigned char* dst = &Bs[buf][r * ROW + c4 * 32];
        *reinterpret_cast<v4i*>(dst) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        *reinterpret_cast<v4i*>(dst + 16) = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
      } else {
        const int p = idx / (BN / 4), c4 = idx % (BN / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t lo, hi;
          widen16(rb[i][j], lo, hi);
          *reinterpret_cast<v2i*>(&Bs[buf][(c4 * 4 + j) * ROW + p * 8]) = v2i{(int)lo, (int)hi};
        }
      }
    }
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) load_stage(ks + 1);
    const unsigned char* as = As[cur] + (wm * C::WM + li) * ROW + lg * 16;
    const unsigned char* bs = Bs[cur] + (wn * C::WN + li) * ROW + lg * 16;
#pragma unroll
    for (int kk = 0; kk < BK / 64; ++kk) {
      v4i fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[i] = *reinterpret_cast<const v4i*>(as + i * 16 * ROW + kk * 64);
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[j] = *reinterpret_cast<const v4i*>(bs + j * 16 * ROW + kk * 64);
      // Transposed product: the accumulator of block (i, j) holds C[m][n] at
      // m = 16i + lane%16, n = 16j + 4(lane/16) + r, i.e. four consecutive n.
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    if (ks + 1 < nk) store_stage(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: undo the 256x scale, two float32 products, one rounding.
  using T = typename OT::T;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * C::WM + 16 * i + li;
    if (m >= M) continue;
    const float s_a = load_scale(sa, sad, m);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * C::WN + 16 * j + 4 * lg;
      T v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nn = n + r < N ? n + r : N - 1;
        v[r] = OT::cvt(scale_out(acc[i][j][r] >> 8, s_a, load_scale(sb, sbd, nn)));
      }
      T* o = out + (int64_t)m * ldc + n;
      if (n + 3 < N) {
        if constexpr (sizeof(T) == 2) {
          typedef short v4s __attribute__((ext_vector_type(4)));
          v4s pk;
#pragma unroll
          for (int r = 0; r < 4; ++r) pk[r] = __builtin_bit_cast(short, v[r]);
          *reinterpret_cast<v4s*>(o) = pk;
        } else {
          *reinterpret_cast<v4f*>(o) = v4f{v[0], v[1], v[2], v[3]};
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) o[r] = v[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------

template <class OT>
static void launch_generic(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn,
                           const void* sa, int sad, const void* sb, int sbd, void* out, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, hipStream_t stream) {
  dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
  hipLaunchKernelGGL(gemm_i4_generic<OT>, grid, dim3(256), 0, stream, a, lda, b, bsp, bsn, sa, sad, sb, sbd,
                     reinterpret_cast<typename OT::T*>(out), ldc, M, N, K / 8);
}

template <int BM, int BN, int BK, int WGM, int WGN, bool B_NK, class OT>
static void launch_mfma(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, const void* sa, int sad,
                        const void* sb, int sbd, void* out, int64_t ldc, int M, int N, int K, hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_i4_mfma<BM, BN, BK, WGM, WGN, B_NK, OT>), dim3(tiles_m * tiles_n),
                     dim3(64 * WGM * WGN), 0, stream, a, lda,
                     b, ldb, sa, sad, sb, sbd, reinterpret_cast<typename OT::T*>(out), ldc, M, N, K, tiles_m,
                     tiles_n);
}

template <class OT>
static void dispatch(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, const void* sa,
                     int sad, const void* sb, int sbd, void* out, int64_t ldc, int64_t M, int64_t N, int64_t K,
                     hipStream_t stream, bool allow_fast) {
  using T = typename OT::T;
  const bool b_nk = (bsp == 1);
  const bool b_kn = (bsn == 1) && !b_nk;
  const int64_t ldb = b_nk ? bsn : bsp;
  const bool fits = M <= INT32_MAX / 2 && N <= INT32_MAX / 2 && K <= 65536;
  const bool aligned = ((uintptr_t)a % 16 == 0) && (lda % 4 == 0) && ((uintptr_t)b % 16 == 0) && (ldb % 4 == 0) &&
                       ((uintptr_t)out % (4 * sizeof(T)) == 0) && (ldc % 4 == 0);
  if (allow_fast && fits && aligned && (b_nk || b_kn)) {
    const int m = (int)M, n = (int)N, k = (int)K;
    if (b_nk)
      launch_mfma<QO_GEMM_TILE, true, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, m, n, k, stream);
    else
      launch_mfma<QO_GEMM_TILE, false, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, m, n, k, stream);
    return;
  }
  launch_generic<OT>(a, lda, b, bsp, bsn, sa, sad, sb, sbd, out, ldc, M, N, K, stream);
}

}  // namespace qo

// QO_GEMM_FORCE_GENERIC=1 routes every call through the generic kernel (tests
// use it to cross-check the two).
static bool gemm_allow_fast() {
  const char* e = getenv("QO_GEMM_FORCE_GENERIC");
  return !(e && e[0] == '1');
}

static bool is_float_code(int d) { return d == QO_DTYPE_F32 || d == QO_DTYPE_F16 || d == QO_DTYPE_BF16; }

extern "C" int qo_int4_gemm(const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                            int64_t b_stride_n, const void* scale_a, int scale_a_dtype, const void* scale_b,
                            int scale_b_dtype, void* out, int out_dtype, int64_t ldc, int64_t M, int64_t N,
                            int64_t K, void* stream) {
  using namespace qo;
  if (M < 0 || N < 0 || K < 0 || (K % 8) != 0) {
    qo_set_error("qo_int4_gemm: invalid sizes M=%lld N=%lld K=%lld (K must be a multiple of 8)", (long long)M,
                 (long long)N, (long long)K);
    return QO_ERR_SHAPE;
  }
  if (K >= (int64_t(1) << 21)) {
    qo_set_error("qo_int4_gemm: K=%lld exceeds the exact int32 accumulation range (K < 2^21)", (long long)K);
    return QO_ERR_SHAPE;
  }
  if (lda < K / 8 || ldc < N) {
    qo_set_error("qo_int4_gemm: leading dimensions too small (lda=%lld, ldc=%lld)", (long long)lda,
                 (long long)ldc);
    return QO_ERR_SHAPE;
  }
  if (!is_float_code(scale_a_dtype) || !is_float_code(scale_b_dtype) || !is_float_code(out_dtype)) {
    qo_set_error("qo_int4_gemm: unsupported dtype codes (scale_a=%d, scale_b=%d, out=%d)", scale_a_dtype,
                 scale_b_dtype, out_dtype);
    return QO_ERR_DTYPE;
  }
  if (M == 0 || N == 0) return QO_OK;
  if (!a || !b || !scale_a || !scale_b || !out) {
    qo_set_error("qo_int4_gemm: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool fast = gemm_allow_fast();
  switch (out_dtype) {
    case QO_DTYPE_F16:
      dispatch<OutF16>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out, ldc,
                       M, N, K, s, fast);
      break;
    case QO_DTYPE_BF16:
      dispatch<OutBF16>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out,
                        ldc, M, N, K, s, fast);
      break;
    default:
      dispatch<OutF32>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out, ldc,
                       M, N, K, s, fast);
      break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qo_set_error("qo_int4_gemm: launch failed: %s", hipGetErrorString(e));
    return QO_ERR_LAUNCH;
  }
  return QO_OK;
}
