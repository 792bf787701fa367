// W4A4 GEMM for gfx950 (MI355X): packed int4 x packed int4 -> int32 -> scaled fp.
//
// out[m, n] = rnd_out((float(acc) * scale_a[m]) * scale_b[n]), acc = sum_k qa[m,k] qb[k,n]
// exactly. Replaces the reference's dp4a kernel (int4_matmul/kernels/
// cuda_int4_matmul_kernel.cu:49-189); numerics are those of its fallback
// int4_matmul_pytorch (int4_matmul/ops.py:69-103): the float32 matmul of
// integers is exact, then two separate float32 products, then one rounding.
//
// MFMA kernels: gfx950 has no int4 MFMA, so nibbles are widened to int8 and
// fed to v_mfma_i32_16x16x64_i8. gemm_i4_pp and gemm_i4_pp2 (K % 128 == 0,
// the main path; gemm_i4_pp2 is its ping-pong form for 256-row tiles with
// 16-bit outputs) stage packed words in LDS and widen after the LDS read; gemm_i4_mfma
// (any K % 8 == 0) widens on the way from registers into LDS. Widening trick: XOR with 0x8 turns the offset code
// (q + 8) into q's 4-bit two's-complement pattern; placing it in the high half
// of a byte gives the int8 value 16*q. Both operands carry the factor 16, so the
// accumulator holds 256*acc, exact while 256 * 64 * K < 2^31 (K <= 65536); the
// epilogue shifts it back. Each packed word gives a "low" dword (nibbles
// 0,2,4,6) and a "high" dword (nibbles 1,3,5,7); A and B use the same k order.
//
// Generic kernel (gemm_i4_generic): one output per thread, any strides and
// sizes (K < 2^21). Used when the fast kernel's layout / alignment
// requirements are not met.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"

#ifndef QO_GEMM_TILE
#define QO_GEMM_TILE 256, 256, 128, 4, 2
#endif

namespace qo {

// ---------------------------------------------------------------------------
// Generic kernel.
// ---------------------------------------------------------------------------
template <class OT>
__global__ void __launch_bounds__(256)
gemm_i4_generic(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t bsp,
                int64_t bsn, const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
                typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int64_t M,
                int64_t N, int64_t KP) {
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
  out[m * ldc + n] = add_bias<OT>(OT::cvt(scale_out(acc, load_scale(sa, sad, m), load_scale(sb, sbd, n))), bias, n);
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
             typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M, int N, int K,
             int tiles_m, int tiles_n) {
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
        v[r] = add_bias<OT>(OT::cvt(scale_out(acc[i][j][r] >> 8, s_a, load_scale(sb, sbd, nn))), bias, nn);
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
// Pipelined MFMA kernel (gemm_i4_pp): packed words go from global memory to
// LDS by LDS-DMA (global_load_lds_dwordx4, no VGPR staging) through a ring of
// STAGES buffers, 128 k (16 packed words per row) per stage; nibbles are
// widened to int8 in registers after the LDS read, so LDS holds and serves
// half the bytes of a widened layout.
//
// Operand layout. A lane's 16-byte DMA chunk is four consecutive packed words
// of one row (A) or column (B): lane L of chunk c holds row 16c + L%16, words
// 4(L/16) .. 4(L/16)+3 of the stage. Those four words feed two MFMAs: words
// 4g, 4g+1 the first (h = 0) and 4g+2, 4g+3 the second (h = 1), g = L/16, each
// word widened to a "low" and a "high" dword. A and B follow the same word
// order, which is all the MFMA needs (k order is free if both operands agree).
//
// B layouts:
//  * NK (b_stride_p == 1, the W.t() view): B chunks exactly like A's.
//  * KN (b_stride_n == 1, the reference's [K/8, N]): the DMA copies rows of
//    packed words (256 columns per 1 KiB DMA) into LDS rows of KN_ROW bytes
//    (1040: the four lane groups' rows start on different banks). A lane needs
//    words 4g .. 4g+3 of its column, one per row; with the interleaved column
//    plan (ColPlan) one 16-byte read of a row returns that word for four
//    adjacent columns, which feed four different accumulator blocks.
// ---------------------------------------------------------------------------

template <int BM, int BN, bool B_NK>
struct DmaStage {
  static constexpr int A_BYTES = BM / 16 * 1024;
  static constexpr int KN_ROW = 1040;
  static constexpr int B_BYTES = B_NK ? BN / 16 * 1024 : 16 * KN_ROW;
  static constexpr int BYTES = A_BYTES + B_BYTES;
  static constexpr int A_DMA = BM / 16;
  static constexpr int B_DMA = B_NK ? BN / 16 : 16;
  static constexpr int DMA = A_DMA + B_DMA;
  static_assert(BM % 16 == 0 && BN % 16 == 0, "tile");
  static_assert(B_NK || BN <= 256, "a KN row of the tile must fit one 1 KiB DMA");
};

// Which output columns a wave's FN accumulator blocks hold. A block's 16
// "rows" in the transposed product are 16 B columns, one per lane li of its
// operand. Plain (IL false): block j holds columns 16j .. 16j + 15 of the
// wave's WN. Interleaved (IL true, the [K/8, N] layout, where one LDS read of
// a packed row returns adjacent columns): the first G4 groups of 64 columns
// are spread over 4 blocks each, lane li's 16-byte read giving columns
// 4li .. 4li + 3 to blocks 4q .. 4q + 3; then an optional 32-column group over
// 2 blocks (8-byte reads); then 16-column blocks as in the plain plan.
// A lane (li, lg) of block j holds rows r = 0..3, column f (4lg + r) + c of its
// group (f the interleave, c = the block's place in the group), so it owns FN
// runs ("chunks") of 4 adjacent columns; chunk u's element e is
// acc[.][blk(u, e)][reg(u, e)].
template <int WN, bool IL>
struct ColPlan {
  static constexpr int FN = WN / 16;
  static constexpr int G4 = IL ? WN / 64 : 0;
  static constexpr int G2 = IL ? (WN % 64) / 32 : 0;
  static constexpr int J2 = 4 * G4, J1 = 4 * G4 + 2 * G2;   // first block of the 32- and 16-column groups
  // first column (in the wave's WN) of chunk u for lane group lg
  __device__ static constexpr int col(int u, int lg) {
    return u < J2 ? 64 * (u / 4) + 16 * lg + 4 * (u % 4)
         : u < J1 ? 64 * G4 + 8 * lg + 4 * (u - J2)
                  : 64 * G4 + 32 * G2 + 16 * (u - J1) + 4 * lg;
  }
  __device__ static constexpr int blk(int u, int e) { return u < J2 ? 4 * (u / 4) + e : u < J1 ? J2 + e % 2 : u; }
  __device__ static constexpr int reg(int u, int e) { return u < J2 ? u % 4 : u < J1 ? 2 * (u - J2) + e / 2 : e; }
};

// Epilogue of a wave's FM x FN blocks of a tile (float32 outputs): undo the
// 256x scale of the widened operands, two float32 products (acc * sa) * sb,
// one rounding to the output type, then the optional bias in the output type,
// added as the reference's `output + bias.to(dtype)` does (one float32 add of
// the two output-type values, one rounding back). acc[i][j][r] holds row
// m = mrow + 16i + li (the transposed product) and the column ColPlan gives; a
// lane stores runs of four adjacent outputs; rows and columns past the matrix
// edge are skipped (N % 4 == 0 whenever IL, so a run is all in or all out).
// The tile's scales and bias are in LDS as float32: ssa = the wave's rows,
// ssb / sbias = its columns (sbias null: no bias).
template <int FM, int WN, bool IL, class OT>
__device__ inline void store_c_lds(const v4i (&acc)[FM][WN / 16], const float* ssa, const float* ssb,
                                   const float* sbias, typename OT::T* out, int64_t ldc, int M, int N, int mrow,
                                   int ncol, int li, int lg) {
  using T = typename OT::T;
  using CP = ColPlan<WN, IL>;
  constexpr int FN = CP::FN;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = mrow + 16 * i + li;
    const float sav = ssa[16 * i + li];
    if (m >= M) continue;
#pragma unroll
    for (int u = 0; u < FN; ++u) {
      const int c = CP::col(u, lg);
      const int n = ncol + c;
      if (n >= N) continue;
      const v4f sbv = *reinterpret_cast<const v4f*>(ssb + c);
      T v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = OT::cvt(scale_out(acc[i][CP::blk(u, r)][CP::reg(u, r)] >> 8, sav, sbv[r]));
      if (sbias) {
        const v4f bb = *reinterpret_cast<const v4f*>(sbias + c);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = OT::cvt((float)v[r] + bb[r]);
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

// First half of the staged epilogue: the wave's values (scaled, rounded, bias
// added as in store_c_lds) written as 8-byte runs into an LDS tile; c_tile
// points at the wave's first row and column, pitch in bytes.
template <int FM, int WN, bool IL, class OT>
__device__ __attribute__((always_inline)) inline void stage_c(const v4i (&acc)[FM][WN / 16], const float* ssa, const float* ssb, const float* sbias,
                               unsigned char* c_tile, int pitch, int li, int lg) {
  using T = typename OT::T;
  using CP = ColPlan<WN, IL>;
  static_assert(sizeof(T) == 2, "16-bit outputs");
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const float sav = ssa[16 * i + li];
#pragma unroll
    for (int u = 0; u < CP::FN; ++u) {
      const int c = CP::col(u, lg);
      const v4f sbv = *reinterpret_cast<const v4f*>(ssb + c);
      T v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = OT::cvt(scale_out(acc[i][CP::blk(u, r)][CP::reg(u, r)] >> 8, sav, sbv[r]));
      if (sbias) {
        const v4f bb = *reinterpret_cast<const v4f*>(sbias + c);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = OT::cvt((float)v[r] + bb[r]);
      }
      *reinterpret_cast<v2i*>(c_tile + (16 * i + li) * pitch + 2 * c) =
          v2i{(int)(out_bits<OT>(v[0]) | out_bits<OT>(v[1]) << 16), (int)(out_bits<OT>(v[2]) | out_bits<OT>(v[3]) << 16)};
    }
  }
}

// ---------------------------------------------------------------------------
// A stage's packed words are read from LDS into a second register set while
// the previous stage's MFMAs run, so LDS latency is never waited on between
// MFMAs. Step s (buffer J = s % STAGES, registers
// P = s % 2, filled during step s - 1):
//   wait for this wave's DMA of stage s + 1; lgkmcnt(0) + barrier (every
//   wave's share of stage s + 1 has landed and every wave holds stage s in
//   registers, so buffer J is free); DMA stage s + STAGES into buffer J; read
//   stage s + 1 into registers 1 - P; widen and multiply stage s.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WGM, int WGN, int STAGES, bool B_NK, class OT>
__global__ void __launch_bounds__(64 * WGM * WGN, 1)
gemm_i4_pp(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t ldb,
           const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
           typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M, int N,
           int K, int tiles_m) {
  using S = DmaStage<BM, BN, B_NK>;
  constexpr int W = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int PER = (S::DMA + W - 1) / W;   // DMA instructions per wave per stage
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile");
  static_assert(STAGES >= 2 && STAGES <= 4 && STAGES % 2 == 0, "stages (even: register sets alternate)");
  static_assert(PER * (STAGES - 1) < 64, "vmcnt range");

  // The stage ring; after the last stage it holds the output tile on its way
  // to global memory (16-bit outputs), so it is one object sized for both.
  constexpr int C_PITCH = BN * 2 + 16;
  constexpr int RING = STAGES * S::BYTES, CTILE = sizeof(typename OT::T) == 2 ? BM * C_PITCH : 0;
  __shared__ __align__(16) unsigned char ring[RING > CTILE ? RING : CTILE];
  __shared__ __align__(16) float s_sa[BM];
  __shared__ __align__(16) float s_sb[BN];
  __shared__ __align__(16) float s_bias[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int li = lane & 15, lg = lane >> 4;

  const int nblk = gridDim.x;
  int pid = blockIdx.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  // Grouped tile order: groups of 4 row tiles x every column tile, so the
  // workgroups an XCD runs at once cover a compact block of C and share its
  // A and B tiles in that XCD's L2 (at 4096 x 14336: 4 row tiles and 8 column
  // tiles instead of all 16 row tiles and 2 column tiles; 1-5 % faster at the
  // benched shapes).
  constexpr int GM = 4;
  const int tiles_n = (N + BN - 1) / BN;
  const int g = pid / (GM * tiles_n), w = pid % (GM * tiles_n);
  const int gm = min(GM, tiles_m - g * GM);
  const int tm = g * GM + w % gm, tn = w / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K >> 7;

  // Copy t of this wave reads base + voff[t] (+ the stage's advance): the
  // base is wave-uniform (SGPRs), voff the lane's 32-bit byte offset inside
  // the tile. Rows and columns past the matrix edge are clamped; they only
  // feed accumulators that are never stored. Spare slots repeat the last copy.
  const char* const a_base = reinterpret_cast<const char*>(a + (int64_t)m0 * lda);
  const char* const b_base = reinterpret_cast<const char*>(B_NK ? b + (int64_t)n0 * ldb : b + n0);
  const int64_t b_adv = B_NK ? 64 : 64 * ldb;   // bytes per stage
  bool is_a[PER];
  uint32_t dst[PER], voff[PER];
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    int i = __builtin_amdgcn_readfirstlane(wave) + W * t;
    i = i < S::DMA ? i : S::DMA - 1;
    is_a[t] = i < S::A_DMA;
    if (i < S::A_DMA) {
      voff[t] = (uint32_t)(min(16 * i + li, M - 1 - m0) * (int)lda * 4 + 16 * lg);
      dst[t] = i * 1024;
    } else if (B_NK) {
      const int c = i - S::A_DMA;
      voff[t] = (uint32_t)(min(16 * c + li, N - 1 - n0) * (int)ldb * 4 + 16 * lg);
      dst[t] = S::A_BYTES + c * 1024;
    } else {
      const int p = i - S::A_DMA;
      voff[t] = (uint32_t)(p * (int)ldb * 4 + 4 * min(4 * lane, N - 4 - n0));
      dst[t] = S::A_BYTES + p * S::KN_ROW;
    }
    // wave-uniform: kept in SGPRs (M0 operands), not in VGPRs that compete
    // with the operands and accumulators
    dst[t] = __builtin_amdgcn_readfirstlane(dst[t]);
  }

  auto stage_ptr = [&](auto buf) -> unsigned char* { return ring + decltype(buf)::value * S::BYTES; };
  auto issue = [&](int ks, auto buf) {
    const uint32_t base =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)stage_ptr(buf);
    const char* ab = a_base + 64 * (int64_t)ks;
    const char* bb = b_base + b_adv * ks;
#pragma unroll
    for (int t = 0; t < PER; ++t) dma16_s(voff[t], is_a[t] ? ab : bb, base + dst[t]);
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // B operand words: word(P, j, t) is packed word 4lg + t of block j's column
  // for this lane. W.t() layout: one 16-byte read per block (br). [K/8, N]
  // layout, interleaved column plan: per packed row 4lg + t, one 16-byte read
  // per 64-column group (b4), one 8-byte read for the 32-column group (b2),
  // one 4-byte read per remaining 16-column block (b1).
  using CP = ColPlan<WN, !B_NK>;
  constexpr int N4 = CP::G4 > 0 ? CP::G4 : 1, N1 = FN - CP::J1 > 0 ? FN - CP::J1 : 1;
  v4i ar[2][FM], br[2][B_NK ? FN : 1];
  v4i b4[2][4][N4];
  v2i b2[2][4];
  int b1[2][4][N1];
  auto word = [&](auto set, int j, int t) -> int {
    constexpr int P = decltype(set)::value;
    if constexpr (B_NK) return br[P][j][t];
    else if (j < CP::J2) return b4[P][t][j / 4][j % 4];
    else if (j < CP::J1) return b2[P][t][j - CP::J2];
    else return b1[P][t][j - CP::J1];
  };
  auto load_regs = [&](auto buf, auto set) {
    constexpr int P = decltype(set)::value;
    const unsigned char* base = stage_ptr(buf);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      ar[P][i] = *reinterpret_cast<const v4i*>(base + (wm * FM + i) * 1024 + 16 * lane);
    if constexpr (B_NK) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        br[P][j] = *reinterpret_cast<const v4i*>(base + S::A_BYTES + (wn * FN + j) * 1024 + 16 * lane);
    } else {
      const unsigned char* cols = base + S::A_BYTES + wn * WN * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const unsigned char* row = cols + (4 * lg + t) * S::KN_ROW;
#pragma unroll
        for (int q = 0; q < CP::G4; ++q) b4[P][t][q] = *reinterpret_cast<const v4i*>(row + 256 * q + 16 * li);
        if constexpr (CP::G2 > 0) b2[P][t] = *reinterpret_cast<const v2i*>(row + 256 * CP::G4 + 8 * li);
#pragma unroll
        for (int j = CP::J1; j < FN; ++j)
          b1[P][t][j - CP::J1] = *reinterpret_cast<const int*>(row + 256 * CP::G4 + 128 * CP::G2 +
                                                               64 * (j - CP::J1) + 4 * li);
      }
    }
  };
  auto compute = [&](auto set) {
    constexpr int P = decltype(set)::value;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i fa[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[i] = widen_pair64(ar[P][i], h);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        v4i fb;
        if constexpr (B_NK) fb = widen_pair64(br[P][j], h);
        else fb = widen_pair(word(set, j, 2 * h), word(set, j, 2 * h + 1));
#pragma unroll
        for (int i = 0; i < FM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb, fa[i], acc[i][j], 0, 0, 0);
      }
    }
  };
  auto step_stage = [&](int s, auto buf, auto set) {
    constexpr int J = decltype(buf)::value;
    constexpr int P = decltype(set)::value;
    gemm_wait_vmcnt<PER * (STAGES - 2)>();
    // lgkmcnt(0) and the barrier as builtins: the compiler's wait tracking then
    // knows this stage's registers have arrived and adds no wait of its own
    // after the next stage's reads are issued. The builtins do not order
    // memory accesses, so empty asm statements with a memory clobber keep the
    // previous step's LDS reads above them and this step's below.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0), vmcnt / expcnt unchanged (max)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(min(s + STAGES, nk - 1), buf);
    load_regs(std::integral_constant<int, (J + 1) % STAGES>{}, std::integral_constant<int, 1 - P>{});
    compute(set);
  };

  // The tile's scales (and bias) as float32 in LDS for the epilogue: one load
  // per thread, issued before the first stages' copies so that its latency
  // overlaps theirs.
  static_assert(BM <= 256 && BN <= 64 * W - 256, "one scale per thread");
  float sv = 0.f, bv = 0.f;
  if (tid < BM) sv = load_scale(sa, sad, min(m0 + tid, M - 1));
  else if (tid >= 256 && tid - 256 < BN) {   // threads 256 .. 256 + BN - 1 (any BM <= 256)
    sv = load_scale(sb, sbd, min(n0 + tid - 256, N - 1));
    if (bias) bv = (float)bias[min(n0 + tid - 256, N - 1)];
  }
  issue(0, std::integral_constant<int, 0>{});
  issue(min(1, nk - 1), std::integral_constant<int, 1>{});
  if constexpr (STAGES > 2) issue(min(2, nk - 1), std::integral_constant<int, 2>{});
  if constexpr (STAGES > 3) issue(min(3, nk - 1), std::integral_constant<int, 3>{});
  gemm_wait_vmcnt<PER * (STAGES - 1)>();
  if (tid < BM) s_sa[tid] = sv;
  else if (tid >= 256 && tid - 256 < BN) {
    s_sb[tid - 256] = sv;
    s_bias[tid - 256] = bv;
  }
  lds_barrier();
  load_regs(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  for (int s = 0; s < nk; s += STAGES) {
    step_stage(s, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    if (s + 1 < nk) step_stage(s + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    if constexpr (STAGES > 2)
      if (s + 2 < nk) step_stage(s + 2, std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{});
    if constexpr (STAGES > 3)
      if (s + 3 < nk) step_stage(s + 3, std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{});
  }
  gemm_wait_vmcnt<0>();

  const float* sbias = bias ? s_bias + wn * WN : nullptr;
  if constexpr (CTILE > 0) {
    // 16-bit outputs: the tile goes through LDS so that each store
    // instruction writes whole 16-byte pieces of a few rows (the store
    // instruction count, not the bytes, bounds the epilogue).
    lds_barrier();   // every wave is done with the ring (its copies were waited above)
    stage_c<FM, WN, !B_NK, OT>(acc, s_sa + wm * WM, s_sb + wn * WN, sbias, ring + wm * WM * C_PITCH + wn * WN * 2,
                               C_PITCH, li, lg);
    lds_barrier();
    copy_out_c<BM, BN, 64 * W, OT>(ring, C_PITCH, out, ldc, M, N, m0, n0, tid);
  } else {
    store_c_lds<FM, WN, !B_NK, OT>(acc, s_sa + wm * WM, s_sb + wn * WN, sbias, out, ldc, M, N, m0 + wm * WM,
                                   n0 + wn * WN, li, lg);
  }
}

// ---------------------------------------------------------------------------
// Ping-pong tiled kernel (gemm_i4_pp2): gemm_i4_pp's tile, stage ring and
// operand layouts with the eight waves split into two groups of one wave per
// SIMD (waves 0-3: rows 0 .. BM/2 - 1, waves 4-7: the rest) that alternate,
// one slot apart, between a load slot (the stage's LDS reads, the copies of
// stage t + 3, the widening of the stage's first half) and a compute slot (its
// MFMAs, the second half widened in their shadow), with a workgroup barrier
// between slots: on every SIMD one wave multiplies while the other loads.
// The tile's scales are requested as raw bits before the first copies and
// converted in the last load slot, where no copy is in flight any more. Each
// group stages and copies out its half of the output tile while the other
// group is still busy: group 0 stages its rows during group 1's last compute
// slot.
// ---------------------------------------------------------------------------
template <int BM, int BN, bool B_NK, class OT>
__global__ void __launch_bounds__(512, 1)
gemm_i4_pp2(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t ldb,
            const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
            typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M, int N,
            int K, int tiles_m) {
  constexpr int WGM = 4, WGN = 2, W = 8, STAGES = 4;
  using S = DmaStage<BM, BN, B_NK>;
  using T = typename OT::T;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int PER = (S::DMA + W - 1) / W;
  static_assert(BM == 256 && FM == 4 && WN % 16 == 0 && BN <= 256, "256-row tiles, 4 x 2 waves");
  static_assert(sizeof(T) == 2, "16-bit outputs (staged epilogue)");
  static_assert(S::A_DMA % W == 0, "copies 0 .. A_DMA / W - 1 of every wave are A's");
  constexpr int TA = S::A_DMA / W;
  constexpr int C_PITCH = BN * 2 + 16;
  constexpr int RING = STAGES * S::BYTES, CTILE = BM * C_PITCH;
  __shared__ __align__(16) unsigned char ring[RING > CTILE ? RING : CTILE];
  __shared__ __align__(16) float s_sa[BM];
  __shared__ __align__(16) float s_sb[BN];
  __shared__ __align__(16) float s_bias[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int li = lane & 15, lg = lane >> 4;
  const bool grp1 = __builtin_amdgcn_readfirstlane(wave) >= W / 2;

  const int nblk = gridDim.x;
  int pid = blockIdx.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  constexpr int GM = 4;
  const int tiles_n = (N + BN - 1) / BN;
  const int g = pid / (GM * tiles_n), w = pid % (GM * tiles_n);
  const int gm = min(GM, tiles_m - g * GM);
  const int tm = g * GM + w % gm, tn = w / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K >> 7;

  const char* const a_base = reinterpret_cast<const char*>(a + (int64_t)m0 * lda);
  const char* const b_base = reinterpret_cast<const char*>(B_NK ? b + (int64_t)n0 * ldb : b + n0);
  const int64_t b_adv = B_NK ? 64 : 64 * ldb;
  uint32_t dst[PER], voff[PER];
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    int i = __builtin_amdgcn_readfirstlane(wave) + W * t;
    i = i < S::DMA ? i : S::DMA - 1;
    if (t < TA) {
      voff[t] = (uint32_t)(min(16 * i + li, M - 1 - m0) * (int)lda * 4 + 16 * lg);
      dst[t] = i * 1024;
    } else if (B_NK) {
      const int c = i - S::A_DMA;
      voff[t] = (uint32_t)(min(16 * c + li, N - 1 - n0) * (int)ldb * 4 + 16 * lg);
      dst[t] = S::A_BYTES + c * 1024;
    } else {
      const int p = i - S::A_DMA;
      voff[t] = (uint32_t)(p * (int)ldb * 4 + 4 * min(4 * lane, N - 4 - n0));
      dst[t] = S::A_BYTES + p * S::KN_ROW;
    }
    dst[t] = __builtin_amdgcn_readfirstlane(dst[t]);
  }
  auto issue = [&](int ks, auto bufc) {
    constexpr uint32_t BUF = decltype(bufc)::value * S::BYTES;
    const uint32_t base = lds_addr(ring) + BUF;
    const char* ab = a_base + 64 * (int64_t)ks;
    const char* bb = b_base + b_adv * ks;
#pragma unroll
    for (int t = 0; t < PER; ++t) dma16_s(voff[t], t < TA ? ab : bb, base + dst[t]);
  };

  using CP = ColPlan<WN, !B_NK>;
  constexpr int N4 = CP::G4 > 0 ? CP::G4 : 1, N1 = FN - CP::J1 > 0 ? FN - CP::J1 : 1;
  v4i ar[FM], br[B_NK ? FN : 1];
  v4i b4[4][N4];
  v2i b2[4];
  int b1[4][N1];
  auto word = [&](int j, int t) -> int {
    if constexpr (B_NK) return br[j][t];
    else if (j < CP::J2) return b4[t][j / 4][j % 4];
    else if (j < CP::J1) return b2[t][j - CP::J2];
    else return b1[t][j - CP::J1];
  };
  auto load_regs = [&](auto bufc) {
    const unsigned char* base = ring + decltype(bufc)::value * S::BYTES;
#pragma unroll
    for (int i = 0; i < FM; ++i) ar[i] = *reinterpret_cast<const v4i*>(base + (wm * FM + i) * 1024 + 16 * lane);
    if constexpr (B_NK) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        br[j] = *reinterpret_cast<const v4i*>(base + S::A_BYTES + (wn * FN + j) * 1024 + 16 * lane);
    } else {
      const unsigned char* cols = base + S::A_BYTES + wn * WN * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const unsigned char* row = cols + (4 * lg + t) * S::KN_ROW;
#pragma unroll
        for (int q = 0; q < CP::G4; ++q) b4[t][q] = *reinterpret_cast<const v4i*>(row + 256 * q + 16 * li);
        if constexpr (CP::G2 > 0) b2[t] = *reinterpret_cast<const v2i*>(row + 256 * CP::G4 + 8 * li);
#pragma unroll
        for (int j = CP::J1; j < FN; ++j)
          b1[t][j - CP::J1] =
              *reinterpret_cast<const int*>(row + 256 * CP::G4 + 128 * CP::G2 + 64 * (j - CP::J1) + 4 * li);
      }
    }
  };
  auto wb = [&](int j, int h) -> v4i {
    if constexpr (B_NK) return widen_pair64(br[j], h);
    else return widen_pair(word(j, 2 * h), word(j, 2 * h + 1));
  };
  auto bar = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // The tile's scales and bias as raw bits, requested by group 0 before the
  // first copies and converted in the last load slot (where the compiler's
  // wait for them costs nothing: no copy is in flight there).
  auto raw16 = [](const void* p, int64_t i) -> uint32_t { return reinterpret_cast<const uint16_t*>(p)[i]; };
  auto raw32 = [](const void* p, int64_t i) -> uint32_t { return reinterpret_cast<const uint32_t*>(p)[i]; };
  uint32_t rsa = 0, rsb = 0, rbias = 0;
  if (tid < BM) {
    const int64_t i = min(m0 + tid, M - 1);
    rsa = sad == QO_DTYPE_F32 ? raw32(sa, i) : raw16(sa, i);
    if (tid < BN) {
      const int64_t j = min(n0 + tid, N - 1);
      rsb = sbd == QO_DTYPE_F32 ? raw32(sb, j) : raw16(sb, j);
      if (bias) rbias = raw16(bias, j);
    }
  }
  issue(0, std::integral_constant<int, 0>{});
  issue(min(1, nk - 1), std::integral_constant<int, 1>{});
  issue(min(2, nk - 1), std::integral_constant<int, 2>{});
  gemm_wait_vmcnt<PER * 2>();
  lds_barrier();

  if (grp1) bar();
  auto phase = [&](int t, auto bufc) {
    constexpr int J = decltype(bufc)::value;
    load_regs(bufc);
    if (t + 3 < nk) issue(t + 3, std::integral_constant<int, (J + 3) & 3>{});
    // wait for this wave's copies of stage t + 1 (min(2, nk - 2 - t) younger stages may stay in flight)
    gemm_wait_groups<PER, 2>(nk - 2 - t);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    if (t == nk - 1 && !grp1) {
      asm volatile("" : "+v"(rsa), "+v"(rsb), "+v"(rbias));
      if (tid < BM) s_sa[tid] = scale_from_bits(rsa, sad);
      if (tid < BN) {
        s_sb[tid] = scale_from_bits(rsb, sbd);
        s_bias[tid] = (float)__builtin_bit_cast(T, (uint16_t)rbias);
      }
    }
    // stage t's first half widened here; the second half one fragment ahead of its MFMAs
    v4i fa[FM], fbn = wb(0, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[i] = widen_pair64(ar[i], 0);
    bar();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const v4i fb = fbn;
        if (j + 1 < FN) fbn = wb(j + 1, h);
        else if (h == 0) fbn = wb(0, 1);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb, fa[i], acc[i][j], 0, 0, 0);
          if (h == 0 && j == FN - 1) fa[i] = widen_pair64(ar[i], 1);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 2 * FM * FN; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }
    bar();
  };
  for (int s = 0; s < nk; s += 4) {
    phase(s, std::integral_constant<int, 0>{});
    if (s + 1 < nk) phase(s + 1, std::integral_constant<int, 1>{});
    if (s + 2 < nk) phase(s + 2, std::integral_constant<int, 2>{});
    if (s + 3 < nk) phase(s + 3, std::integral_constant<int, 3>{});
  }
  // Epilogue. Group 0 (rows 0 .. 127): stage its rows while group 1 runs its
  // last compute slot, then copy them out while group 1 stages its rows;
  // group 1 copies its rows out last.
  const float* sbias = bias ? s_bias + wn * WN : nullptr;
  unsigned char* const c_half = ring + (grp1 ? (BM / 2) * C_PITCH : 0);
  auto stage_half = [&]() {
    stage_c<FM, WN, !B_NK, OT>(acc, s_sa + wm * WM, s_sb + wn * WN, sbias, ring + wm * WM * C_PITCH + wn * WN * 2,
                               C_PITCH, li, lg);
  };
  auto copy_half = [&]() {
    copy_out_c<BM / 2, BN, 256, OT>(c_half, C_PITCH, out, ldc, M, N, m0 + (grp1 ? BM / 2 : 0), n0, tid & 255);
  };
  stage_half();
  lds_barrier();
  copy_half();
  if (!grp1) bar();
}

// The epilogue of a skinny-kernel lane (row m, columns nc .. nc + 3). Its
// scales and bias are requested before the main loop (load), as raw bits
// without a branch on the scale dtype, so that the epilogue (store) does not
// wait a memory round trip for them: (float(acc) * sa) * sb, one rounding,
// then add_bias's arithmetic, 8- or 16-byte stores (element stores at the
// matrix edge).
template <class OT>
struct SkinnyEpilogue {
  using T = typename OT::T;
  uint32_t sa_bits, sb_bits[4];
  T bias_v[4] = {};

  __device__ void load(const void* sa, int sad, const void* sb, int sbd, const T* bias, int m, int nc, int M,
                       int N) {
    sa_bits = scale_bits(sa, sad, min(m, M - 1));
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(nc + r, N - 1);
      sb_bits[r] = scale_bits(sb, sbd, n);
      if (bias) bias_v[r] = bias[n];
    }
  }

  __device__ void store(const v4i& sum, int sad, int sbd, const T* bias, T* out, int64_t ldc, int m, int nc,
                        int N) const {
    const float sam = scale_from_bits(sa_bits, sad);
    T v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const T o = OT::cvt(scale_out(sum[r] >> 8, sam, scale_from_bits(sb_bits[r], sbd)));
      v[r] = bias ? OT::cvt((float)o + (float)bias_v[r]) : o;
    }
    T* o = out + (int64_t)m * ldc + nc;
    if (nc + 3 < N) {
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
        if (nc + r < N) o[r] = v[r];
    }
  }
};

// ---------------------------------------------------------------------------
// Skinny kernel (gemm_i4_skinny): M <= 64, the decode shapes of the [K/8, N]
// layout that the LDS-DMA kernel below does not take (N % 4 != 0 with a padded
// row stride, or B beyond 32-bit byte offsets). The time is the
// read of B, so the work is spread over columns and K instead of tiles: a
// workgroup owns 16 output columns and all M rows; its 8 waves split K into
// contiguous slices of 128-deep stages, stream their slice of B and A from
// global memory straight into registers (CH stages per batch, the next batch
// in flight while this one is multiplied), and the 8 partial int32
// accumulators are summed exactly through LDS before the scale epilogue.
// Operand layout per stage as in the tiled kernels: lane (li, lg) holds words
// 4lg .. 4lg + 3 of row li (A) or column li (B).
// ---------------------------------------------------------------------------
template <int MT, bool B_NK, class OT>
struct SkinnyCfg {
  // stages per batch (two batches in registers). Measured at 16 x 4096 x
  // 14336: 4 is best; 8 and 16 stages per batch were 15 % and 80 % slower.
  static constexpr int CH = 4;
};

template <int MT, bool B_NK, class OT>
__global__ void __launch_bounds__(512)
gemm_i4_skinny(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t ldb,
               const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
               typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M, int N,
               int K) {
  constexpr int CH = SkinnyCfg<MT, B_NK, OT>::CH;
  __shared__ __align__(16) v4i part[8][MT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nk = K >> 7;
  const int s_begin = wave * nk / 8, s_end = (wave + 1) * nk / 8;

  SkinnyEpilogue<OT> epi;   // waves 0 .. MT-1: row 16 wave + li, columns n0 + 4 lg .. + 3
  epi.load(sa, sad, sb, sbd, bias, 16 * wave + li, n0 + 4 * lg, M, N);

  const int n = min(n0 + li, N - 1);
  const int32_t* bcol = B_NK ? b + (int64_t)n * ldb + 4 * lg : b + (int64_t)(4 * lg) * ldb + n;
  const int32_t* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) arow[mt] = a + (int64_t)min(16 * mt + li, M - 1) * lda + 4 * lg;

  v4i acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};

  // Loads of stage s (clamped into the slice, so every batch issues the same
  // loads; stages past the slice end are loaded but not multiplied).
  v4i bq[2][CH], aq[2][CH][MT];
  auto load = [&](int s0, auto set) {
    constexpr int P = decltype(set)::value;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int s = min(s0 + c, s_end - 1);
      if constexpr (B_NK) {
        bq[P][c] = *reinterpret_cast<const v4i*>(bcol + 16 * s);
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) bq[P][c][t] = bcol[(int64_t)(16 * s + t) * ldb];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) aq[P][c][mt] = *reinterpret_cast<const v4i*>(arow[mt] + 16 * s);
    }
  };
  auto compute = [&](int s0, auto set) {
    constexpr int P = decltype(set)::value;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (s0 + c >= s_end) break;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const v4i fb = widen_pair64(bq[P][c], h);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              fb, widen_pair64(aq[P][c][mt], h), acc[mt], 0, 0, 0);
      }
    }
  };
  if (s_begin < s_end) {
    load(s_begin, std::integral_constant<int, 0>{});
    for (int s0 = s_begin; s0 < s_end; s0 += 2 * CH) {
      load(s0 + CH, std::integral_constant<int, 1>{});
      compute(s0, std::integral_constant<int, 0>{});
      if (s0 + CH >= s_end) break;
      load(s0 + 2 * CH, std::integral_constant<int, 0>{});
      compute(s0 + CH, std::integral_constant<int, 1>{});
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) part[wave][mt][lane] = acc[mt];
  __syncthreads();

  // Waves 0 .. MT-1 each finish one 16-row block: exact int32 sum of the 8
  // slices, then (float(acc) * sa) * sb and one rounding, as the tiled kernels.
  if (wave >= MT) return;
  const int mt = wave;
  v4i sum = part[0][mt][lane];
#pragma unroll
  for (int w = 1; w < 8; ++w) sum += part[w][mt][lane];
  const int m = 16 * mt + li;
  const int nc = n0 + 4 * lg;
  if (m >= M || nc >= N) return;
  epi.store(sum, sad, sbd, bias, out, ldc, m, nc, N);
}

// ---------------------------------------------------------------------------
// Skinny kernel for the W.t() layout (gemm_i4_skinny_nk), the decode GEMM of
// the linear layer, and (KN) for the [K/8, N] layout, whose B copies differ
// (see the KN set-up below). Same split as gemm_i4_skinny (16 output columns and all M
// rows per workgroup, exact int32 sums of per-wave partials through LDS), but
// A and B reach LDS by LDS-DMA in "chunks" of CB contiguous bytes of every
// row (the 16 B rows = columns n0 .. n0 + 15, then the 16 MT rows of A): each
// DMA instruction reads 1 KiB of one or two rows. Measured at 16 x 4096 x
// 14336, the same bytes read as 16 rows x 64 B per instruction (one MFMA
// operand straight into registers) take half as long again.
// Chunk c holds stages c SPC .. c SPC + SPC - 1 (stage = 64 B = 128 k per row);
// wave w multiplies SPW of them. LDS slot of 16-byte piece p of row r is
// p ^ (r % 16), so the 16 rows of an operand read sit on distinct banks (the
// DMA's lane -> slot placement is fixed, its source addresses are permuted).
// Chunks go through a ring of RING buffers behind one barrier each, as the
// tiled kernels' stages do. PAIR: a ring small enough (<= 80 KiB) for two
// workgroups to share a CU, so that one's copies overlap the other's multiply
// and epilogue; the host takes it when the columns need more than one round
// of workgroups (or a row has at most two chunks, which a ring of two holds
// whole).
// ---------------------------------------------------------------------------
template <int MT, bool PAIR>
struct SkinnyNkCfg {
  static constexpr int CB = MT == 1 ? 1024 : 512;            // bytes per row per chunk
  static constexpr int SPC = CB / 64, SPW = SPC / 8;         // stages per chunk, per wave
  static constexpr int ROWS = 16 + 16 * MT;
  static constexpr int BUF = ROWS * CB;
  static constexpr bool PAIR_OK = 2 * BUF <= 80 * 1024;     // a two-per-CU ring exists (M <= 64)
  static constexpr int RING = PAIR ? (3 * BUF <= 80 * 1024 ? 3 : 2)
                                   : 4 * BUF <= 150 * 1024 ? 4 : 3 * BUF <= 150 * 1024 ? 3 : 2;
  static constexpr int NI = BUF / 1024;                      // DMA instructions per chunk
  static constexpr int D = (NI + 7) / 8;                     // ... per wave
  static_assert(SPW >= 1 && D * (RING - 1) < 64 && MT <= 8, "chunk shape");
  static_assert(!PAIR || (PAIR_OK && RING * BUF <= 80 * 1024), "two workgroups per CU");
};

template <int MT, bool PAIR, bool KN, class OT>
__global__ void __launch_bounds__(512)
gemm_i4_skinny_nk(const int32_t* __restrict__ a, int64_t lda, const int32_t* __restrict__ b, int64_t ldb,
                  const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
                  typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M,
                  int N, int K) {
  using C = SkinnyNkCfg<MT, PAIR>;
  __shared__ __align__(16) unsigned char ring[C::RING * C::BUF];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // KN: consecutive column blocks on one XCD (workgroup j runs on XCD j % 8),
  // so the two 64-byte halves of a 128-byte line of B are read through one L2.
  // W.t(): block j on XCD j % 8, the placement the linear layer's read-ahead
  // assumes.
  const int nblk = gridDim.x;
  const int cblk = KN && nblk % 8 == 0 ? (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int n0 = cblk * 16;
  const int nk = K >> 7;                        // stages
  const int rowbytes = K >> 1;                  // bytes of a packed row
  const int nch = (rowbytes + C::CB - 1) / C::CB;

  SkinnyEpilogue<OT> epi;   // waves 0 .. MT-1: row 16 wave + li, columns n0 + 4 lg .. + 3
  epi.load(sa, sad, sb, sbd, bias, 16 * wave + li, n0 + 4 * lg, M, N);

  // DMA instruction t of this wave: SGPR base (its first row), the lane's
  // offset to its row (the second row for CB = 512) and to its swizzled piece,
  // and the LDS destination.
  const char* rbase[C::D];
  uint32_t rdiff[C::D], poff[C::D], ldst[C::D];
  auto row_ptr = [&](int r) -> const char* {
    return r < 16 ? reinterpret_cast<const char*>(b + (int64_t)min(n0 + r, N - 1) * ldb)
                  : reinterpret_cast<const char*>(a + (int64_t)min(r - 16, M - 1) * lda);
  };
  // [K/8, N] layout (KN): B instruction i of a chunk copies its stage i, the
  // 16 packed rows x 64 bytes of columns n0 .. n0 + 15, to 1 KiB of LDS; lane
  // l fills LDS row position l / 4, piece l % 4 (columns 4 (l % 4) .. + 3).
  // Packed row 4 g + t of the stage sits at position 4 t + g, so the four rows
  // an operand read takes (g = 0..3, one t) lie on four distinct bank groups.
  // Columns past N (N % 4 == 0) re-read the last four; packed rows past K / 8
  // re-read the last row (never multiplied).
  const int kn_rows = K >> 3;
  const uint32_t kn_ld = (uint32_t)ldb * 4u;
  const uint32_t kn_col = 4u * (uint32_t)min(n0 + 4 * (lane & 3), N - 4);
  const int kn_row = 4 * ((lane >> 2) & 3) + (lane >> 4);
  bool kn_b[C::D];
#pragma unroll
  for (int t = 0; t < C::D; ++t) {
    int i = __builtin_amdgcn_readfirstlane(wave) + 8 * t;
    i = i < C::NI ? i : C::NI - 1;              // spare slots repeat the last copy
    constexpr int RPI = 1024 / C::CB;           // rows per instruction
    const int r0 = RPI * i;
    const int r = r0 + (RPI == 2 ? lane >> 5 : 0);
    const int q = RPI == 2 ? lane & 31 : lane;  // LDS slot in the row
    kn_b[t] = KN && r0 < 16;
    rbase[t] = row_ptr(r0);
    rdiff[t] = (uint32_t)(row_ptr(r) - row_ptr(r0));   // 0 or one row stride (rows clamp monotonically)
    poff[t] = kn_b[t] ? (uint32_t)(16 * i + kn_row) : 16 * (q ^ (r & 15));   // KN: packed row in the chunk
    ldst[t] = __builtin_amdgcn_readfirstlane(i * 1024);
  }
  auto issue = [&](int c, int buf) {
    const uint32_t base = lds_addr(ring) + buf * C::BUF;
    const uint32_t coff = c * C::CB;
#pragma unroll
    for (int t = 0; t < C::D; ++t) {
      if (kn_b[t]) {
        const uint32_t row = min((uint32_t)(c * 16 * C::SPC) + poff[t], (uint32_t)kn_rows - 1);
        dma16_s(row * kn_ld + kn_col, b, base + ldst[t]);
      } else {   // pieces past the row's end re-read its last piece (never multiplied)
        dma16_s(rdiff[t] + min(coff + poff[t], (uint32_t)rowbytes - 16), rbase[t], base + ldst[t]);
      }
    }
  };

  v4i acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};

  auto compute = [&](int c, int buf) {
    const unsigned char* base = ring + buf * C::BUF;
#pragma unroll
    for (int u = 0; u < C::SPW; ++u) {
      const int ls = wave * C::SPW + u;         // stage within the chunk
      if (c * C::SPC + ls >= nk) break;
      const int slot = (4 * ls + lg) ^ li;
      v4i bw;
      if constexpr (KN) {   // packed rows 4 lg + t of stage ls, column n0 + li
        const unsigned char* bs = base + ls * 1024 + 64 * lg + 4 * li;
        bw = v4i{*reinterpret_cast<const int*>(bs), *reinterpret_cast<const int*>(bs + 256),
                 *reinterpret_cast<const int*>(bs + 512), *reinterpret_cast<const int*>(bs + 768)};
      } else {
        bw = *reinterpret_cast<const v4i*>(base + li * C::CB + 16 * slot);
      }
      v4i aw[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        aw[mt] = *reinterpret_cast<const v4i*>(base + (16 + 16 * mt + li) * C::CB + 16 * slot);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const v4i fb = widen_pair64(bw, h);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb, widen_pair64(aw[mt], h), acc[mt],
                                                          0, 0, 0);
      }
    }
  };

  if constexpr (PAIR) {
    // The RING buffers start empty, so the first RING chunks go out at once;
    // step c (c >= 1) refills the buffer of chunk c - 1 with chunk c - 1 + RING.
    // Chunks past the row's end are never issued, so each wait leaves in
    // flight exactly the chunks issued after chunk c.
    for (int c = 0; c < C::RING; ++c)
      if (c < nch) issue(c, c);
    for (int c = 0; c < nch; ++c) {
      const int last = min(max(c + C::RING - 2, C::RING - 1), nch - 1);   // last chunk issued so far
      gemm_wait_groups<C::D, C::RING - 1>(last - c);
      lds_barrier();   // chunk c has landed for every wave; every wave is done with chunk c - 1's buffer
      if (c > 0 && c - 1 + C::RING < nch) issue(c - 1 + C::RING, (c - 1) % C::RING);
      compute(c, c % C::RING);
    }
  } else {
    for (int c = 0; c < C::RING - 1; ++c) issue(min(c, nch - 1), c);
    for (int c = 0; c < nch; ++c) {
      gemm_wait_vmcnt<C::D * (C::RING - 2)>();
      lds_barrier();   // chunk c has landed for every wave; every wave is done with chunk c - 1's buffer
      // Past the row's end the last chunk is copied again (never multiplied)
      // and the waits stay constant: branching round the copy measured
      // 0.4-0.6 us slower in the 32- and 64-token linear step.
      issue(min(c + C::RING - 1, nch - 1), (c + C::RING - 1) % C::RING);
      compute(c, c % C::RING);
    }
  }
  gemm_wait_vmcnt<0>();
  lds_barrier();

  // Partials of the 8 waves, summed exactly by waves 0 .. MT-1 (one 16-row
  // block each), then (float(acc) * sa) * sb, one rounding, optional bias.
  v4i* part = reinterpret_cast<v4i*>(ring);     // [8][MT][64]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) part[(wave * MT + mt) * 64 + lane] = acc[mt];
  __syncthreads();
  if (wave >= MT) return;
  const int mt = wave;
  v4i sum = part[mt * 64 + lane];
#pragma unroll
  for (int w = 1; w < 8; ++w) sum += part[(w * MT + mt) * 64 + lane];
  const int m = 16 * mt + li;
  const int nc = n0 + 4 * lg;
  if (m >= M || nc >= N) return;
  epi.store(sum, sad, sbd, bias, out, ldc, m, nc, N);
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------

// QO_ROUTE_GEMM_NO_DMA keeps the register-staged MFMA kernel for every shape
// (tests use it to cross-check the two MFMA kernels).
static bool gemm_allow_dma() {
  return !route_off(QO_ROUTE_GEMM_NO_DMA);
}

template <class OT>
static void launch_generic(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn,
                           const void* sa, int sad, const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int64_t M,
                           int64_t N, int64_t K, hipStream_t stream) {
  dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
  launch(gemm_i4_generic<OT>, grid, dim3(256), 0, stream, a, lda, b, bsp, bsn, sa, sad, sb, sbd,
                     reinterpret_cast<typename OT::T*>(out), ldc, reinterpret_cast<const typename OT::T*>(bias), M, N, K / 8);
}

template <int BM, int BN, int BK, int WGM, int WGN, bool B_NK, class OT>
static void launch_mfma(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, const void* sa, int sad,
                        const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int M, int N, int K, hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  launch((gemm_i4_mfma<BM, BN, BK, WGM, WGN, B_NK, OT>), dim3(tiles_m * tiles_n),
                     dim3(64 * WGM * WGN), 0, stream, a, lda,
                     b, ldb, sa, sad, sb, sbd, reinterpret_cast<typename OT::T*>(out), ldc, reinterpret_cast<const typename OT::T*>(bias), M, N, K, tiles_m,
                     tiles_n);
}

// Launch of the pipelined kernel: 4 x 2 waves, four-stage ring, either B layout.
template <int BM, int BN, bool B_NK, class OT>
static void launch_dma(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, const void* sa, int sad,
                       const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int M, int N, int K, hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  launch((gemm_i4_pp<BM, BN, 4, 2, 4, B_NK, OT>), dim3(tiles_m * tiles_n), dim3(512), 0, stream, a, lda,
                     b, ldb, sa, sad, sb, sbd, reinterpret_cast<typename OT::T*>(out), ldc,
                     reinterpret_cast<const typename OT::T*>(bias), M, N, K, tiles_m);
}

// 256-row tiles: the ping-pong kernel for 16-bit outputs (its epilogue stages
// 16-bit values), gemm_i4_pp for float32 outputs. Measured against gemm_i4_pp
// (same process, outputs bit-equal): config 4 (4096 x 14336 x 4096, [K/8, N])
// 200.7 -> 192.2 us, its W.t() layout 201.2 -> 187.8 us, 4096 x 4096 x 14336
// W.t() bf16 (the linear layer at 4096 tokens) 172.8 -> 154.1 us.
template <int BN, bool B_NK, class OT>
static void launch_tiled(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, const void* sa, int sad,
                         const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int M, int N, int K,
                         hipStream_t stream) {
  if constexpr (sizeof(typename OT::T) == 2) {
    const int tiles_m = (M + 255) / 256, tiles_n = (N + BN - 1) / BN;
    launch((gemm_i4_pp2<256, BN, B_NK, OT>), dim3(tiles_m * tiles_n), dim3(512), 0, stream, a, lda, b, ldb, sa, sad,
           sb, sbd, reinterpret_cast<typename OT::T*>(out), ldc, reinterpret_cast<const typename OT::T*>(bias), M, N, K,
           tiles_m);
  } else {
    launch_dma<256, BN, B_NK, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
  }
}

// Fraction of the machine's workgroup slots doing useful output in a launch
// of BM x BN tiles (one workgroup per CU): tile-count rounding plus ragged
// edge tiles.
static double tile_efficiency(int64_t M, int64_t N, int BM, int BN, int cus) {
  const int64_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const int64_t tiles = tm * tn, rounds = (tiles + cus - 1) / cus;
  return (double)(M * N) / ((double)rounds * cus * BM * BN);
}



template <bool B_NK, class OT>
static void dispatch_dma(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, const void* sa, int sad,
                         const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int M, int N, int K, hipStream_t stream) {
  const int cus = device_cu_count();
  const double e224 = tile_efficiency(M, N, 256, 224, cus), e256 = tile_efficiency(M, N, 256, 256, cus);
  // At most half a round of 256-row tiles (M of a few hundred rows over many
  // columns): 128 x 128 tiles, four times as many, two workgroups per CU.
  // Measured at 14336 x 4096 (N x K): M = 512 (0.5) 48.6 -> 40.6 us, M = 768
  // (0.75) 48.9 -> 57.6 us, so the limit is 0.5.
  if (std::max(e224, e256) <= 0.5)
    launch_dma<128, 128, B_NK, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
  else if (e224 > e256)
    launch_tiled<224, B_NK, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
  else
    launch_tiled<256, B_NK, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
}

// QO_ROUTE_GEMM_NO_SKINNY sends small M to the tiled kernels (tests use it to
// cross-check the two).
static bool gemm_allow_skinny() {
  return !route_off(QO_ROUTE_GEMM_NO_SKINNY);
}

static bool skinny_kn_dma_ok(int64_t N, int64_t K, int64_t ldb) {
  return N >= 4 && N % 4 == 0 && (K / 8 - 1) * ldb * 4 + N * 4 < (1LL << 31);
}

template <class OT>
static void launch_skinny(const int32_t* a, int64_t lda, const int32_t* b, int64_t ldb, bool b_nk, const void* sa,
                          int sad, const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int M, int N, int K,
                          hipStream_t stream) {
  const dim3 grid((unsigned)((N + 15) / 16));
  using T = typename OT::T;
  // The LDS-DMA kernel for both layouts; [K/8, N] needs whole 4-column groups
  // and 32-bit byte offsets over B, else the register-streaming kernel.
  const bool kn_dma = !b_nk && skinny_kn_dma_ok(N, K, ldb);
  auto go = [&](auto mt, auto nk_layout) {
    constexpr int MT = decltype(mt)::value;
    constexpr bool NK = decltype(nk_layout)::value;
    using Cfg = SkinnyNkCfg<MT, false>;
    const int64_t cb = Cfg::CB;
    const bool pair = (K / 2 + cb - 1) / cb <= 2 || (N + 15) / 16 > device_cu_count();
    if (NK || kn_dma) {
      bool launched = false;
      if constexpr (Cfg::PAIR_OK) {
        if (pair) {
          launch((gemm_i4_skinny_nk<MT, true, !NK, OT>), grid, dim3(512), 0, stream, a, lda, b, ldb, sa, sad, sb,
                 sbd, reinterpret_cast<T*>(out), ldc, reinterpret_cast<const T*>(bias), M, N, K);
          launched = true;
        }
      }
      if (!launched)
        launch((gemm_i4_skinny_nk<MT, false, !NK, OT>), grid, dim3(512), 0, stream, a, lda, b, ldb, sa, sad, sb,
               sbd, reinterpret_cast<T*>(out), ldc, reinterpret_cast<const T*>(bias), M, N, K);
    } else if constexpr (MT <= 4) {
      launch((gemm_i4_skinny<MT, false, OT>), grid, dim3(512), 0, stream, a, lda, b, ldb, sa, sad, sb, sbd,
             reinterpret_cast<T*>(out), ldc, reinterpret_cast<const T*>(bias), M, N, K);
    } else if (g_launch_error == hipSuccess) {
      // M > 64 comes here only with a layout the LDS-DMA kernel takes; report
      // rather than leave the output unwritten if that ever changes
      g_launch_error = hipErrorInvalidConfiguration;
    }
  };
  auto by_layout = [&](auto mt) {
    if (b_nk) go(mt, std::true_type{});
    else go(mt, std::false_type{});
  };
  const int mt = (M + 15) / 16;
  if (mt == 1) by_layout(std::integral_constant<int, 1>{});
  else if (mt == 2) by_layout(std::integral_constant<int, 2>{});
  else if (mt == 3) by_layout(std::integral_constant<int, 3>{});
  else if (mt == 4) by_layout(std::integral_constant<int, 4>{});
  else if (mt == 5) by_layout(std::integral_constant<int, 5>{});
  else if (mt == 6) by_layout(std::integral_constant<int, 6>{});
  else if (mt == 7) by_layout(std::integral_constant<int, 7>{});
  else by_layout(std::integral_constant<int, 8>{});
}

// Shapes that take the FP6 route when the caller gives a workspace: the
// tiled shapes (more than 256 rows; fewer take the small-M kernels), 16-bit
// outputs, B with one unit stride, K within the exact float32 range.
static bool f6_route(int64_t M, int64_t N, int64_t K, int out_dtype, int64_t bsp, int64_t bsn) {
  return (out_dtype == QO_DTYPE_F16 || out_dtype == QO_DTYPE_BF16) && M > 256 && N >= 1 && K >= 8 && K <= 65536 &&
         M <= INT32_MAX / 2 && N <= INT32_MAX / 2 && (bsp == 1 || bsn == 1) && !route_off(QO_ROUTE_GEMM_NO_F6);
}

template <class OT>
static void dispatch(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, const void* sa,
                     int sad, const void* sb, int sbd, void* out, int64_t ldc, const void* bias, int64_t M, int64_t N, int64_t K,
                     hipStream_t stream, bool allow_fast, void* workspace, int64_t ws_bytes) {
  using T = typename OT::T;
  if constexpr (sizeof(T) == 2) {
    if (allow_fast && workspace && (uintptr_t)workspace % 256 == 0 &&
        f6_route(M, N, K, std::is_same_v<OT, OutF16> ? QO_DTYPE_F16 : QO_DTYPE_BF16, bsp, bsn) &&
        ws_bytes >= f6_workspace_bytes(M, N, K)) {
      f6_gemm_launch<OT>(a, lda, b, bsp, bsn, sa, sad, sb, sbd, static_cast<T*>(out), ldc,
                         static_cast<const T*>(bias), M, N, K, workspace, stream);
      return;
    }
  }
  const bool b_nk = (bsp == 1);
  const bool b_kn = (bsn == 1) && !b_nk;
  const int64_t ldb = b_nk ? bsn : bsp;
  // 32-bit in-tile byte offsets of the pipelined kernels: 256 rows of A or B
  const bool fits = M <= INT32_MAX / 2 && N <= INT32_MAX / 2 && K <= 65536 && lda < (1 << 21) &&
                    ldb < (1 << 21);
  const bool aligned = ((uintptr_t)a % 16 == 0) && (lda % 4 == 0) && ((uintptr_t)b % 16 == 0) && (ldb % 4 == 0) &&
                       ((uintptr_t)out % (4 * sizeof(T)) == 0) && (ldc % 4 == 0);
  if (allow_fast && fits && aligned && (b_nk || b_kn)) {
    const int m = (int)M, n = (int)N, k = (int)K;
    // decode shapes: the skinny kernel (columns x K-slices, B streamed once)
    const bool dma_layout = b_nk || skinny_kn_dma_ok(n, k, ldb);
    if (m <= 64 && k % 128 == 0 && k > 0 && gemm_allow_skinny()) {
      launch_skinny<OT>(a, lda, b, ldb, b_nk, sa, sad, sb, sbd, out, ldc, bias, m, n, k, stream);
      return;
    }
    // Up to 256 rows over few columns (the tiled grid would fill at most 1/8
    // of the CUs, each tile streaming all of K): one skinny launch per 128
    // rows. Measured at N x K = 4096 x 14336, M = 128 / 200 / 256 / 512:
    // 26.8 / 42.0 / 51.6 / 101.6 us this way, - / 62.1 / 66.1 / 65.3 us on
    // 128 x 128 tiles, 133.7 / 137.7 / 139.0 / 138.0 us on 256-row tiles.
    // Over many columns the 128 x 128 tiles win from 65 rows (14336 x 4096,
    // M = 80 / 128: 21.1 / 24.1 us against 27.9 / 36.6 us skinny).
    const int64_t tiles = (int64_t)((m + 255) / 256) * ((n + 255) / 256);
    if (m <= 256 && dma_layout && tiles * 8 <= device_cu_count() && k % 128 == 0 && k > 0 &&
        gemm_allow_skinny()) {
      const int sa_size = sad == QO_DTYPE_F32 ? 4 : 2;
      for (int r0 = 0; r0 < m; r0 += 128)
        launch_skinny<OT>(a + (int64_t)r0 * lda, lda, b, ldb, b_nk,
                          static_cast<const char*>(sa) + (int64_t)r0 * sa_size, sad, sb, sbd,
                          reinterpret_cast<T*>(out) + (int64_t)r0 * ldc, ldc, bias, min(128, m - r0), n, k, stream);
      return;
    }
    // pipelined kernel: whole 128-deep stages; KN rows read as 16-byte column groups
    if (k % 128 == 0 && k > 0 && (b_nk || n % 4 == 0) && gemm_allow_dma()) {
      if (b_nk)
        dispatch_dma<true, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, m, n, k, stream);
      else
        dispatch_dma<false, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, m, n, k, stream);
      return;
    }
    if (b_nk)
      launch_mfma<QO_GEMM_TILE, true, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, m, n, k, stream);
    else
      launch_mfma<QO_GEMM_TILE, false, OT>(a, lda, b, ldb, sa, sad, sb, sbd, out, ldc, bias, m, n, k, stream);
    return;
  }
  launch_generic<OT>(a, lda, b, bsp, bsn, sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
}

}  // namespace qo

// QO_ROUTE_GEMM_GENERIC routes every call through the generic kernel (tests
// use it to cross-check the two).
static bool gemm_allow_fast() {
  return !qo::route_off(QO_ROUTE_GEMM_GENERIC);
}

static bool is_float_code(int d) { return d == QO_DTYPE_F32 || d == QO_DTYPE_F16 || d == QO_DTYPE_BF16; }

static int gemm_entry(const char* who, const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                      int64_t b_stride_n, const void* scale_a, int scale_a_dtype, const void* scale_b,
                      int scale_b_dtype, void* out, int out_dtype, int64_t ldc, const void* bias, int64_t M,
                      int64_t N, int64_t K, void* stream, void* workspace = nullptr, int64_t ws_bytes = 0) {
  using namespace qo;
  if (M < 0 || N < 0 || K < 0 || (K % 8) != 0) {
    qo_set_error("%s: invalid sizes M=%lld N=%lld K=%lld (K must be a multiple of 8)", who, (long long)M,
                 (long long)N, (long long)K);
    return QO_ERR_SHAPE;
  }
  if (K >= (int64_t(1) << 21)) {
    qo_set_error("%s: K=%lld exceeds the exact int32 accumulation range (K < 2^21)", who, (long long)K);
    return QO_ERR_SHAPE;
  }
  if (lda < K / 8 || ldc < N) {
    qo_set_error("%s: leading dimensions too small (lda=%lld, ldc=%lld)", who, (long long)lda, (long long)ldc);
    return QO_ERR_SHAPE;
  }
  if (!is_float_code(scale_a_dtype) || !is_float_code(scale_b_dtype) || !is_float_code(out_dtype)) {
    qo_set_error("%s: unsupported dtype codes (scale_a=%d, scale_b=%d, out=%d)", who, scale_a_dtype,
                 scale_b_dtype, out_dtype);
    return QO_ERR_DTYPE;
  }
  if (M == 0 || N == 0) return QO_OK;
  if (!a || !b || !scale_a || !scale_b || !out) {
    qo_set_error("%s: NULL pointer argument", who);
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool fast = gemm_allow_fast();
  launch_begin();
  switch (out_dtype) {
    case QO_DTYPE_F16:
      dispatch<OutF16>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out, ldc,
                       bias, M, N, K, s, fast, workspace, ws_bytes);
      break;
    case QO_DTYPE_BF16:
      dispatch<OutBF16>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out,
                        ldc, bias, M, N, K, s, fast, workspace, ws_bytes);
      break;
    default:
      dispatch<OutF32>(a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b, scale_b_dtype, out, ldc,
                       bias, M, N, K, s, fast, workspace, ws_bytes);
      break;
  }
  return launch_result(who);
}

extern "C" int qo_int4_gemm(const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                            int64_t b_stride_n, const void* scale_a, int scale_a_dtype, const void* scale_b,
                            int scale_b_dtype, void* out, int out_dtype, int64_t ldc, int64_t M, int64_t N,
                            int64_t K, void* stream) {
  return gemm_entry("qo_int4_gemm", a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b,
                    scale_b_dtype, out, out_dtype, ldc, nullptr, M, N, K, stream);
}

extern "C" int qo_int4_gemm_bias(const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                                 int64_t b_stride_n, const void* scale_a, int scale_a_dtype, const void* scale_b,
                                 int scale_b_dtype, const void* bias, void* out, int out_dtype, int64_t ldc,
                                 int64_t M, int64_t N, int64_t K, void* stream) {
  if (!bias && M > 0 && N > 0) {
    qo_set_error("qo_int4_gemm_bias: NULL bias (use qo_int4_gemm for no bias)");
    return QO_ERR_NULL_POINTER;
  }
  return gemm_entry("qo_int4_gemm_bias", a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b,
                    scale_b_dtype, out, out_dtype, ldc, bias, M, N, K, stream);
}

extern "C" int qo_int4_gemm_ws(const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                               int64_t b_stride_n, const void* scale_a, int scale_a_dtype, const void* scale_b,
                               int scale_b_dtype, const void* bias, void* out, int out_dtype, int64_t ldc, int64_t M,
                               int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_entry("qo_int4_gemm_ws", a, lda, b, b_stride_p, b_stride_n, scale_a, scale_a_dtype, scale_b,
                    scale_b_dtype, out, out_dtype, ldc, bias, M, N, K, stream, workspace, workspace_bytes);
}

extern "C" int64_t qo_int4_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype) {
  // sized for either B layout (the route also needs one unit stride of B)
  if (!gemm_allow_fast() || K % 8 != 0 || !qo::f6_route(M, N, K, out_dtype, 1, 0)) return 0;
  return qo::f6_workspace_bytes(M, N, K);
}

// Checks shared by the two halves of the FP6 route.
static int f6_check(const char* who, int64_t M, int64_t N, int64_t K, const void* workspace, int64_t ws_bytes) {
  if (M < 1 || N < 1 || K < 8 || K % 8 != 0 || K > 65536 || M > INT32_MAX / 2 || N > INT32_MAX / 2) {
    qo_set_error("%s: sizes M=%lld N=%lld K=%lld outside the FP6 route (M, N >= 1, K a multiple of 8 in 8 .. 65536)",
                 who, (long long)M, (long long)N, (long long)K);
    return QO_ERR_SHAPE;
  }
  if (!workspace) {
    qo_set_error("%s: NULL workspace", who);
    return QO_ERR_NULL_POINTER;
  }
  if ((uintptr_t)workspace % 256 != 0 || ws_bytes < qo::f6_workspace_bytes(M, N, K)) {
    qo_set_error("%s: workspace not 256-byte aligned or smaller than %lld bytes", who,
                 (long long)qo::f6_workspace_bytes(M, N, K));
    return QO_ERR_SHAPE;
  }
  return QO_OK;
}

extern "C" int qo_int4_gemm_f6_prepare(const int32_t* a, int64_t lda, const int32_t* b, int64_t b_stride_p,
                                       int64_t b_stride_n, int64_t M, int64_t N, int64_t K, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  const char* who = "qo_int4_gemm_f6_prepare";
  const int st = f6_check(who, M, N, K, workspace, workspace_bytes);
  if (st != QO_OK) return st;
  if (a && lda < K / 8) {
    qo_set_error("%s: lda=%lld below K/8", who, (long long)lda);
    return QO_ERR_SHAPE;
  }
  if (b && b_stride_p != 1 && b_stride_n != 1) {
    qo_set_error("%s: B needs a unit stride (row-major [K/8, N] or the W.t() view)", who);
    return QO_ERR_SHAPE;
  }
  qo::launch_begin();
  qo::f6_prepare(a, lda, b, b_stride_p, b_stride_n, M, N, K, workspace, reinterpret_cast<hipStream_t>(stream));
  return qo::launch_result(who);
}

extern "C" int qo_int4_gemm_f6_run(const void* scale_a, int scale_a_dtype, const void* scale_b, int scale_b_dtype,
                                   const void* bias, void* out, int out_dtype, int64_t ldc, int64_t M, int64_t N,
                                   int64_t K, const void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace qo;
  const char* who = "qo_int4_gemm_f6_run";
  const int st = f6_check(who, M, N, K, workspace, workspace_bytes);
  if (st != QO_OK) return st;
  if (!is_float_code(scale_a_dtype) || !is_float_code(scale_b_dtype) ||
      (out_dtype != QO_DTYPE_F16 && out_dtype != QO_DTYPE_BF16)) {
    qo_set_error("%s: unsupported dtype codes (scale_a=%d, scale_b=%d, out=%d; out must be F16 or BF16)", who,
                 scale_a_dtype, scale_b_dtype, out_dtype);
    return QO_ERR_DTYPE;
  }
  if (ldc < N) {
    qo_set_error("%s: ldc=%lld below N", who, (long long)ldc);
    return QO_ERR_SHAPE;
  }
  if (!scale_a || !scale_b || !out) {
    qo_set_error("%s: NULL pointer argument", who);
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_begin();
  if (out_dtype == QO_DTYPE_F16)
    f6_run<OutF16>(scale_a, scale_a_dtype, scale_b, scale_b_dtype, static_cast<_Float16*>(out), ldc,
                   static_cast<const _Float16*>(bias), M, N, K, workspace, s);
  else
    f6_run<OutBF16>(scale_a, scale_a_dtype, scale_b, scale_b_dtype, static_cast<__bf16*>(out), ldc,
                    static_cast<const __bf16*>(bias), M, N, K, workspace, s);
  return launch_result(who);
}

extern "C" int64_t qo_int4_gemm_f6_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 8 || K > 65536) return 0;
  return qo::f6_workspace_bytes(M, N, K);
}

extern "C" int64_t qo_int4_gemm_f6_operand_bytes(int64_t rows, int64_t K) {
  if (rows < 1 || K < 8 || K > 65536) return 0;
  return qo::f6_operand_bytes(rows, K);
}

extern "C" int qo_int4_gemm_f6_convert(const int32_t* src, int64_t row_stride, int64_t word_stride, int64_t rows,
                                       int64_t K, void* dst, int64_t dst_bytes, void* stream) {
  const char* who = "qo_int4_gemm_f6_convert";
  if (rows < 1 || K < 8 || K % 8 != 0 || K > 65536 || rows > INT32_MAX / 2) {
    qo_set_error("%s: sizes rows=%lld K=%lld outside the FP6 route (K a multiple of 8 in 8 .. 65536)", who,
                 (long long)rows, (long long)K);
    return QO_ERR_SHAPE;
  }
  if (!src || !dst) {
    qo_set_error("%s: NULL pointer argument", who);
    return QO_ERR_NULL_POINTER;
  }
  if ((word_stride != 1 && row_stride != 1) || (word_stride == 1 && rows > 1 && row_stride < K / 8) ||
      (row_stride == 1 && word_stride != 1 && word_stride < rows) || (uintptr_t)dst % 256 != 0 ||
      dst_bytes < qo::f6_operand_bytes(rows, K)) {
    qo_set_error("%s: strides (%lld, %lld) need a unit stride and no overlap; dst 256-byte aligned, %lld bytes", who,
                 (long long)row_stride, (long long)word_stride, (long long)qo::f6_operand_bytes(rows, K));
    return QO_ERR_SHAPE;
  }
  qo::launch_begin();
  qo::f6_convert_operand(src, row_stride, word_stride, rows, K, dst, reinterpret_cast<hipStream_t>(stream));
  return qo::launch_result(who);
}

extern "C" int qo_int4_gemm_f6_run2(const void* a6, int64_t a6_bytes, const void* b6, int64_t b6_bytes,
                                    const void* scale_a, int scale_a_dtype, const void* scale_b, int scale_b_dtype,
                                    const void* bias, void* out, int out_dtype, int64_t ldc, int64_t M, int64_t N,
                                    int64_t K, void* stream) {
  using namespace qo;
  const char* who = "qo_int4_gemm_f6_run2";
  if (M < 1 || N < 1 || K < 8 || K % 8 != 0 || K > 65536 || M > INT32_MAX / 2 || N > INT32_MAX / 2) {
    qo_set_error("%s: sizes M=%lld N=%lld K=%lld outside the FP6 route", who, (long long)M, (long long)N,
                 (long long)K);
    return QO_ERR_SHAPE;
  }
  if (!a6 || !b6 || !scale_a || !scale_b || !out) {
    qo_set_error("%s: NULL pointer argument", who);
    return QO_ERR_NULL_POINTER;
  }
  if (a6_bytes < f6_operand_bytes(M, K) || b6_bytes < f6_operand_bytes(N, K) || ldc < N) {
    qo_set_error("%s: operand buffers below %lld / %lld bytes or ldc below N", who,
                 (long long)f6_operand_bytes(M, K), (long long)f6_operand_bytes(N, K));
    return QO_ERR_SHAPE;
  }
  if ((uintptr_t)a6 % 256 != 0 || (uintptr_t)b6 % 256 != 0) {
    qo_set_error("%s: operand buffers must be 256-byte aligned (as qo_int4_gemm_f6_convert writes them)", who);
    return QO_ERR_SHAPE;
  }
  if (!is_float_code(scale_a_dtype) || !is_float_code(scale_b_dtype) ||
      (out_dtype != QO_DTYPE_F16 && out_dtype != QO_DTYPE_BF16)) {
    qo_set_error("%s: unsupported dtype codes (scale_a=%d, scale_b=%d, out=%d; out must be F16 or BF16)", who,
                 scale_a_dtype, scale_b_dtype, out_dtype);
    return QO_ERR_DTYPE;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_begin();
  if (out_dtype == QO_DTYPE_F16)
    f6_run2<OutF16>(a6, b6, scale_a, scale_a_dtype, scale_b, scale_b_dtype, static_cast<_Float16*>(out), ldc,
                    static_cast<const _Float16*>(bias), M, N, K, s);
  else
    f6_run2<OutBF16>(a6, b6, scale_a, scale_a_dtype, scale_b, scale_b_dtype, static_cast<__bf16*>(out), ldc,
                     static_cast<const __bf16*>(bias), M, N, K, s);
  return launch_result(who);
}
