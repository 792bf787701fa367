// The W4A4 GEMM on gfx950's FP6 matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4
// with both operands in FP6 e2m3), for the large tiled shapes.
//
// Why it is exact: an int4 code q (-8 .. 7) divided by 8 is an FP6 e2m3 value
// (e2m3 with exponent bias 1 holds m / 8 for every 5-bit magnitude field
// m <= 15: subnormals 0 .. 7/8 and the first normal binade 1 .. 15/8), so the
// FP6 code of q / 8 is simply sign-magnitude: sign in bit 5, |q| <= 8 in bits
// 0 .. 3. With both operands' block scales set to 2^3 (e8m0 exponent 130) the
// matrix core multiplies q_a * q_b exactly and accumulates in float32; every
// partial sum is an integer of magnitude at most 64 K < 2^24 (K <= 65536 on
// this route), so it is exact and equals float(int32 accumulator) of the
// integer kernels, and the epilogue (float(acc) * sa) * sb gives the same bits.
//
// Why it pays: the FP6 MFMA does 16 x 16 x 128 in the issue time of the int8
// 16 x 16 x 64, and draws less power per operation (the matrix cores run the
// board at its power limit on these shapes).
//
// Two launches: f6_convert_kernel turns the packed int4 operands (A rows, and
// B in either layout) into FP6 fragment blocks in a workspace, once per
// element; gemm_f6_pp2 then streams those blocks through an LDS-DMA ring and
// does no per-element work before its MFMAs.
//
// Operand layout (fragment pairs): the MFMA's fragment of 16 rows x 128 codes
// gives lane l = r % 16 + 16 g row r's codes k = 128 kb + 32 g + j,
// j = 0 .. 31, as a 192-bit value with code j in bits 6 j .. 6 j + 5. Two
// fragments of 32 consecutive rows (16-row groups 2 p and 2 p + 1) are stored
// together in 3072 bytes: lane l's two values (group 2 p's in bits 0 .. 191,
// group 2 p + 1's in bits 192 .. 383) as three 16-byte pieces t = 0, 1, 2 at
// byte t * 1024 + 16 l. A wave reads each piece of all 64 lanes as 1 KiB of
// contiguous LDS with ds_read_b128, the LDS read with the highest bandwidth
// (8- and 12-byte reads move a half to two thirds as much per clock), and the
// two operands land in registers 0 .. 5 and 6 .. 11 of the 12 read. Operand X
// (R rows: A's M rows or B's N columns) is stored as pair rows of
// kblocks = ceil(K / 128) pairs: pair (r / 32, kb) at
// ((r / 32) * kblocks + kb) * 3072. Rows past R and codes past K are FP6 zeros.
#include <algorithm>
#include <type_traits>

#include "int4_common.h"

namespace qo {

namespace {

constexpr int kF6Pair = 3072;   // bytes of one fragment pair (32 rows x 128 codes)

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Eight offset codes (nibble i = q_i + 8) -> the FP6 e2m3 codes of q_i / 8,
// code i in bits 6 i .. 6 i + 5 (48 bits).
__device__ inline uint64_t f6_codes8(uint32_t w) {
  const uint32_t x = w ^ 0x88888888u;                // q as 4-bit two's complement
  const uint32_t neg = x & 0x88888888u;              // bit 3 of each negative q
  const uint32_t mask = neg | (neg - (neg >> 3));    // 0xF in each negative q's nibble
  const uint32_t mag = (x ^ mask) + (neg >> 3);      // |q| (0 .. 8), no carry between nibbles
  // nibble i from bits 4 i .. 4 i + 3 to bits 6 i .. 6 i + 3
  auto spread = [](uint32_t v) -> uint64_t {
    uint64_t d = (uint64_t)(v & 0xFFFFu) | ((uint64_t)(v & 0xFFFF0000u) << 8);
    d = (d & 0x00000000FF0000FFull) | ((d & 0x000000FF0000FF00ull) << 4);
    d = (d & 0x000000F00F00F00Full) | ((d & 0x00000F00F00F00F0ull) << 2);
    return d;
  };
  return spread(mag) | (spread(neg) << 2);   // sign: bit 4 i + 3 -> 6 i + 3 -> 6 i + 5
}

// One operand to convert: word p (codes 8 p .. 8 p + 7) of row r at
// src[r * ld + p] (row_major) or src[p * ld + r].
struct F6Job {
  const int32_t* src;
  int64_t ld;
  uint8_t* dst;
  int rows, kw, kblocks;   // rows, packed words per row (K / 8), ceil(K / 128)
  int row_major, vec;      // vec: 16-byte loads of a row's words (row_major, src and ld aligned)
  int blocks;              // workgroups of this job
};

// The 192-bit lane value of four packed words (codes 8 t + i in word t):
// three 64-bit pieces.
struct F6Lane {
  uint64_t u0, u1, u2;
};
__device__ inline F6Lane f6_lane(const uint32_t (&w)[4]) {
  const uint64_t d0 = f6_codes8(w[0]), d1 = f6_codes8(w[1]), d2 = f6_codes8(w[2]), d3 = f6_codes8(w[3]);
  return F6Lane{d0 | (d1 << 48), (d1 >> 16) | (d2 << 32), (d2 >> 32) | (d3 << 16)};
}

// 256 threads; a thread converts lane l = r % 16 + 16 g of one pair (32 rows,
// one k-block): rows r and r + 16, 32 codes each, and writes the pair's three
// whole 16-byte pieces of that lane. Row-major sources: a wave is one pair and
// k-block (reads: 32 rows x 64 contiguous bytes), a workgroup 4 consecutive
// k-blocks of that pair. Column sources ([K/8, N]): a wave is k-group g of
// 4 consecutive pairs (reads: 4 x 2 runs of 64 bytes per packed row), a
// workgroup the 4 k-groups of one k-block. Rows past R read as code 8
// (q = 0), so every pair is written whole.
__global__ void __launch_bounds__(256) f6_convert_kernel(F6Job j0, F6Job j1) {
  const bool second = (int)blockIdx.x >= j0.blocks;
  const F6Job j = second ? j1 : j0;
  const int b = second ? (int)blockIdx.x - j0.blocks : (int)blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pairs = (j.rows + 31) >> 5;
  int pr, kb, g, rr;
  if (j.row_major) {
    const int kq = (j.kblocks + 3) >> 2;
    kb = (b % kq) * 4 + wave;
    if (kb >= j.kblocks) return;
    pr = b / kq;
    rr = lane & 15;
    g = lane >> 4;
  } else {
    const int pq = (pairs + 3) >> 2;
    kb = b / pq;
    pr = (b % pq) * 4 + (lane >> 4);
    if (pr >= pairs) return;
    rr = lane & 15;
    g = wave;
  }
  const int p0 = kb * 16 + g * 4;
  const int r0 = pr * 32 + rr, r1 = r0 + 16;
  uint32_t w0[4], w1[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) w0[t] = w1[t] = 0x88888888u;   // code 8: q = 0
  if (j.row_major) {
    auto row = [&](int r, uint32_t (&w)[4]) {
      if (r >= j.rows) return;
      const int32_t* src = j.src + (int64_t)r * j.ld + p0;
      if (j.vec && p0 + 4 <= j.kw) {
        const v4i v = *reinterpret_cast<const v4i*>(src);
#pragma unroll
        for (int t = 0; t < 4; ++t) w[t] = (uint32_t)v[t];
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (p0 + t < j.kw) w[t] = (uint32_t)src[t];
      }
    };
    row(r0, w0);
    row(r1, w1);
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (p0 + t >= j.kw) continue;
      const int32_t* src = j.src + (int64_t)(p0 + t) * j.ld;
      if (r0 < j.rows) w0[t] = (uint32_t)src[r0];
      if (r1 < j.rows) w1[t] = (uint32_t)src[r1];
    }
  }
  const F6Lane x = f6_lane(w0), y = f6_lane(w1);
  uint8_t* base = j.dst + ((int64_t)pr * j.kblocks + kb) * kF6Pair + 16 * (rr + 16 * g);
  typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u64x2*>(base) = u64x2{x.u0, x.u1};          // bits 0 .. 127
  *reinterpret_cast<u64x2*>(base + 1024) = u64x2{x.u2, y.u0};   // bits 128 .. 255
  *reinterpret_cast<u64x2*>(base + 2048) = u64x2{y.u1, y.u2};   // bits 256 .. 383
}

// ---------------------------------------------------------------------------
// gemm_f6_pp2: BM x BN tiles (BM = 256; BN = 224 or 256), eight waves as
// 4 x 2, each wave 64 x BN/2 of the output in FM x FN blocks of 16 x 16; the
// ping-pong of the integer kernel gemm_i4_pp2 (waves 0-3 and 4-7 alternate,
// one slot apart, between a load slot, the stage's LDS reads and the copies
// of stage t + 2, and a compute slot, its MFMAs, with a workgroup barrier
// between slots) on a three-stage ring of FP6 fragment pairs (45 KiB per
// stage at BN = 224). Stage t holds k-block t of the tile's 8 A pairs and
// BN / 32 B pairs; LDS-DMA instruction i of a stage copies its bytes
// 1024 i .. 1024 i + 1023 (the A part ends on a 1 KiB boundary).
// A wave reads its 2 A pairs and its B pairs as whole 16-byte pieces; at
// BN = 224 a wave's 7 column groups are 3 pairs and one half of the pair it
// shares with the other column wave (wave column 0: groups 0 .. 6, the
// shared pair's first half, pieces 0 and 1's low 8 bytes; wave column 1:
// groups 7 .. 13, the shared pair's second half, piece 1's high 8 bytes
// and piece 2).
// ---------------------------------------------------------------------------
template <int BM, int BN>
struct F6Stage {
  static constexpr int A_BYTES = BM / 32 * kF6Pair;
  static constexpr int BYTES = (BM + BN) / 32 * kF6Pair;
  static constexpr int A_DMA = A_BYTES / 1024;
  static constexpr int DMA = BYTES / 1024;
  static_assert(BM % 32 == 0 && BN % 32 == 0, "whole pairs");
};

template <int BM, int BN, class OT>
__global__ void __launch_bounds__(512, 1)
gemm_f6_pp2(const uint8_t* __restrict__ a6, const uint8_t* __restrict__ b6, int pr_a, int pr_b, int nk,
            const void* __restrict__ sa, int sad, const void* __restrict__ sb, int sbd,
            typename OT::T* __restrict__ out, int64_t ldc, const typename OT::T* __restrict__ bias, int M, int N,
            int tiles_m) {
  constexpr int WGM = 4, WGN = 2, W = 8, STAGES = 3;
  using S = F6Stage<BM, BN>;
  using T = typename OT::T;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int PER = (S::DMA + W - 1) / W;
  static_assert(BM == 256 && FM == 4 && (FN == 7 || FN == 8), "256 x 224 or 256 x 256 tiles, 4 x 2 waves");
  static_assert(sizeof(T) == 2, "16-bit outputs (staged epilogue)");
  static_assert(S::A_DMA % W == 0, "copies 0 .. A_DMA / W - 1 of every wave are A's");
  static_assert(PER * (STAGES - 1) < 64, "vmcnt range");
  constexpr int TA = S::A_DMA / W;
  constexpr int C_PITCH = BN * 2 + 16;
  constexpr int RING = STAGES * S::BYTES, CTILE = BM * C_PITCH;
  __shared__ __align__(16) unsigned char ring[RING > CTILE ? RING : CTILE];
  __shared__ __align__(16) float s_sa[BM];
  __shared__ __align__(16) float s_sb[BN];
  __shared__ __align__(16) float s_bias[BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;   // wave-uniform (scalar branches on wn)
  const int li = lane & 15, lg = lane >> 4;
  const bool grp1 = __builtin_amdgcn_readfirstlane(wave) >= W / 2;

  // Tile order as gemm_i4_pp2: each XCD a contiguous run of tiles, grouped
  // 4 row tiles x every column tile.
  const int nblk = gridDim.x;
  int pid = blockIdx.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  constexpr int GM = 4;
  const int tiles_n = (N + BN - 1) / BN;
  const int g = pid / (GM * tiles_n), w = pid % (GM * tiles_n);
  const int gm = min(GM, tiles_m - g * GM);
  const int tm = g * GM + w % gm, tn = w / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  // Copy t of this wave is stage instruction i = wave + 8 t (spare slots
  // repeat the last); lane u's 16 bytes are the stage's bytes 1024 i + 16 u,
  // from pair f = that / 3072 of the tile's row (column) pairs, clamped to
  // the operand's last pair (those rows only feed accumulators that are never
  // stored).
  const int64_t prs = (int64_t)nk * kF6Pair;   // bytes per pair row
  const uint8_t* const a_base = a6 + (int64_t)(m0 >> 5) * prs;
  const uint8_t* const b_base = b6 + (int64_t)(n0 >> 5) * prs;
  uint32_t dst[PER], voff[PER];
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    int i = __builtin_amdgcn_readfirstlane(wave) + W * t;
    i = i < S::DMA ? i : S::DMA - 1;
    const int o = 1024 * i + 16 * lane;
    if (t < TA) {
      const int f = min(o / kF6Pair, pr_a - 1 - (m0 >> 5));
      voff[t] = (uint32_t)(f * prs + o % kF6Pair);
    } else {
      const int ob = o - S::A_BYTES;
      const int f = min(ob / kF6Pair, pr_b - 1 - (n0 >> 5));
      voff[t] = (uint32_t)(f * prs + ob % kF6Pair);
    }
    dst[t] = __builtin_amdgcn_readfirstlane((uint32_t)(1024 * i));
  }
  auto issue = [&](int ks, auto bufc) {
    constexpr uint32_t BUF = decltype(bufc)::value * S::BYTES;
    const uint32_t base = lds_addr(ring) + BUF;
    const uint8_t* ab = a_base + (int64_t)ks * kF6Pair;
    const uint8_t* bb = b_base + (int64_t)ks * kF6Pair;
#pragma unroll
    for (int t = 0; t < PER; ++t) dma16_s(voff[t], t < TA ? ab : bb, base + dst[t]);
  };

  // Operands: pairs of fragments as 12 registers (3 x 16-byte reads); the
  // MFMA takes registers 0 .. 5 (first fragment) or 6 .. 11 (second) of an
  // 8-register window.
  v16i ap[FM / 2], bp[4];
  auto piece = [](const unsigned char* p) -> v4i { return *reinterpret_cast<const v4i*>(p); };
  auto load_regs = [&](auto bufc) {
    const unsigned char* base = ring + decltype(bufc)::value * S::BYTES + 16 * lane;
#pragma unroll
    for (int q = 0; q < FM / 2; ++q) {
      const unsigned char* pp = base + (wm * (FM / 2) + q) * kF6Pair;
      const v4i x0 = piece(pp), x1 = piece(pp + 1024), x2 = piece(pp + 2048);
      ap[q] = v16i{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3], x2[0], x2[1], x2[2], x2[3], 0, 0, 0, 0};
    }
    const unsigned char* bbase = base + S::A_BYTES;
    if constexpr (FN == 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned char* pp = bbase + (wn * 4 + q) * kF6Pair;
        const v4i x0 = piece(pp), x1 = piece(pp + 1024), x2 = piece(pp + 2048);
        bp[q] = v16i{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3], x2[0], x2[1], x2[2], x2[3], 0, 0, 0, 0};
      }
    } else if (wn == 0) {   // groups 0 .. 5 = pairs 0 .. 2, group 6 = first half of pair 3
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const unsigned char* pp = bbase + q * kF6Pair;
        const v4i x0 = piece(pp), x1 = piece(pp + 1024), x2 = piece(pp + 2048);
        bp[q] = v16i{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3], x2[0], x2[1], x2[2], x2[3], 0, 0, 0, 0};
      }
      const unsigned char* pp = bbase + 3 * kF6Pair;
      const v4i x0 = piece(pp);
      const v2i x1 = *reinterpret_cast<const v2i*>(pp + 1024);
      bp[3] = v16i{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    } else {                // groups 8 .. 13 = pairs 4 .. 6, group 7 = second half of pair 3
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const unsigned char* qp = bbase + (4 + q) * kF6Pair;
        const v4i x0 = piece(qp), y1 = piece(qp + 1024), y2 = piece(qp + 2048);
        bp[q] = v16i{x0[0], x0[1], x0[2], x0[3], y1[0], y1[1], y1[2], y1[3], y2[0], y2[1], y2[2], y2[3], 0, 0, 0, 0};
      }
      const unsigned char* pp = bbase + 3 * kF6Pair;
      const v2i x1 = *reinterpret_cast<const v2i*>(pp + 1024 + 8);
      const v4i x2 = piece(pp + 2048);
      bp[3] = v16i{x1[0], x1[1], x2[0], x2[1], x2[2], x2[3], 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto lo = [](const v16i& v) -> v8i { return __builtin_shufflevector(v, v, 0, 1, 2, 3, 4, 5, 6, 7); };
  auto hi = [](const v16i& v) -> v8i { return __builtin_shufflevector(v, v, 6, 7, 8, 9, 10, 11, 12, 13); };
  // Operand slot j: registers of both wave columns alike (no per-wave
  // selects in the MFMA sequence). A slot i: rows 16 i .. of the wave. B slot
  // j: pairs bp[0 .. 2] then bp[3]'s single fragment; at BN = 224 that is
  // column group j of wave column 0, and group (j + 1) % 7 of wave column 1
  // (whose bp[3] holds its first group), which only the epilogue's column
  // map (bcol) sees.
  auto afrag = [&](int i) -> v8i { return (i & 1) ? hi(ap[i >> 1]) : lo(ap[i >> 1]); };
  auto bfrag = [&](int j) -> v8i { return (j & 1) ? hi(bp[j >> 1]) : lo(bp[j >> 1]); };
  auto bcol = [&](int j) -> int { return (FN == 8 || wn == 0) ? j : (j + 1) % 7; };
  auto bar = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // The tile's scales and bias as raw bits, requested by group 0 before the
  // first copies and converted in the last load slot.
  auto raw16 = [](const void* p, int64_t i) -> uint32_t { return reinterpret_cast<const uint16_t*>(p)[i]; };
  auto raw32 = [](const void* p, int64_t i) -> uint32_t { return reinterpret_cast<const uint32_t*>(p)[i]; };
  uint32_t rsa = 0, rsb = 0, rbias = 0;
  if (tid < BM) {
    const int64_t i = min(m0 + tid, M - 1);
    rsa = sad == QO_DTYPE_F32 ? raw32(sa, i) : raw16(sa, i);
    if (tid < BN) {
      const int64_t jn = min(n0 + tid, N - 1);
      rsb = sbd == QO_DTYPE_F32 ? raw32(sb, jn) : raw16(sb, jn);
      if (bias) rbias = raw16(bias, jn);
    }
  }
  issue(0, std::integral_constant<int, 0>{});
  issue(min(1, nk - 1), std::integral_constant<int, 1>{});
  gemm_wait_vmcnt<PER>();
  lds_barrier();

  if (grp1) bar();
  auto phase = [&](int t, auto bufc) {
    constexpr int J = decltype(bufc)::value;
    load_regs(bufc);
    if (t + 2 < nk) issue(t + 2, std::integral_constant<int, (J + 2) % STAGES>{});
    // wait for this wave's copies of stage t + 1 (stage t + 2 may stay in flight)
    gemm_wait_groups<PER, 1>(nk - 2 - t);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    if (t == nk - 1 && !grp1) {
      asm volatile("" : "+v"(rsa), "+v"(rsb), "+v"(rbias));
      if (tid < BM) s_sa[tid] = scale_from_bits(rsa, sad);
      if (tid < BN) {
        s_sb[tid] = scale_from_bits(rsb, sbd);
        s_bias[tid] = (float)__builtin_bit_cast(T, (uint16_t)rbias);
      }
    }
    bar();
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const v8i fb = bfrag(j);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb, afrag(i), acc[i][j], 2, 2, 0, 130, 0, 130);
    }
    bar();
  };
  for (int s = 0; s < nk; s += 3) {
    phase(s, std::integral_constant<int, 0>{});
    if (s + 1 < nk) phase(s + 1, std::integral_constant<int, 1>{});
    if (s + 2 < nk) phase(s + 2, std::integral_constant<int, 2>{});
  }

  // Epilogue as gemm_i4_pp2's: group 0 stages its rows while group 1 runs its
  // last compute slot, then copies them out while group 1 stages its rows.
  // acc[i][j][r] is row wm * WM + 16 i + li, column wn * WN + 16 bcol(j) + 4 lg + r;
  // its value is the integer sum itself (exact in float32).
  const float* ssa = s_sa + wm * WM;
  const float* ssb = s_sb + wn * WN;
  const float* sbias = bias ? s_bias + wn * WN : nullptr;
  unsigned char* const c_half = ring + (grp1 ? (BM / 2) * C_PITCH : 0);
  unsigned char* const c_wave = ring + wm * WM * C_PITCH + wn * WN * 2;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const float sav = ssa[16 * i + li];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int c = 16 * bcol(j) + 4 * lg;
      const v4f sbv = *reinterpret_cast<const v4f*>(ssb + c);
      T v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = OT::cvt((acc[i][j][r] * sav) * sbv[r]);
      if (sbias) {
        const v4f bb = *reinterpret_cast<const v4f*>(sbias + c);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = OT::cvt((float)v[r] + bb[r]);
      }
      *reinterpret_cast<v2i*>(c_wave + (16 * i + li) * C_PITCH + 2 * c) =
          v2i{(int)(out_bits<OT>(v[0]) | out_bits<OT>(v[1]) << 16), (int)(out_bits<OT>(v[2]) | out_bits<OT>(v[3]) << 16)};
    }
  }
  lds_barrier();
  // non-temporal: measured 140.6 -> 134.5 us at config 4 (no change at config 5's 256 tiles)
  copy_out_c<BM / 2, BN, 256, OT, true>(c_half, C_PITCH, out, ldc, M, N, m0 + (grp1 ? BM / 2 : 0), n0, tid & 255);
  if (!grp1) bar();
}

// Job for operand rows [R, K] given by (src, strides): row r's word p at
// src[r * s_r + p * s_p], with s_p == 1 (row-major) or s_r == 1.
F6Job f6_job(const int32_t* src, int64_t s_r, int64_t s_p, int64_t R, int64_t K, uint8_t* dst) {
  F6Job j{};
  j.src = src;
  j.dst = dst;
  j.rows = (int)R;
  j.kw = (int)(K / 8);
  j.kblocks = (int)((K + 127) / 128);
  j.row_major = s_p == 1 ? 1 : 0;
  j.ld = j.row_major ? s_r : s_p;
  j.vec = j.row_major && (uintptr_t)src % 16 == 0 && s_r % 4 == 0;
  // row-major: every pair x groups of 4 k-blocks; columns: groups of 4 pairs x every k-block
  const int64_t pairs = (R + 31) / 32;
  j.blocks = j.row_major ? (int)(pairs * ((j.kblocks + 3) / 4)) : (int)((pairs + 3) / 4 * j.kblocks);
  return j;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace

int64_t f6_operand_bytes(int64_t rows, int64_t K) { return (rows + 31) / 32 * ((K + 127) / 128) * kF6Pair; }

int64_t f6_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return align256(f6_operand_bytes(M, K)) + f6_operand_bytes(N, K);
}

namespace {
// column tile: 224 or 256, whichever leaves fewer idle CU slots over the rounds
bool f6_wide(int64_t M, int64_t N) {
  const int cus = device_cu_count();
  const int64_t tiles_m = (M + 255) / 256;
  const int64_t t224 = tiles_m * ((N + 223) / 224), t256 = tiles_m * ((N + 255) / 256);
  return ((t256 + cus - 1) / cus) * 256 < ((t224 + cus - 1) / cus) * 224;
}
}  // namespace

void f6_prepare(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, int64_t M, int64_t N,
                int64_t K, void* workspace, hipStream_t stream) {
  uint8_t* a6 = static_cast<uint8_t*>(workspace);
  uint8_t* b6 = a6 + align256(f6_operand_bytes(M, K));
  F6Job ja{}, jb{};
  if (a) ja = f6_job(a, lda, 1, M, K, a6);
  // B's columns are the operand's rows: word p of column n at b[p * bsp + n * bsn]
  if (b) jb = f6_job(b, bsn, bsp, N, K, b6);
  if (ja.blocks + jb.blocks > 0) launch(f6_convert_kernel, dim3(ja.blocks + jb.blocks), dim3(256), 0, stream, ja, jb);
}

void f6_convert_operand(const int32_t* src, int64_t s_r, int64_t s_p, int64_t R, int64_t K, void* dst,
                        hipStream_t stream) {
  const F6Job j = f6_job(src, s_r, s_p, R, K, static_cast<uint8_t*>(dst));
  if (j.blocks > 0) launch(f6_convert_kernel, dim3(j.blocks), dim3(256), 0, stream, j, F6Job{});
}

template <class OT>
void f6_run(const void* sa, int sad, const void* sb, int sbd, typename OT::T* out, int64_t ldc,
            const typename OT::T* bias, int64_t M, int64_t N, int64_t K, const void* workspace, hipStream_t stream) {
  const uint8_t* a6 = static_cast<const uint8_t*>(workspace);
  f6_run2<OT>(a6, a6 + align256(f6_operand_bytes(M, K)), sa, sad, sb, sbd, out, ldc, bias, M, N, K, stream);
}

template <class OT>
void f6_run2(const void* a6v, const void* b6v, const void* sa, int sad, const void* sb, int sbd, typename OT::T* out,
             int64_t ldc, const typename OT::T* bias, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  constexpr int BM = 256;
  const uint8_t* a6 = static_cast<const uint8_t*>(a6v);
  const uint8_t* b6 = static_cast<const uint8_t*>(b6v);
  const bool wide = f6_wide(M, N);
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + (wide ? 255 : 223)) / (wide ? 256 : 224));
  auto go = [&](auto kernel) {
    launch(kernel, dim3(tiles_m * tiles_n), dim3(512), 0, stream, a6, b6, (int)((M + 31) / 32), (int)((N + 31) / 32),
           (int)((K + 127) / 128), sa, sad, sb, sbd, out, ldc, bias, (int)M, (int)N, tiles_m);
  };
  if (wide) go(gemm_f6_pp2<BM, 256, OT>);
  else go(gemm_f6_pp2<BM, 224, OT>);
}

template <class OT>
void f6_gemm_launch(const int32_t* a, int64_t lda, const int32_t* b, int64_t bsp, int64_t bsn, const void* sa,
                    int sad, const void* sb, int sbd, typename OT::T* out, int64_t ldc, const typename OT::T* bias,
                    int64_t M, int64_t N, int64_t K, void* workspace, hipStream_t stream) {
  f6_prepare(a, lda, b, bsp, bsn, M, N, K, workspace, stream);
  f6_run<OT>(sa, sad, sb, sbd, out, ldc, bias, M, N, K, workspace, stream);
}

template void f6_run2<OutF16>(const void*, const void*, const void*, int, const void*, int, _Float16*, int64_t,
                              const _Float16*, int64_t, int64_t, int64_t, hipStream_t);
template void f6_run2<OutBF16>(const void*, const void*, const void*, int, const void*, int, __bf16*, int64_t,
                               const __bf16*, int64_t, int64_t, int64_t, hipStream_t);
template void f6_run<OutF16>(const void*, int, const void*, int, _Float16*, int64_t, const _Float16*, int64_t, int64_t,
                             int64_t, const void*, hipStream_t);
template void f6_run<OutBF16>(const void*, int, const void*, int, __bf16*, int64_t, const __bf16*, int64_t, int64_t,
                              int64_t, const void*, hipStream_t);
template void f6_gemm_launch<OutF16>(const int32_t*, int64_t, const int32_t*, int64_t, int64_t, const void*, int,
                                     const void*, int, _Float16*, int64_t, const _Float16*, int64_t, int64_t,
                                     int64_t, void*, hipStream_t);
template void f6_gemm_launch<OutBF16>(const int32_t*, int64_t, const int32_t*, int64_t, int64_t, const void*, int,
                                      const void*, int, __bf16*, int64_t, const __bf16*, int64_t, int64_t, int64_t,
                                      void*, hipStream_t);

}  // namespace qo
