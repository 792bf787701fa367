// Pack / unpack of int4 codes and the word transpose between the two layouts
// of a packed weight. All three are HBM-bound byte work (no MFMA). Their
// 16-byte stores are non-temporal (the output streams to memory instead of
// waiting in L2 for the write-back at the kernel's end; config 4's weight,
// same process: pack 19.7 -> 18.8 us, unpack 18.8 -> 14.9, transpose of full
// tiles 12.7 -> 9.7).
//
// * pack:   int8 codes [rows, F] -> int32 words [rows, F/8],
//           word p = sum_i ((q[8p + i] + 8) mod 256) << 4i (mod 2^32)
//           (pack_int4_to_int32, int4_matmul/ops.py:23-45: the int8 add, the
//           uint8 cast and the int32 shifted sum wrap exactly like this, so
//           out-of-range codes pack the same way too).
// * unpack: int32 words [rows, W] -> int8 codes [rows, 8W],
//           q[8p + i] = ((w >> 4i) & 0xF) - 8 (unpack_int32_to_int4, :48-66).
// * transpose of 32-bit words [R, C] -> [C, R]: a packed weight stored
//           [K/8, N] (word [p, n] holds k = 8p .. 8p+7 of column n) and the
//           same weight stored [N, K/8] hold identical words, so converting
//           one layout to the other is a plain word transpose
//           (examples/int4_matmul_benchmark.py:21-22 builds the first as
//           pack(b.T).T).
#include "common.h"

namespace qo {

// Nibble of one code: the low 8 bits of q + 8, as the reference's uint8 cast
// leaves them (any int8 q).
__device__ inline uint32_t pack_word(uint32_t c0, uint32_t c1) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w += (((c0 >> (8 * i)) + 8u) & 0xFFu) << (4 * i);
    w += (((c1 >> (8 * i)) + 8u) & 0xFFu) << (4 * (4 + i));
  }
  return w;
}

// 16 codes (two words) per thread; rows of `words_per_row` words.
__global__ void __launch_bounds__(256)
pack_kernel_v16(const int8_t* __restrict__ codes, int64_t codes_ld, int64_t rows, int64_t pairs_per_row,
                int32_t* __restrict__ out, int64_t out_ld) {
  const int64_t total = rows * pairs_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / pairs_per_row, p = i - r * pairs_per_row;
    const v4i c = *reinterpret_cast<const v4i*>(codes + r * codes_ld + 16 * p);
    const v2i w = {(int)pack_word((uint32_t)c[0], (uint32_t)c[1]), (int)pack_word((uint32_t)c[2], (uint32_t)c[3])};
    __builtin_nontemporal_store(w, reinterpret_cast<v2i*>(out + r * out_ld + 2 * p));
  }
}

// One word per thread, byte loads (any alignment).
__global__ void __launch_bounds__(256)
pack_kernel_any(const int8_t* __restrict__ codes, int64_t codes_ld, int64_t rows, int64_t words_per_row,
                int32_t* __restrict__ out, int64_t out_ld) {
  const int64_t total = rows * words_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / words_per_row, p = i - r * words_per_row;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(codes + r * codes_ld + 8 * p);
    uint32_t c0 = 0, c1 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c0 |= (uint32_t)src[j] << (8 * j);
      c1 |= (uint32_t)src[4 + j] << (8 * j);
    }
    out[r * out_ld + p] = (int)pack_word(c0, c1);
  }
}

// Four codes of a word's nibbles n..n+3 as bytes: each nibble moved to its own
// byte, then (b + 0x78) ^ 0x80 per byte = b - 8 in two's complement (b <= 15,
// so the add never carries out of a byte).
__device__ inline uint32_t unpack4(uint32_t h) {
  const uint32_t b = (h & 0xFu) | ((h & 0xF0u) << 4) | ((h & 0xF00u) << 8) | ((h & 0xF000u) << 12);
  return (b + 0x78787878u) ^ 0x80808080u;
}

// Two words (16 codes) per thread.
__global__ void __launch_bounds__(256)
unpack_kernel_v16(const int32_t* __restrict__ words, int64_t words_ld, int64_t rows, int64_t pairs_per_row,
                  int8_t* __restrict__ out, int64_t out_ld) {
  const int64_t total = rows * pairs_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / pairs_per_row, p = i - r * pairs_per_row;
    const v2i w = *reinterpret_cast<const v2i*>(words + r * words_ld + 2 * p);
    const uint32_t w0 = (uint32_t)w[0], w1 = (uint32_t)w[1];
    const v4i c = {(int)unpack4(w0), (int)unpack4(w0 >> 16), (int)unpack4(w1), (int)unpack4(w1 >> 16)};
    __builtin_nontemporal_store(c, reinterpret_cast<v4i*>(out + r * out_ld + 16 * p));
  }
}

// One word per thread, byte stores (any alignment).
__global__ void __launch_bounds__(256)
unpack_kernel_any(const int32_t* __restrict__ words, int64_t words_ld, int64_t rows, int64_t words_per_row,
                  int8_t* __restrict__ out, int64_t out_ld) {
  const int64_t total = rows * words_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / words_per_row, p = i - r * words_per_row;
    const uint32_t w = (uint32_t)words[r * words_ld + p];
    const uint32_t lo = unpack4(w), hi = unpack4(w >> 16);
    uint8_t* dst = reinterpret_cast<uint8_t*>(out + r * out_ld + 8 * p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dst[j] = (uint8_t)(lo >> (8 * j));
      dst[4 + j] = (uint8_t)(hi >> (8 * j));
    }
  }
}

// 64 x 64 word tiles through LDS (rows padded to 65 words: the column reads
// of the second half hit 64 different banks). 256 threads: lane x of wave y
// moves column x of rows y, y + 4, ..., so every global access of a wave
// covers 256 contiguous bytes of a row.
constexpr int kTile = 64;

template <bool VEC>
__global__ void __launch_bounds__(256)
transpose_words_kernel(const int32_t* __restrict__ in, int64_t in_ld, int64_t rows, int64_t cols,
                       int32_t* __restrict__ out, int64_t out_ld, int64_t tiles_c) {
  __shared__ int32_t tile[kTile][kTile + 1];
  const int x = threadIdx.x & 63, y = threadIdx.x >> 6;
  const int64_t tr = blockIdx.x / tiles_c, tc = blockIdx.x - tr * tiles_c;
  const int64_t r0 = tr * kTile, c0 = tc * kTile;
  const bool full = r0 + kTile <= rows && c0 + kTile <= cols;
  if (VEC && full) {
    // 16-byte accesses: lane (x4, y4) = (tid % 16, tid / 16) moves words
    // 4 x4 .. 4 x4 + 3 of rows y4, y4 + 16, ... (a row of the tile is 16 lanes,
    // 256 contiguous bytes). With the 65-word row pitch both the scattered
    // writes and the column reads hit 64 different banks per wave.
    const int x4 = threadIdx.x & 15, y4 = threadIdx.x >> 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rr = y4 + 16 * k;
      const v4i v = *reinterpret_cast<const v4i*>(in + (r0 + rr) * in_ld + c0 + 4 * x4);
#pragma unroll
      for (int i = 0; i < 4; ++i) tile[rr][4 * x4 + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cc = y4 + 16 * k;
      const v4i v = {tile[4 * x4][cc], tile[4 * x4 + 1][cc], tile[4 * x4 + 2][cc], tile[4 * x4 + 3][cc]};
      __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(out + (c0 + cc) * out_ld + r0 + 4 * x4));
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < kTile / 4; ++k) {
    const int rr = y + 4 * k;
    if (full || (r0 + rr < rows && c0 + x < cols)) tile[rr][x] = in[(r0 + rr) * in_ld + c0 + x];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kTile / 4; ++k) {
    const int cc = y + 4 * k;
    if (full || (c0 + cc < cols && r0 + x < rows)) out[(c0 + cc) * out_ld + r0 + x] = tile[x][cc];
  }
}

static unsigned grid_for(int64_t items) {
  int64_t blocks = (items + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}


}  // namespace qo

extern "C" int qo_pack_int4_to_int32(const int8_t* codes, int64_t codes_ld, int64_t rows, int64_t features,
                                     int32_t* out, int64_t out_ld, void* stream) {
  using namespace qo;
  if (rows < 0 || features < 0 || features % 8 != 0 || (rows > 1 && (codes_ld < features || out_ld < features / 8))) {
    qo_set_error("qo_pack_int4_to_int32: invalid sizes rows=%lld features=%lld (features must be a multiple of 8) "
                 "codes_ld=%lld out_ld=%lld", (long long)rows, (long long)features, (long long)codes_ld,
                 (long long)out_ld);
    return QO_ERR_SHAPE;
  }
  if (rows == 0 || features == 0) return QO_OK;
  if (!codes || !out) {
    qo_set_error("qo_pack_int4_to_int32: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_begin();
  const bool vec = features % 16 == 0 && (uintptr_t)codes % 16 == 0 && (uintptr_t)out % 8 == 0 &&
                   (rows == 1 || (codes_ld % 16 == 0 && out_ld % 2 == 0));
  if (vec) {
    const int64_t pairs = features / 16;
    launch(pack_kernel_v16, dim3(grid_for(rows * pairs)), dim3(256), 0, s, codes, codes_ld, rows, pairs,
                       out, out_ld);
  } else {
    const int64_t wpr = features / 8;
    launch(pack_kernel_any, dim3(grid_for(rows * wpr)), dim3(256), 0, s, codes, codes_ld, rows, wpr, out,
                       out_ld);
  }
  return launch_result("qo_pack_int4_to_int32");
}

extern "C" int qo_unpack_int32_to_int4(const int32_t* words, int64_t words_ld, int64_t rows, int64_t nwords,
                                       int8_t* out, int64_t out_ld, void* stream) {
  using namespace qo;
  if (rows < 0 || nwords < 0 || (rows > 1 && (words_ld < nwords || out_ld < 8 * nwords))) {
    qo_set_error("qo_unpack_int32_to_int4: invalid sizes rows=%lld words=%lld words_ld=%lld out_ld=%lld",
                 (long long)rows, (long long)nwords, (long long)words_ld, (long long)out_ld);
    return QO_ERR_SHAPE;
  }
  if (rows == 0 || nwords == 0) return QO_OK;
  if (!words || !out) {
    qo_set_error("qo_unpack_int32_to_int4: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_begin();
  const bool vec = nwords % 2 == 0 && (uintptr_t)words % 8 == 0 && (uintptr_t)out % 16 == 0 &&
                   (rows == 1 || (words_ld % 2 == 0 && out_ld % 16 == 0));
  if (vec) {
    const int64_t pairs = nwords / 2;
    launch(unpack_kernel_v16, dim3(grid_for(rows * pairs)), dim3(256), 0, s, words, words_ld, rows,
                       pairs, out, out_ld);
  } else {
    launch(unpack_kernel_any, dim3(grid_for(rows * nwords)), dim3(256), 0, s, words, words_ld, rows,
                       nwords, out, out_ld);
  }
  return launch_result("qo_unpack_int32_to_int4");
}

extern "C" int qo_transpose_int32(const int32_t* in, int64_t in_ld, int64_t rows, int64_t cols, int32_t* out,
                                  int64_t out_ld, void* stream) {
  using namespace qo;
  if (rows < 0 || cols < 0 || (rows > 1 && in_ld < cols) || (cols > 1 && out_ld < rows)) {
    qo_set_error("qo_transpose_int32: invalid sizes rows=%lld cols=%lld in_ld=%lld out_ld=%lld", (long long)rows,
                 (long long)cols, (long long)in_ld, (long long)out_ld);
    return QO_ERR_SHAPE;
  }
  if (rows == 0 || cols == 0) return QO_OK;
  if (!in || !out) {
    qo_set_error("qo_transpose_int32: NULL pointer argument");
    return QO_ERR_NULL_POINTER;
  }
  const int64_t tiles_r = (rows + kTile - 1) / kTile, tiles_c = (cols + kTile - 1) / kTile;
  if (tiles_r * tiles_c > 0x7FFFFFFF) {
    qo_set_error("qo_transpose_int32: %lld x %lld words is too large for one launch", (long long)rows,
                 (long long)cols);
    return QO_ERR_SHAPE;
  }
  // 16-byte accesses for full tiles when both matrices allow them; edge tiles
  // (and everything otherwise) move one word per access
  const bool vec = (uintptr_t)in % 16 == 0 && (uintptr_t)out % 16 == 0 && (rows == 1 || in_ld % 4 == 0) &&
                   (cols == 1 || out_ld % 4 == 0);
  launch_begin();
  if (vec)
    launch(transpose_words_kernel<true>, dim3((unsigned)(tiles_r * tiles_c)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), in, in_ld, rows, cols, out, out_ld, tiles_c);
  else
    launch(transpose_words_kernel<false>, dim3((unsigned)(tiles_r * tiles_c)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), in, in_ld, rows, cols, out, out_ld, tiles_c);
  return launch_result("qo_transpose_int32");
}
