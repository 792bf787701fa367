// Microbenchmarks of the hardware ceilings the design is measured against
// (measurement infrastructure for bench.py --ceilings; not part of the C ABI):
//
//  * qo_probe_mfma_i8: v_mfma_i32_16x16x64_i8 issue rate with a chosen number
//    of independent VALU instructions per MFMA, one or two waves per SIMD on
//    every CU (the int8 matrix-core ceiling under load, and how much VALU work
//    it hides);
//  * qo_probe_mfma_i8_data: the same with operands taken from a buffer of
//    random bytes (eight different A and B fragments per lane in turn, so the
//    matrix cores switch like they do on real data; constant operands draw
//    less power), and each wave's s_memtime ticks over the loop;
//  * qo_probe_mfma_f6_data: the same for the FP6 matrix cores
//    (v_mfma_scale_f32_16x16x128_f8f6f4, both operands FP6 e2m3, block
//    scales 2^3 as the FP6 GEMM route uses them), 32-byte operands of which
//    the instruction reads 24;
//  * qo_probe_mfma_lds_overlap: one wave per SIMD issuing FP6 MFMAs, the
//    other issuing 16-byte LDS reads (either alone, or both), to see how far
//    the two overlap on one SIMD (the FP6 GEMM's ping-pong relies on it);
//  * qo_probe_lds_dma: LDS-DMA copies (global_load_lds_dwordx4, 1 KiB per
//    instruction) from an L2-resident 32 KiB source into LDS, 16-byte LDS
//    reads, or four waves of each per CU (the FP6 GEMM's operand path: its
//    copies and its fragment reads share each CU's LDS);
//  * qo_probe_empty: an empty kernel (launch and wave start-up cost);
//  * qo_probe_stream: a streaming kernel with the quantize's traffic shape,
//    16 bytes read and 4 bytes written per lane per step (config 2 reads
//    16.8 MB of fp16 activations and writes 4.2 MB of packed codes).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// KV independent VALU instructions (one v_xor each, on four rotating
// registers) after each MFMA; eight independent accumulator chains.
template <int KV>
__global__ void __launch_bounds__(512) probe_mfma_i8(int iters, int* out) {
  const int t = threadIdx.x;
  const v4i a = {t, 1, 2, 3}, b = {3, 2, 1, t};
  v4i acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = v4i{0, 0, 0, 0};
  uint32_t x0 = t, x1 = 3 * t, x2 = 5 * t, x3 = 7 * t;
  const uint32_t c = 0x5bd1e995u;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        if (k % 4 == 0) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x0) : "v"(c));
        if (k % 4 == 1) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x1) : "v"(c));
        if (k % 4 == 2) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x2) : "v"(c));
        if (k % 4 == 3) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x3) : "v"(c));
      }
    }
  }
  int s = (int)(x0 ^ x1 ^ x2 ^ x3);
#pragma unroll
  for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[blockIdx.x * blockDim.x + t] = s;
}

// Operands from `src` (16 x 1024 fragments of 16 bytes; wave w of block b takes
// set (8 b + w) % 16): eight (A, B) pairs per lane, MFMA j on pair j.
// cycles[global wave] = s_memtime at the loop's end minus at its start.
template <int KV>
__global__ void __launch_bounds__(512) probe_mfma_i8_data(int iters, const v4i* __restrict__ src, int* out,
                                                          unsigned long long* cycles) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const v4i* set = src + (size_t)((blockIdx.x * 8 + wave) % 16) * 1024;
  v4i a[8], b[8], acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = set[j * 64 + lane];
    b[j] = set[512 + j * 64 + lane];
    acc[j] = v4i{0, 0, 0, 0};
  }
  uint32_t x0 = t, x1 = 3 * t, x2 = 5 * t, x3 = 7 * t;
  const uint32_t c = 0x5bd1e995u;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[j], b[j], acc[j], 0, 0, 0);
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        if (k % 4 == 0) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x0) : "v"(c));
        if (k % 4 == 1) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x1) : "v"(c));
        if (k % 4 == 2) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x2) : "v"(c));
        if (k % 4 == 3) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x3) : "v"(c));
      }
    }
  }
  int s = (int)(x0 ^ x1 ^ x2 ^ x3);
#pragma unroll
  for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * blockDim.x + t] = s;
  if (lane == 0) cycles[blockIdx.x * (blockDim.x >> 6) + wave] = t1 - t0;
}

// As probe_mfma_i8_data on FP6 operands: src holds 16 x 1024 fragments of 32
// bytes (6 of 8 dwords used per lane).
template <int KV>
__global__ void __launch_bounds__(512) probe_mfma_f6_data(int iters, const v8i* __restrict__ src, float* out,
                                                          unsigned long long* cycles) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const v8i* set = src + (size_t)((blockIdx.x * 8 + wave) % 16) * 1024;
  v8i a[8], b[8];
  v4f acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = set[j * 64 + lane];
    b[j] = set[512 + j * 64 + lane];
    acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  uint32_t x0 = t, x1 = 3 * t, x2 = 5 * t, x3 = 7 * t;
  const uint32_t c = 0x5bd1e995u;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j], b[j], acc[j], 2, 2, 0, 130, 0, 130);
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        if (k % 4 == 0) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x0) : "v"(c));
        if (k % 4 == 1) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x1) : "v"(c));
        if (k % 4 == 2) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x2) : "v"(c));
        if (k % 4 == 3) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x3) : "v"(c));
      }
    }
  }
  float s = (float)(x0 ^ x1 ^ x2 ^ x3);
#pragma unroll
  for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * blockDim.x + t] = s;
  if (lane == 0) cycles[blockIdx.x * (blockDim.x >> 6) + wave] = t1 - t0;
}

// 512 threads: waves 0-3 (one per SIMD) run FP6 MFMAs when mode bit 0 is set,
// waves 4-7 run ds_read_b128 loops (4 x 1 KiB per iteration) when bit 1 is.
__global__ void __launch_bounds__(512) probe_mfma_lds_overlap(int mode, int iters, float* out) {
  __shared__ __align__(16) unsigned char buf[65536];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int i = t; i < 16384; i += 512) reinterpret_cast<int*>(buf)[i] = i;
  __syncthreads();
  float s = 0.f;
  if (wave < 4) {
    if (mode & 1) {
      const v8i a = {t, 1, 2, 3, 4, 5, 6, 7}, b = {7, 6, 5, 4, 3, 2, 1, t};
      v4f acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
      for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], 2, 2, 0, 127, 0, 127);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += acc[j][0];
    }
  } else if (mode & 2) {
    v4i acc = {0, 0, 0, 0};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc ^= *reinterpret_cast<const v4i*>(buf + ((wave * 4 + k + it) & 31) * 2048 + 16 * lane);
    s = (float)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
  }
  out[blockIdx.x * 512 + t] = s;
}

// 512 threads. Copying waves: 8 copies of 1 KiB per iteration into the upper
// 32 KiB of LDS (at most 16 in flight); reading waves: 16 ds_read_b128 of
// 1 KiB per iteration from the lower 32 KiB. Mode 1: every wave copies;
// 2: every wave reads; 3: waves 0-3 copy, waves 4-7 read. Every access lies
// inside the 32 KiB source and the 64 KiB LDS buffer.
__global__ void __launch_bounds__(512) probe_lds_dma(int mode, int iters, const unsigned char* __restrict__ src,
                                                     float* out) {
  __shared__ __align__(16) unsigned char buf[65536];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int i = t; i < 16384; i += 512) reinterpret_cast<int*>(buf)[i] = i;
  __syncthreads();
  const bool copier = mode == 1 || (mode == 3 && wave < 4);
  float s = 0.f;
  if (copier) {
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)(buf + 32768);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int c = (wave * 8 + k + it) & 31;   // source KiB; destination KiB (wave * 8 + k) % 32
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src + c * 1024 + 16 * lane),
                     "{m0}"(base + (uint32_t)(((wave * 8 + k) & 31) * 1024))
                     : "memory");
      }
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    v4i acc = {0, 0, 0, 0};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int k = 0; k < 16; ++k) acc ^= *reinterpret_cast<const v4i*>(buf + ((wave * 16 + k + it) & 31) * 1024 + 16 * lane);
    s = (float)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
  }
  out[blockIdx.x * 512 + t] = s;
}

__global__ void probe_empty() {}

// grid-stride: 16 bytes in, their four words XORed into 4 bytes out
__global__ void __launch_bounds__(256) probe_stream(const v4i* __restrict__ in, int* __restrict__ out, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) {
    const v4i v = in[i];
    out[i] = v[0] ^ v[1] ^ v[2] ^ v[3];
  }
}

}  // namespace

// threads per block: 512 (two waves per SIMD) or 256 (one)
extern "C" int qo_probe_mfma_i8(int kvalu, int blocks, int iters, int* out, void* stream, int threads) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (threads != 256 && threads != 512) return 1;
  switch (kvalu) {
    case 0: probe_mfma_i8<0><<<blocks, threads, 0, s>>>(iters, out); break;
    case 1: probe_mfma_i8<1><<<blocks, threads, 0, s>>>(iters, out); break;
    case 2: probe_mfma_i8<2><<<blocks, threads, 0, s>>>(iters, out); break;
    case 3: probe_mfma_i8<3><<<blocks, threads, 0, s>>>(iters, out); break;
    case 4: probe_mfma_i8<4><<<blocks, threads, 0, s>>>(iters, out); break;
    case 8: probe_mfma_i8<8><<<blocks, threads, 0, s>>>(iters, out); break;
    default: return 1;
  }
  return (int)hipGetLastError();
}

// src: 16 x 1024 x 16 bytes; out: blocks x threads ints; cycles: blocks x threads / 64
extern "C" int qo_probe_mfma_i8_data(int kvalu, int blocks, int iters, const void* src, int* out,
                                     unsigned long long* cycles, void* stream, int threads) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (threads != 256 && threads != 512) return 1;
  const v4i* v = static_cast<const v4i*>(src);
  switch (kvalu) {
    case 0: probe_mfma_i8_data<0><<<blocks, threads, 0, s>>>(iters, v, out, cycles); break;
    case 2: probe_mfma_i8_data<2><<<blocks, threads, 0, s>>>(iters, v, out, cycles); break;
    case 4: probe_mfma_i8_data<4><<<blocks, threads, 0, s>>>(iters, v, out, cycles); break;
    default: return 1;
  }
  return (int)hipGetLastError();
}

// src: 16 x 1024 x 32 bytes; out: blocks x 512 floats; cycles: blocks x 8; 512 threads
extern "C" int qo_probe_mfma_f6_data(int kvalu, int blocks, int iters, const void* src, float* out,
                                     unsigned long long* cycles, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const v8i* v = static_cast<const v8i*>(src);
  switch (kvalu) {
    case 0: probe_mfma_f6_data<0><<<blocks, 512, 0, s>>>(iters, v, out, cycles); break;
    case 2: probe_mfma_f6_data<2><<<blocks, 512, 0, s>>>(iters, v, out, cycles); break;
    default: return 1;
  }
  return (int)hipGetLastError();
}

// mode 1: MFMAs only, 2: LDS reads only, 3: both; out: blocks x 512 floats
extern "C" int qo_probe_mfma_lds_overlap(int mode, int blocks, int iters, float* out, void* stream) {
  if (mode < 1 || mode > 3) return 1;
  probe_mfma_lds_overlap<<<blocks, 512, 0, reinterpret_cast<hipStream_t>(stream)>>>(mode, iters, out);
  return (int)hipGetLastError();
}

// src: 32 KiB; out: blocks x 512 floats
extern "C" int qo_probe_lds_dma(int mode, int blocks, int iters, const void* src, float* out, void* stream) {
  if (mode < 1 || mode > 3) return 1;
  probe_lds_dma<<<blocks, 512, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      mode, iters, static_cast<const unsigned char*>(src), out);
  return (int)hipGetLastError();
}

extern "C" int qo_probe_empty(void* stream) {
  probe_empty<<<1, 64, 0, reinterpret_cast<hipStream_t>(stream)>>>();
  return (int)hipGetLastError();
}

extern "C" int qo_probe_stream(const void* in, void* out, int64_t bytes_in, int blocks, void* stream) {
  if (bytes_in % 16 != 0) return 1;
  probe_stream<<<blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(static_cast<const v4i*>(in),
                                                                         static_cast<int*>(out), bytes_in / 16);
  return (int)hipGetLastError();
}
