// common.hpp -- device helpers shared by the gfx950 MoE kernels.
//
// Weight formats (same numbering as qmoe_format in include/qmoe.h):
//   F32   4 B/elem      BF16  2 B/elem (bf16f32: bits << 16, model/model.go:113)
//   INT8  1 B/elem + fp16 scale per 32      INT4  0.5 B/elem + fp16 scale per 32
// INT4 packs element 2c in the high nibble and 2c+1 in the low nibble of byte c,
// value = nibble - 8 (model/moe.go:146-153).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmoe {

enum Fmt : int { kF32 = 0, kBF16 = 1, kINT8 = 2, kINT4 = 3 };

constexpr int kGroup = 32;  // quantGroup, model/moe.go:124

// Bytes per stored element, times 2 (so INT4 = 1).
__host__ __device__ constexpr int fmt_bytes_x2(int fmt) {
  return fmt == kF32 ? 8 : fmt == kBF16 ? 4 : fmt == kINT8 ? 2 : 1;
}
__host__ __device__ constexpr bool fmt_quant(int fmt) { return fmt == kINT8 || fmt == kINT4; }
// Storage bytes of a (rows, cols) matrix in fmt.
__host__ __device__ inline int64_t fmt_matrix_bytes(int fmt, int64_t rows, int64_t cols) {
  return rows * cols * fmt_bytes_x2(fmt) / 2;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round-to-nearest-even mode
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// LDS offset of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from global memory straight into LDS at lds_wave_base +
// 16 * lane (lds_wave_base is wave-uniform).  Issued through asm so that the
// compiler does not track these loads: the GEMM waits for them explicitly
// (wait_vm), and loads the compiler does track that were issued later only make
// its own waits more conservative, never insufficient.  The LDS base goes in
// through a "{m0}" operand, so the compiler itself writes M0 (and knows its
// value) before the statement; the s_nop is the wait state between that write
// and the LDS-direct load that reads it.
__device__ __forceinline__ void dma16(const void *src, const unsigned char *lds_wave_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds_wave_base));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// The same with the nontemporal hint (streamed weights that are read once).
__device__ __forceinline__ void dma16_nt(const void *src, const unsigned char *lds_wave_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds_wave_base));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(m0) : "memory");
}

// 16-byte load with the nontemporal hint.
__device__ __forceinline__ uint4 load_nt(const void *p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of the group receives the sum.
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Loads one 16-byte chunk of a weight row and widens it to f32.
// Elements per chunk: F32 4, BF16 8, INT8 16, INT4 32.  For the INT formats the
// returned values are the raw integers (code, or nibble - 8) and *scale holds
// the chunk's group scale (a chunk never straddles a group of 32).
template <int FMT>
struct Chunk {
  static constexpr int kElems = FMT == kF32 ? 4 : FMT == kBF16 ? 8 : FMT == kINT8 ? 16 : 32;
};

template <int FMT>
__device__ __forceinline__ void load_chunk(const uint8_t *__restrict__ row, const uint16_t *__restrict__ srow,
                                           int chunk, float (&w)[Chunk<FMT>::kElems], float &scale) {
  const uint4 v = *reinterpret_cast<const uint4 *>(row + (size_t)chunk * 16);
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if constexpr (FMT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = __uint_as_float(u[i]);
    scale = 1.0f;
  } else if constexpr (FMT == kBF16) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w[2 * i] = __uint_as_float(u[i] << 16);
      w[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
    scale = 1.0f;
  } else if constexpr (FMT == kINT8) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int b = 0; b < 4; b++) w[4 * i + b] = (float)(int8_t)((u[i] >> (8 * b)) & 0xffu);
    }
    scale = f16_to_f32(srow[(chunk * 16) / kGroup]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        uint32_t byte = (u[i] >> (8 * b)) & 0xffu;
        w[8 * i + 2 * b] = (float)((int)(byte >> 4) - 8);
        w[8 * i + 2 * b + 1] = (float)((int)(byte & 0xfu) - 8);
      }
    }
    scale = f16_to_f32(srow[chunk]);  // 32 elements = one group
  }
}

// f32 -> bf16, round to nearest even (NaN stays a NaN): x for the batched
// GEMMs' A operand.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);  // NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

}  // namespace qmoe
