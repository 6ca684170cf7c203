// gemv_common.hpp -- device helpers of the bandwidth-bound expert products
// (fused.hip): 16-byte weight chunks dotted with f32 activations in LDS.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace qmoe {

constexpr int kBlock = 256;

// Largest power of two <= 64 that divides n (lanes per row).
__host__ __device__ inline int lanes_per_row(int n) {
  int l = 64;
  while (l > 1 && (n % l) != 0) l >>= 1;
  return l;
}

// Dot of one 16-byte chunk with EPC activations in LDS.
template <int FMT>
__device__ __forceinline__ float chunk_dot(const uint4 v, const float *__restrict__ xc) {
  constexpr int EPC = Chunk<FMT>::kElems;
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  float acc = 0.0f;
  const float4 *x4 = reinterpret_cast<const float4 *>(xc);
#pragma unroll
  for (int q = 0; q < EPC / 4; q++) {
    const float4 xx = x4[q];
    float w0, w1, w2, w3;
    if constexpr (FMT == kF32) {  // EPC == 4: q == 0
      w0 = __uint_as_float(u[0]);
      w1 = __uint_as_float(u[1]);
      w2 = __uint_as_float(u[2]);
      w3 = __uint_as_float(u[3]);
    } else if constexpr (FMT == kBF16) {
      const uint32_t a = u[2 * q], b = u[2 * q + 1];
      w0 = __uint_as_float(a << 16);
      w1 = __uint_as_float(a & 0xffff0000u);
      w2 = __uint_as_float(b << 16);
      w3 = __uint_as_float(b & 0xffff0000u);
    } else if constexpr (FMT == kINT8) {
      const uint32_t a = u[q];
      w0 = (float)(int8_t)(a & 0xffu);
      w1 = (float)(int8_t)((a >> 8) & 0xffu);
      w2 = (float)(int8_t)((a >> 16) & 0xffu);
      w3 = (float)(int8_t)(a >> 24);
    } else {
      // 4 elements = 2 bytes; byte c holds (2c: high nibble, 2c+1: low nibble)
      const uint32_t a = u[q / 2] >> (16 * (q % 2));
      w0 = (float)((int)((a >> 4) & 0xfu) - 8);
      w1 = (float)((int)(a & 0xfu) - 8);
      w2 = (float)((int)((a >> 12) & 0xfu) - 8);
      w3 = (float)((int)((a >> 8) & 0xfu) - 8);
    }
    acc = fmaf(w0, xx.x, acc);
    acc = fmaf(w1, xx.y, acc);
    acc = fmaf(w2, xx.z, acc);
    acc = fmaf(w3, xx.w, acc);
  }
  return acc;
}

// Partial dot of a stored row with activations xs (LDS): this lane takes
// chunks sl, sl+lpr, ..., ITER of them; all loads are issued first.
template <int FMT, int ITER>
__device__ __forceinline__ float row_dot(const uint8_t *__restrict__ row, const uint16_t *__restrict__ srow,
                                         const float *__restrict__ xs, int sl, int lpr) {
  constexpr int EPC = Chunk<FMT>::kElems;
  uint4 v[ITER];
#pragma unroll
  for (int i = 0; i < ITER; i++) v[i] = *reinterpret_cast<const uint4 *>(row + (size_t)(sl + i * lpr) * 16);
  float sc[ITER];
  if constexpr (fmt_quant(FMT)) {
#pragma unroll
    for (int i = 0; i < ITER; i++) sc[i] = f16_to_f32(srow[((sl + i * lpr) * EPC) / kGroup]);
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < ITER; i++) {
    const float d = chunk_dot<FMT>(v[i], xs + (sl + i * lpr) * EPC);
    if constexpr (fmt_quant(FMT)) acc = fmaf(d, sc[i], acc);
    else acc += d;
  }
  return acc;
}

// Same with a run-time chunk count (rare shapes).
template <int FMT>
__device__ __forceinline__ float row_dot_rt(const uint8_t *__restrict__ row, const uint16_t *__restrict__ srow,
                                            const float *__restrict__ xs, int sl, int lpr, int nch) {
  constexpr int EPC = Chunk<FMT>::kElems;
  float acc = 0.0f;
  for (int c = sl; c < nch; c += lpr) {
    const uint4 v = *reinterpret_cast<const uint4 *>(row + (size_t)c * 16);
    const float d = chunk_dot<FMT>(v, xs + c * EPC);
    if constexpr (fmt_quant(FMT)) acc = fmaf(d, f16_to_f32(srow[(c * EPC) / kGroup]), acc);
    else acc += d;
  }
  return acc;
}

template <int FMT, int ITER>
__device__ __forceinline__ float row_dot_any(const uint8_t *row, const uint16_t *srow, const float *xs, int sl,
                                             int lpr, int nch) {
  if constexpr (ITER > 0) return row_dot<FMT, ITER>(row, srow, xs, sl, lpr);
  else return row_dot_rt<FMT>(row, srow, xs, sl, lpr, nch);
}

__device__ __forceinline__ float silu_ref(float g) {
  // silu, model/tensors.go:91-95
  return g / (1.0f + (float)exp(-(double)g));
}

// Chunks per lane for a row of `cols` elements in fmt (0 = no compile-time
// specialisation available).
inline int iter_of(int fmt, int cols) {
  const int epc = fmt == kF32 ? 4 : fmt == kBF16 ? 8 : fmt == kINT8 ? 16 : 32;
  const int nch = cols / epc;
  const int it = nch / lanes_per_row(nch);
  return (it == 1 || it == 2 || it == 3 || it == 4 || it == 8) ? it : 0;
}

// Dispatch helper: the compile-time chunk counts that realistic shapes use.
#define QMOE_ITER_CASES(F, MACRO) \
  MACRO(F, 1) MACRO(F, 2) MACRO(F, 3) MACRO(F, 4) MACRO(F, 8)

}  // namespace qmoe
