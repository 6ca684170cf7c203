// quant.hip -- device quantiser and dequantiser for the group-32 formats.
//
// quantize_kernel restates quantizeInt8 / quantizeInt4 (model/moe.go:165-217)
// with the same IEEE operations, so codes are bit-identical to the
// reference's: amax = max |w| over the group, s = amax / 127 (or / 7) as an
// f32 divide, floored at 1e-8, code = clamp(round_half_away(w / s)).  The
// stored scale is the f32 s rounded to fp16 (nearest-even), the device format.
//
// dequantize_kernel restates quantLinear.dequantize (model/moe.go:134-157):
// one exact f32 multiply float(code) * scale, so its output is bit-exact.
#include "common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace qmoe {

template <int BITS>
__global__ void __launch_bounds__(256) quantize_kernel(const float *__restrict__ w, int64_t n_rows, int cols,
                                                       uint8_t *__restrict__ codes,
                                                       uint16_t *__restrict__ scales) {
#pragma clang fp contract(off)
  const int ng = cols / kGroup;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= n_rows * ng) return;
  const int64_t row = gid / ng;
  const int b = (int)(gid % ng);
  const float *g = w + row * cols + (int64_t)b * kGroup;
  float v[kGroup];
#pragma unroll
  for (int q = 0; q < kGroup / 4; q++) {
    float4 f = reinterpret_cast<const float4 *>(g)[q];
    v[4 * q] = f.x;
    v[4 * q + 1] = f.y;
    v[4 * q + 2] = f.z;
    v[4 * q + 3] = f.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < kGroup; j++) {
    float a = v[j] < 0.0f ? -v[j] : v[j];  // abs32, model/moe.go:241-246
    if (a > amax) amax = a;
  }
  float s = amax / (BITS == 8 ? 127.0f : 7.0f);
  if (s < 1e-8f) s = 1e-8f;
  scales[gid] = f32_to_f16_rne(s);
  if constexpr (BITS == 8) {
    uint32_t packed[kGroup / 4];
#pragma unroll
    for (int q = 0; q < kGroup / 4; q++) {
      uint32_t word = 0;
#pragma unroll
      for (int bb = 0; bb < 4; bb++) {
        float r = roundf(v[4 * q + bb] / s);  // roundF32: half away from zero
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        word |= ((uint32_t)(uint8_t)(int8_t)r) << (8 * bb);
      }
      packed[q] = word;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(codes + row * cols + (int64_t)b * kGroup);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  } else {
    uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kGroup; j++) {
      float r = roundf(v[j] / s);
      r = r < -7.0f ? -7.0f : (r > 7.0f ? 7.0f : r);
      uint32_t nib = (uint32_t)((int)(r + 8.0f) & 0xf);
      int byte = j / 2;
      uint32_t shift = 8 * (byte % 4) + ((j % 2 == 0) ? 4 : 0);  // even element -> high nibble
      packed[byte / 4] |= nib << shift;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(codes + row * (cols / 2) + (int64_t)b * (kGroup / 2));
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
}

hipError_t launch_quantize(int bits, const float *w, int64_t n_rows, int cols, uint8_t *codes,
                           uint16_t *scales, hipStream_t st) {
  const int64_t n = n_rows * (cols / kGroup);
  if (n == 0) return hipSuccess;
  dim3 grid((unsigned)((n + 255) / 256));
  if (bits == 8)
    hipLaunchKernelGGL(quantize_kernel<8>, grid, dim3(256), 0, st, w, n_rows, cols, codes, scales);
  else
    hipLaunchKernelGGL(quantize_kernel<4>, grid, dim3(256), 0, st, w, n_rows, cols, codes, scales);
  return hipGetLastError();
}

template <int FMT>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint8_t *__restrict__ wq,
                                                         const uint16_t *__restrict__ s, int rows,
                                                         int cols, float *__restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * cols) return;
  const int64_t o = i / cols;
  const int c = (int)(i % cols);
  float v;
  if constexpr (FMT == kF32) {
    v = reinterpret_cast<const float *>(wq)[i];
  } else if constexpr (FMT == kBF16) {
    v = bf16_to_f32(reinterpret_cast<const uint16_t *>(wq)[i]);
  } else if constexpr (FMT == kINT8) {
    v = (float)(int8_t)wq[i] * f16_to_f32(s[o * (cols / kGroup) + c / kGroup]);
  } else {
    uint8_t b = wq[o * (cols / 2) + c / 2];
    int nib = (c % 2 == 0) ? (b >> 4) : (b & 0xf);
    v = ((float)nib - 8.0f) * f16_to_f32(s[o * (cols / kGroup) + c / kGroup]);
  }
  out[i] = v;
}

hipError_t launch_dequantize(const DevMat &m, int64_t index, float *out, hipStream_t st) {
  const int64_t n = (int64_t)m.rows * m.cols;
  dim3 grid((unsigned)((n + 255) / 256));
  const uint8_t *w = m.w + index * m.mat_bytes;
  const uint16_t *s = m.s ? m.s + index * m.mat_scales : nullptr;
  switch (m.fmt) {
  case kF32: hipLaunchKernelGGL(dequantize_kernel<kF32>, grid, dim3(256), 0, st, w, s, m.rows, m.cols, out); break;
  case kBF16: hipLaunchKernelGGL(dequantize_kernel<kBF16>, grid, dim3(256), 0, st, w, s, m.rows, m.cols, out); break;
  case kINT8: hipLaunchKernelGGL(dequantize_kernel<kINT8>, grid, dim3(256), 0, st, w, s, m.rows, m.cols, out); break;
  default: hipLaunchKernelGGL(dequantize_kernel<kINT4>, grid, dim3(256), 0, st, w, s, m.rows, m.cols, out); break;
  }
  return hipGetLastError();
}

}  // namespace qmoe
