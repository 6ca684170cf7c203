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

// Element (row o, column c) of a stored (rows, cols) matrix as f32, exactly as
// quantLinear.dequantize / bf16f32 give it.
template <int FMT>
__device__ __forceinline__ float stored_value(const uint8_t *__restrict__ wq, const uint16_t *__restrict__ s,
                                              int64_t o, int c, int cols) {
#pragma clang fp contract(off)
  if constexpr (FMT == kF32) {
    return reinterpret_cast<const float *>(wq)[o * cols + c];
  } else if constexpr (FMT == kBF16) {
    return bf16_to_f32(reinterpret_cast<const uint16_t *>(wq)[o * cols + c]);
  } else if constexpr (FMT == kINT8) {
    return (float)(int8_t)wq[o * cols + c] * f16_to_f32(s[o * (cols / kGroup) + c / kGroup]);
  } else {
    const uint8_t b = wq[o * (cols / 2) + c / 2];
    const int nib = (c % 2 == 0) ? (b >> 4) : (b & 0xf);
    return ((float)nib - 8.0f) * f16_to_f32(s[o * (cols / kGroup) + c / kGroup]);
  }
}

// out (rows, cols) f32.  With transposed, the matrix is stored as its (cols,
// rows) transpose with groups of 32 along the stored columns' transpose: see
// launch_relayout_transpose.
template <int FMT>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint8_t *__restrict__ wq,
                                                         const uint16_t *__restrict__ s, int rows, int cols,
                                                         bool transposed, float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * cols) return;
  const int64_t o = i / cols;
  const int c = (int)(i % cols);
  if (!transposed) {
    out[i] = stored_value<FMT>(wq, s, o, c, cols);
    return;
  }
  // stored: element (o, c) of the logical matrix sits at (c, o) of a
  // (cols, rows) matrix whose quantisation groups run down its columns
  float v;
  if constexpr (FMT == kF32) {
    v = reinterpret_cast<const float *>(wq)[(int64_t)c * rows + o];
  } else if constexpr (FMT == kBF16) {
    v = bf16_to_f32(reinterpret_cast<const uint16_t *>(wq)[(int64_t)c * rows + o]);
  } else {
    const float sc = f16_to_f32(s[(int64_t)(c / kGroup) * rows + o]);
    if constexpr (FMT == kINT8) {
      v = (float)(int8_t)wq[(int64_t)c * rows + o] * sc;
    } else {
      const uint8_t b = wq[(int64_t)c * (rows / 2) + o / 2];
      const int nib = (o % 2 == 0) ? (b >> 4) : (b & 0xf);
      v = ((float)nib - 8.0f) * sc;
    }
  }
  out[i] = v;
}

hipError_t launch_dequantize(const DevMat &m, int64_t index, float *out, hipStream_t st) {
  const int64_t n = (int64_t)m.rows * m.cols;
  dim3 grid((unsigned)((n + 255) / 256));
  const uint8_t *w = m.w + index * m.mat_bytes;
  const uint16_t *s = m.s ? m.s + index * m.mat_scales : nullptr;
#define L(F) hipLaunchKernelGGL(dequantize_kernel<F>, grid, dim3(256), 0, st, w, s, m.rows, m.cols, m.transposed, out)
  switch (m.fmt) {
  case kF32: L(kF32); break;
  case kBF16: L(kBF16); break;
  case kINT8: L(kINT8); break;
  default: L(kINT4); break;
  }
#undef L
  return hipGetLastError();
}

// quantLinear.dequantize (model/moe.go:134-157) with the reference's own f32
// scales (qwen-quant writes them as F32, cmd/qwen-quant/main.go:207-210):
// n_rows rows of cols elements, w = float32(code) * scale, one f32 multiply
// per element; int4: byte c of a row holds element 2c in its high nibble and
// 2c+1 in its low nibble, value = float32(nibble) - 8.
template <int BITS>
__global__ void __launch_bounds__(256) dequant_f32s_kernel(const uint8_t *__restrict__ codes,
                                                           const float *__restrict__ scales, int64_t n_rows, int cols,
                                                           float *__restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_rows * cols) return;
  const int64_t o = i / cols;
  const int c = (int)(i % cols);
  const float sc = scales[o * (cols / kGroup) + c / kGroup];
  float v;
  if constexpr (BITS == 8) {
    v = (float)(int8_t)codes[i];
  } else {
    const uint8_t b = codes[o * (cols / 2) + c / 2];
    v = (float)((c % 2 == 0) ? (b >> 4) : (b & 0xf)) - 8.0f;
  }
  out[i] = v * sc;
}

hipError_t launch_dequant_f32s(int bits, const uint8_t *codes, const float *scales, int64_t n_rows, int cols,
                               float *out, hipStream_t st) {
  const int64_t n = n_rows * cols;
  if (n <= 0) return hipSuccess;
  dim3 grid((unsigned)((n + 255) / 256));
  if (bits == 8)
    hipLaunchKernelGGL(dequant_f32s_kernel<8>, grid, dim3(256), 0, st, codes, scales, n_rows, cols, out);
  else
    hipLaunchKernelGGL(dequant_f32s_kernel<4>, grid, dim3(256), 0, st, codes, scales, n_rows, cols, out);
  return hipGetLastError();
}

// f32 -> bf16 bit patterns, round to nearest even (NaNs stay quiet NaNs).
__global__ void __launch_bounds__(256) f32_to_bf16_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                          int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t u = __float_as_uint(src[i]);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) {
    dst[i] = (uint16_t)((u >> 16) | 0x40u);
    return;
  }
  dst[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, dst, n);
  return hipGetLastError();
}

// Re-layout of n_mat stored (rows, cols) matrices in the reference layout into
// their (cols, rows) transposes, keeping every stored code and scale: the
// element (o, c) moves to (c, o); INT4 nibbles pair up along the new rows
// (even element in the high nibble); the group-32 scales (rows, cols / 32)
// become (cols / 32, rows), one scale per (group, original row).  Values are
// unchanged, so dequantisation stays bit-exact.
template <int FMT>
__global__ void __launch_bounds__(256) transpose_kernel(const uint8_t *__restrict__ src, const uint16_t *__restrict__ ss,
                                                        int rows, int cols, uint8_t *__restrict__ dst,
                                                        uint16_t *__restrict__ ds) {
  const int64_t mat = blockIdx.y;
  const int64_t mbytes = fmt_matrix_bytes(FMT, rows, cols);
  const int64_t msc = fmt_quant(FMT) ? (int64_t)rows * (cols / kGroup) : 0;
  src += mat * mbytes;
  dst += mat * mbytes;
  if constexpr (FMT == kINT4) {
    // one thread per destination byte: (c, o pair)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)cols * (rows / 2)) return;
    const int c = (int)(i / (rows / 2));
    const int o = (int)(i % (rows / 2)) * 2;
    auto nib = [&](int oo) {
      const uint8_t b = src[(int64_t)oo * (cols / 2) + c / 2];
      return (c % 2 == 0) ? (b >> 4) : (b & 0xf);
    };
    dst[i] = (uint8_t)((nib(o) << 4) | nib(o + 1));
  } else {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // destination element (c, o)
    if (i >= (int64_t)rows * cols) return;
    const int c = (int)(i / rows);
    const int o = (int)(i % rows);
    if constexpr (FMT == kF32) {
      reinterpret_cast<float *>(dst)[i] = reinterpret_cast<const float *>(src)[(int64_t)o * cols + c];
    } else if constexpr (FMT == kBF16) {
      reinterpret_cast<uint16_t *>(dst)[i] = reinterpret_cast<const uint16_t *>(src)[(int64_t)o * cols + c];
    } else {
      dst[i] = src[(int64_t)o * cols + c];
    }
  }
  if constexpr (fmt_quant(FMT)) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // destination scale (g, o)
    if (i < msc) {
      const int g = (int)(i / rows), o = (int)(i % rows);
      ds[mat * msc + i] = ss[mat * msc + (int64_t)o * (cols / kGroup) + g];
    }
  }
}

hipError_t launch_relayout_transpose(int fmt, const uint8_t *src, const uint16_t *ss, int64_t n_mat, int rows,
                                     int cols, uint8_t *dst, uint16_t *ds, hipStream_t st) {
  const int64_t n = (int64_t)rows * cols;
  dim3 grid((unsigned)((n + 255) / 256), (unsigned)n_mat);
#define L(F) hipLaunchKernelGGL(transpose_kernel<F>, grid, dim3(256), 0, st, src, ss, rows, cols, dst, ds)
  switch (fmt) {
  case kF32: L(kF32); break;
  case kBF16: L(kBF16); break;
  case kINT8: L(kINT8); break;
  default: L(kINT4); break;
  }
#undef L
  return hipGetLastError();
}

}  // namespace qmoe
