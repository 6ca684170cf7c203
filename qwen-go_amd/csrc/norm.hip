// norm.hip -- qwen-go's post-attention GemmaRMSNorm on the device, bit for bit
// (gemmaRMSNormApply, model/tensors.go:147-157, applied per token at
// model/model.go:509-511):
//   s = sum_i float64(x_i) * float64(x_i)        (f64, index order)
//   inv = float32(1 / sqrt(s / float64(n) + float64(eps)))
//   xn_i = fl(fl(x_i * inv) * fl(1 + w_i))
//
// The products are exact in f64, so only the order of the f64 additions can
// differ from the reference's.  The workgroup sums in parallel; for n
// non-negative terms any order lies within 2 * gamma(n-1) * s of any other,
// and inv(s) is monotone (every f64 step rounds monotonically, then the f32
// rounding), so when inv takes the same value at both ends of that interval it
// is the reference's inv.  Otherwise (about one token in 10^5..10^6 at
// n = 2048) one lane redoes the sum in index order -- always when force_seq
// (a test of that path).
#include "common.hpp"
#include "kernels.hpp"
#include "norm_common.hpp"

namespace qmoe {

constexpr int kNormThreads = 256;

__global__ void __launch_bounds__(kNormThreads) gemma_norm_kernel(const float *__restrict__ x,
                                                                  const float *__restrict__ w, float eps, int n,
                                                                  float *__restrict__ xn,
                                                                  unsigned int *__restrict__ redo, int force_seq) {
#pragma clang fp contract(off)
  __shared__ double part[kNormThreads / 64];
  __shared__ float s_inv;
  const int t = blockIdx.x;
  const float *xr = x + (size_t)t * n;
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += kNormThreads) s += (double)xr[i] * (double)xr[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double sp = 0.0;
    for (int i = 0; i < kNormThreads / 64; i++) sp += part[i];
    float inv;
    if (!norm_certify(sp, n, eps, &inv) || force_seq) {
      double q = 0.0;
      for (int i = 0; i < n; i++) q += (double)xr[i] * (double)xr[i];
      inv = norm_inv(q, n, eps);
      if (redo) atomicAdd(redo, 1u);
    }
    s_inv = inv;
  }
  __syncthreads();
  const float inv = s_inv;
  float *yr = xn + (size_t)t * n;
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    const float a = xr[i] * inv;
    const float b = 1.0f + w[i];
    yr[i] = a * b;
  }
}

hipError_t launch_gemma_norm(const float *x, int T, int n, const float *w, float eps, float *xn, unsigned int *redo,
                             bool force_seq, hipStream_t st) {
  if (T <= 0 || n <= 0) return hipErrorInvalidValue;
  QMOE_LAUNCH(gemma_norm_kernel, dim3((unsigned)T), dim3(kNormThreads), 0, st, x, w, eps, n, xn, redo,
              (int)force_seq);
  return hipGetLastError();
}

// out (T*H) = src: the residual stream an accumulating path starts from.
__global__ void __launch_bounds__(256) copy_kernel(const float *__restrict__ src, float *__restrict__ dst, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 4 <= n) {
    *reinterpret_cast<float4 *>(dst + i) = *reinterpret_cast<const float4 *>(src + i);
  } else {
    for (int64_t j = i; j < n; j++) dst[j] = src[j];
  }
}

hipError_t launch_copy(const float *src, float *dst, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (src == dst) return hipSuccess;
  QMOE_LAUNCH(copy_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, src, dst, n);
  return hipGetLastError();
}

}  // namespace qmoe
