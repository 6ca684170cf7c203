// norm_common.hpp -- the certified GemmaRMSNorm scale shared by the norm
// kernel (norm.hip) and the decode kernel's prologue (fused.hip).
//
// gemmaRMSNormApply (model/tensors.go:147-157): s = sum of float64(x_i)^2 in
// index order, inv = float32(1 / sqrt(s / n + float64(eps))).  The products are
// exact in f64; a parallel sum sp of the n non-negative terms is within
// 2 gamma(n-1) s of the index-order one, and inv(s) is monotone (each f64 step
// rounds monotonically, then the f32 rounding), so inv(sp (1 - d)) ==
// inv(sp (1 + d)) with d = 3 n 2^-53 proves that value is the reference's.
#pragma once

#include <hip/hip_runtime.h>

namespace qmoe {

__device__ __forceinline__ float norm_inv(double s, int n, float eps) {
  return (float)(1.0 / __builtin_sqrt(s / (double)n + (double)eps));
}

// *inv from the parallel sum sp; false when the interval does not settle the
// f32 value (then the caller sums in index order).
__device__ __forceinline__ bool norm_certify(double sp, int n, float eps, float *inv) {
  const double d = 3.0 * (double)n * 0x1p-53;
  const float lo = norm_inv(sp * (1.0 - d), n, eps);
  *inv = lo;
  return lo == norm_inv(sp * (1.0 + d), n, eps);
}

}  // namespace qmoe
