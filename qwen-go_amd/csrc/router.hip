// router.hip -- router logits, softmax and top-k selection for gfx950.
//
// Parity contract: the expert ids must equal the reference's bit for bit, so
// every router logit is computed exactly as Go computes it:
//   s = 0; for h in 0..H-1: s = fl(s + fl(x[h] * w[e][h]))
// (matmulVec model/tensors.go:77-89, matvecRange model/model.go:167-176,
// quantLinear.forward model/moe.go:159-162).  Each output keeps its own
// sequential h-ordered accumulator; parallelism comes from (token, expert)
// pairs only.  `#pragma clang fp contract(off)` keeps the multiply and the add
// separately rounded, as Go on amd64 does.
#include "common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace qmoe {

// Widens element k of a stored router row to f32 exactly as the reference:
// bf16 -> bits << 16, int8 -> float(code) * scale, int4 -> float(nibble-8) * scale.
template <int FMT>
__device__ __forceinline__ void router_chunk(const uint8_t *__restrict__ row,
                                             const uint16_t *__restrict__ srow, int chunk,
                                             float (&w)[Chunk<FMT>::kElems]) {
#pragma clang fp contract(off)
  float sc;
  load_chunk<FMT>(row, srow, chunk, w, sc);
  if constexpr (fmt_quant(FMT)) {
#pragma unroll
    for (int i = 0; i < Chunk<FMT>::kElems; i++) w[i] = w[i] * sc;
  }
}

// One thread per (token, expert); used when T is small.  The token's x row is
// staged in LDS and read as a broadcast; each lane streams its own router row.
template <int FMT>
__global__ void __launch_bounds__(64) router_rowwise_kernel(const float *__restrict__ x, int T, int H,
                                                            const uint8_t *__restrict__ w,
                                                            const uint16_t *__restrict__ s, int E,
                                                            float *__restrict__ logits) {
#pragma clang fp contract(off)
  extern __shared__ float xs[];
  const int t = blockIdx.y;
  const int e = blockIdx.x * 64 + threadIdx.x;
  for (int i = threadIdx.x; i < H; i += 64) xs[i] = x[(size_t)t * H + i];
  __syncthreads();
  if (e >= E) return;
  constexpr int EPC = Chunk<FMT>::kElems;
  const uint8_t *row = w + (size_t)e * fmt_matrix_bytes(FMT, 1, H);
  const uint16_t *srow = fmt_quant(FMT) ? s + (size_t)e * (H / kGroup) : nullptr;
  float acc = 0.0f;
  const int nch = H / EPC;
  for (int c = 0; c < nch; c++) {
    float wv[EPC];
    router_chunk<FMT>(row, srow, c, wv);
#pragma unroll
    for (int i = 0; i < EPC; i++) acc = acc + xs[c * EPC + i] * wv[i];
  }
  logits[(size_t)t * E + e] = acc;
}

// Register-tiled SIMT product for many tokens: a 256-thread block computes a
// 64-token x 64-expert tile, 4x4 outputs per thread, staging 32-wide k slices
// of x and of the router in LDS.  Every output still sums its products in h
// order, so the result equals the row-wise kernel's bit for bit.
template <int FMT>
__global__ void __launch_bounds__(256) router_tiled_kernel(const float *__restrict__ x, int T, int H,
                                                           const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ s, int E,
                                                           float *__restrict__ logits) {
#pragma clang fp contract(off)
  constexpr int KB = 32, TM = 64, TN = 64, PAD = 4;
  __shared__ __align__(16) float xs[KB][TM + PAD];
  __shared__ __align__(16) float ws[KB][TN + PAD];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int t0 = blockIdx.y * TM, e0 = blockIdx.x * TN;
  constexpr int EPC = Chunk<FMT>::kElems;
  constexpr int CPR = KB / EPC;  // 16-byte chunks per row per k slice
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
  const int nsc = H / kGroup;

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;

  for (int k0 = 0; k0 < H; k0 += KB) {
    // x slice: TM rows x 32 floats, 8 float4 per row.
    for (int i = tid; i < TM * (KB / 4); i += 256) {
      int r = i / (KB / 4), c4 = i % (KB / 4);
      int t = t0 + r;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t < T) v = *reinterpret_cast<const float4 *>(x + (size_t)t * H + k0 + c4 * 4);
      xs[c4 * 4 + 0][r] = v.x;
      xs[c4 * 4 + 1][r] = v.y;
      xs[c4 * 4 + 2][r] = v.z;
      xs[c4 * 4 + 3][r] = v.w;
    }
    // router slice: TN rows x 32 elements, widened to f32.
    for (int i = tid; i < TN * CPR; i += 256) {
      int r = i / CPR, c = i % CPR;
      int e = e0 + r;
      float wv[EPC];
      if (e < E) {
        router_chunk<FMT>(w + (size_t)e * row_bytes, fmt_quant(FMT) ? s + (size_t)e * nsc : nullptr,
                          k0 / EPC + c, wv);
      } else {
#pragma unroll
        for (int q = 0; q < EPC; q++) wv[q] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < EPC; q++) ws[c * EPC + q][r] = wv[q];
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < KB; kk++) {
      float4 a = *reinterpret_cast<const float4 *>(&xs[kk][ty * 4]);
      float4 b = *reinterpret_cast<const float4 *>(&ws[kk][tx * 4]);
      const float av[4] = {a.x, a.y, a.z, a.w};
      const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + av[i] * bv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int t = t0 + ty * 4 + i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int e = e0 + tx * 4 + j;
      if (e < E) logits[(size_t)t * E + e] = acc[i][j];
    }
  }
}

template <int FMT>
static hipError_t router_logits_fmt(const float *x, int T, const DevMat &r, float *logits,
                                    hipStream_t st) {
  const int H = r.cols, E = r.rows;
  if (T <= 32) {
    dim3 grid((E + 63) / 64, T);
    hipLaunchKernelGGL(router_rowwise_kernel<FMT>, grid, dim3(64), (size_t)H * sizeof(float), st, x,
                       T, H, r.w, r.s, E, logits);
  } else {
    dim3 grid((E + 63) / 64, (T + 63) / 64);
    hipLaunchKernelGGL(router_tiled_kernel<FMT>, grid, dim3(256), 0, st, x, T, H, r.w, r.s, E,
                       logits);
  }
  return hipGetLastError();
}

hipError_t launch_router_logits(const float *x, int T, const DevMat &router, float *logits,
                                hipStream_t st) {
  switch (router.fmt) {
  case kF32: return router_logits_fmt<kF32>(x, T, router, logits, st);
  case kBF16: return router_logits_fmt<kBF16>(x, T, router, logits, st);
  case kINT8: return router_logits_fmt<kINT8>(x, T, router, logits, st);
  default: return router_logits_fmt<kINT4>(x, T, router, logits, st);
  }
}

// One wavefront per token.  softmax as model/tensors.go:106-121: max, then
// v = float32(exp(float64(l - max))) summed sequentially in expert order, then
// v / sum.  Selection (model/moe.go:44-53 generalised to the first `scope`
// candidates): k rounds of a wavefront arg-max on (p descending, index
// ascending), which is exactly the order of the reference's stable insertion
// sort.  Renormalisation (moe.go:54-57, 63): wSum summed in rank order,
// w = p / (wSum + 1e-9f).
constexpr int kMaxE = 1024;
constexpr int kMaxK = 64;

__global__ void __launch_bounds__(64) softmax_select_kernel(const float *__restrict__ logits, int T,
                                                            int E, int k, int scope,
                                                            int32_t *__restrict__ ids,
                                                            float *__restrict__ weights) {
#pragma clang fp contract(off)
  __shared__ float buf[kMaxE];
  __shared__ float selp[kMaxK];
  __shared__ int seli[kMaxK];
  __shared__ float ssum;
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int NJ = kMaxE / 64;
  const float *lt = logits + (size_t)t * E;
  float v[NJ];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    int e = lane + 64 * j;
    v[j] = e < E ? lt[e] : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    int e = lane + 64 * j;
    if (e < E) {
      v[j] = (float)exp((double)(v[j] - mx));
      buf[e] = v[j];
    }
  }
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int e = 0; e < E; e++) sum = sum + buf[e];
    ssum = sum;
  }
  __syncthreads();
  const float sum = ssum;
  float key[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    int e = lane + 64 * j;
    float p = v[j] / sum;
    v[j] = p;
    // NaN ranks below every number so that k valid ids are always produced.
    key[j] = (e < scope && p == p) ? p : -INFINITY;
  }
  uint32_t taken = 0;
  for (int r = 0; r < k; r++) {
    float bk = -INFINITY, bp = 0.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      int e = lane + 64 * j;
      bool cand = e < scope && !((taken >> j) & 1u);
      if (cand && (key[j] > bk || (key[j] == bk && e < bi))) {
        bk = key[j];
        bp = v[j];
        bi = e;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      float ok = __shfl_xor(bk, o, 64);
      float op = __shfl_xor(bp, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (ok > bk || (ok == bk && oi < bi)) {
        bk = ok;
        bp = op;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == 0) {
      selp[r] = bp;
      seli[r] = bi;
    }
  }
  __syncthreads();
  if (lane == 0) {
    float wsum = 0.0f;
    for (int r = 0; r < k; r++) wsum = wsum + selp[r];
    const float den = wsum + 1e-9f;
    for (int r = 0; r < k; r++) {
      ids[(size_t)t * k + r] = seli[r];
      weights[(size_t)t * k + r] = selp[r] / den;
    }
  }
}

hipError_t launch_softmax_select(const float *logits, int T, int E, int k, int scope,
                                 int32_t *ids, float *weights, hipStream_t st) {
  hipLaunchKernelGGL(softmax_select_kernel, dim3(T), dim3(64), 0, st, logits, T, E, k, scope, ids,
                     weights);
  return hipGetLastError();
}

}  // namespace qmoe
