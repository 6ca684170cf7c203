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
#include "router_common.hpp"
#include "select.hpp"

#include <math.h>

namespace qmoe {

constexpr int kMaxE = 1024;

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
// 32-token x 32-expert tile, 2 x 2 outputs per thread (tokens ty, ty + 16 and
// experts tx, tx + 16), staging 32-wide k slices of x and of the router in LDS
// with k contiguous.  Small tiles keep every SIMD busy: the work is one
// dependent f32 add chain of length H per output.  Every output still sums its
// products in h order, so the result equals the row-wise kernel's bit for bit.
template <int FMT>
__global__ void __launch_bounds__(256) router_tiled_kernel(const float *__restrict__ x, int T, int H,
                                                           const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ s, int E,
                                                           float *__restrict__ logits) {
#pragma clang fp contract(off)
  constexpr int KB = 32, TM = 32, TN = 32, LD = KB + 4;
  __shared__ __align__(16) float xs[TM][LD];
  __shared__ __align__(16) float ws[TN][LD];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int t0 = blockIdx.y * TM, e0 = blockIdx.x * TN;
  constexpr int EPC = Chunk<FMT>::kElems;
  constexpr int CPR = KB / EPC;  // 16-byte chunks per row per k slice
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
  const int nsc = H / kGroup;

  static_assert(TN * CPR <= 256, "one router chunk per thread and slice");
  // this thread's share of a slice: one float4 of x, at most one 16-byte
  // router chunk; the next slice is loaded raw into registers while the
  // current one is multiplied, and widened once it is stored
  const int xr = tid >> 3, xc4 = tid & 7;
  const bool x_ok = t0 + xr < T;
  const float *xsrc = x + (size_t)min(t0 + xr, T - 1) * H + xc4 * 4;
  const int wr = tid / CPR, wc = tid % CPR;
  const bool w_ok = tid < TN * CPR && e0 + wr < E;
  const uint8_t *wrow = w + (size_t)min(e0 + wr, E - 1) * row_bytes;
  const uint16_t *wsrow = fmt_quant(FMT) ? s + (size_t)min(e0 + wr, E - 1) * nsc : nullptr;
  float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
  uint4 wraw = make_uint4(0u, 0u, 0u, 0u);
  uint16_t wsc = 0;
  auto load_slice = [&](int k0) {
    if (x_ok) xv = *reinterpret_cast<const float4 *>(xsrc + k0);
    if (w_ok) {
      const int chunk = k0 / EPC + wc;
      wraw = *reinterpret_cast<const uint4 *>(wrow + (size_t)chunk * 16);
      if constexpr (fmt_quant(FMT)) wsc = wsrow[(chunk * EPC) / kGroup];
    }
  };

  float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  load_slice(0);
  for (int k0 = 0; k0 < H; k0 += KB) {
    *reinterpret_cast<float4 *>(&xs[xr][xc4 * 4]) = xv;
    if (tid < TN * CPR) {  // widen the router chunk exactly as router_chunk does
      float wv[EPC];
      const uint32_t u[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
      if constexpr (FMT == kF32) {
#pragma unroll
        for (int i = 0; i < 4; i++) wv[i] = __uint_as_float(u[i]);
      } else if constexpr (FMT == kBF16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          wv[2 * i] = __uint_as_float(u[i] << 16);
          wv[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
        }
      } else if constexpr (FMT == kINT8) {
        const float sc = f16_to_f32(wsc);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int b = 0; b < 4; b++) wv[4 * i + b] = (float)(int8_t)((u[i] >> (8 * b)) & 0xffu) * sc;
      } else {
        const float sc = f16_to_f32(wsc);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int b = 0; b < 4; b++) {
            const uint32_t byte = (u[i] >> (8 * b)) & 0xffu;
            wv[8 * i + 2 * b] = (float)((int)(byte >> 4) - 8) * sc;
            wv[8 * i + 2 * b + 1] = (float)((int)(byte & 0xfu) - 8) * sc;
          }
      }
#pragma unroll
      for (int q = 0; q < EPC; q++) ws[wr][wc * EPC + q] = w_ok ? wv[q] : 0.0f;
    }
    __syncthreads();
    if (k0 + KB < H) load_slice(k0 + KB);
#pragma unroll
    for (int kk = 0; kk < KB; kk += 4) {
      const float4 a0 = *reinterpret_cast<const float4 *>(&xs[ty][kk]);
      const float4 a1 = *reinterpret_cast<const float4 *>(&xs[ty + 16][kk]);
      const float4 b0 = *reinterpret_cast<const float4 *>(&ws[tx][kk]);
      const float4 b1 = *reinterpret_cast<const float4 *>(&ws[tx + 16][kk]);
      const float av[2][4] = {{a0.x, a0.y, a0.z, a0.w}, {a1.x, a1.y, a1.z, a1.w}};
      const float bv[2][4] = {{b0.x, b0.y, b0.z, b0.w}, {b1.x, b1.y, b1.z, b1.w}};
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = acc[i][j] + av[i][q] * bv[j][q];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int t = t0 + ty + 16 * i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int e = e0 + tx + 16 * j;
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
    QMOE_LAUNCH(router_rowwise_kernel<FMT>, grid, dim3(64), (size_t)H * sizeof(float), st, x,
                       T, H, r.w, r.s, E, logits);
  } else {
    dim3 grid((E + 31) / 32, (T + 31) / 32);
    QMOE_LAUNCH(router_tiled_kernel<FMT>, grid, dim3(256), 0, st, x, T, H, r.w, r.s, E,
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

// One wavefront per token: exact softmax + selection + renormalisation on

// One wavefront per token: exact softmax + selection + renormalisation on
// the exact logits (select.hpp).
template <int NJ>
__global__ void __launch_bounds__(64) softmax_select_kernel(const float *__restrict__ logits, int E, int k,
                                                            int scope, int32_t *__restrict__ ids,
                                                            float *__restrict__ weights) {
  const int t = blockIdx.x;
  select_exact_nj<NJ>(logits + (size_t)t * E, E, k, scope, ids + (size_t)t * k, weights + (size_t)t * k, nullptr,
                      nullptr);
}

hipError_t launch_softmax_select(const float *logits, int T, int E, int k, int scope, int32_t *ids,
                                 float *weights, hipStream_t st) {
#define L(NJ) QMOE_LAUNCH(softmax_select_kernel<NJ>, dim3(T), dim3(64), 0, st, logits, E, k, scope, ids, weights)
  QMOE_NJ_DISPATCH(E, L);
#undef L
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Certified router for decode-sized T (router_common.hpp): the exact logits
// above cost one dependent f32 add per h per (token, expert) -- about
// 2 instructions x H cycles of latency, several microseconds at T = 1.  This
// path writes {S, B} per (token, expert) instead; selection (select.hpp)
// certifies every rank on them or recomputes the token's exact logits, so the
// ids are the reference's bit for bit either way.
// ---------------------------------------------------------------------------

// One wavefront per (token, expert) writes sb[(t, e)] = {S, B}.  Block (0, t)
// also zeroes out[t] when zero_out != nullptr (the fused expert kernel
// accumulates into it).
template <int FMT, int CPL>
__global__ void __launch_bounds__(256) router_sb_kernel(const float *__restrict__ x, int H,
                                                        const uint8_t *__restrict__ w,
                                                        const uint16_t *__restrict__ s, int E,
                                                        double *__restrict__ sb, float *__restrict__ zero_out) {
  const int t = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  if (zero_out && blockIdx.x == 0)
    for (int i = threadIdx.x; i < H; i += 256) zero_out[(size_t)t * H + i] = 0.0f;
  if (e >= E) return;
  const uint8_t *row = w + (size_t)e * fmt_matrix_bytes(FMT, 1, H);
  const uint16_t *srow = fmt_quant(FMT) ? s + (size_t)e * (H / kGroup) : nullptr;
  double S, B;
  router_sb_wave<FMT, CPL>(x + (size_t)t * H, H, row, srow, S, B);
  if (lane == 0) {
    double *d = sb + ((size_t)t * E + e) * 2;
    d[0] = S;
    d[1] = B;
  }
}

template <int FMT>
static bool sb_fmt(const float *x, int T, const DevMat &r, double *sb, float *zero_out, hipStream_t st) {
  constexpr int EPC = Chunk<FMT>::kElems;
  const int H = r.cols, E = r.rows;
  const int cpl = (H / EPC + 63) / 64;
  dim3 grid((E + 3) / 4, T);
#define L(C) QMOE_LAUNCH((router_sb_kernel<FMT, C>), grid, dim3(256), 0, st, x, H, r.w, r.s, E, sb, zero_out)
  // at most 64 products per lane (H <= 4096)
  switch (cpl) {
  case 1: L(1); return true;
  case 2: if constexpr (2 * EPC <= 64) { L(2); return true; } return false;
  case 4: if constexpr (4 * EPC <= 64) { L(4); return true; } return false;
  case 8: if constexpr (8 * EPC <= 64) { L(8); return true; } return false;
  default: return false;
  }
#undef L
}

bool router_certified_supported(const DevMat &router) {
  const int epc = router.fmt == kF32 ? 4 : router.fmt == kBF16 ? 8 : router.fmt == kINT8 ? 16 : 32;
  const int cpl = (router.cols / epc + 63) / 64;
  return router.cols <= 4096 && router.rows <= kMaxE && (cpl == 1 || cpl == 2 || cpl == 4 || cpl == 8) &&
         cpl * epc <= 64;
}

hipError_t launch_router_sb(const float *x, int T, const DevMat &router, double *sb, float *zero_out,
                            hipStream_t st) {
  switch (router.fmt) {
  case kF32: sb_fmt<kF32>(x, T, router, sb, zero_out, st); break;
  case kBF16: sb_fmt<kBF16>(x, T, router, sb, zero_out, st); break;
  case kINT8: sb_fmt<kINT8>(x, T, router, sb, zero_out, st); break;
  default: sb_fmt<kINT4>(x, T, router, sb, zero_out, st); break;
  }
  return hipGetLastError();
}

// One block per token: certified selection from S/B; on failure the block
// computes the exact logits and selects on them.
template <int NJ>
__global__ void __launch_bounds__(256) select_cert_kernel(const float *__restrict__ x, DevMat router, int k,
                                                          int scope, const double *__restrict__ sb,
                                                          int32_t *__restrict__ ids, float *__restrict__ weights,
                                                          unsigned int *__restrict__ fallbacks) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int ok;
  const int t = blockIdx.x;
  const int E = router.rows, H = router.cols;
  float *xs = reinterpret_cast<float *>(smem);
  float *lt = xs + H;
  if (threadIdx.x < 64) {
    const bool c = certified_select_nj<NJ>(sb + (size_t)t * E * 2, E, k, scope, ids + (size_t)t * k,
                                           weights + (size_t)t * k, nullptr, nullptr);
    if (threadIdx.x == 0) ok = c;
  }
  __syncthreads();
  if (ok) return;
  for (int i = threadIdx.x; i < H; i += 256) xs[i] = x[(size_t)t * H + i];
  __syncthreads();
  exact_logits_block(xs, H, router.w, router.s, router.fmt, E, lt, 256);
  __syncthreads();
  if (threadIdx.x < 64)
    select_exact_nj<NJ>(lt, E, k, scope, ids + (size_t)t * k, weights + (size_t)t * k, nullptr, nullptr);
  if (threadIdx.x == 0) atomicAdd(fallbacks, 1u);
}

size_t select_cert_lds_bytes(int E, int H) { return (size_t)H * 4 + (size_t)E * 4; }

hipError_t launch_select_cert(const float *x, int T, const DevMat &router, int k, int scope, const double *sb,
                              int32_t *ids, float *weights, unsigned int *fallbacks, hipStream_t st) {
  const size_t lds = select_cert_lds_bytes(router.rows, router.cols);
#define L(NJ) QMOE_LAUNCH(select_cert_kernel<NJ>, dim3(T), dim3(256), lds, st, x, router, k, scope, sb, ids, \
                               weights, fallbacks)
  QMOE_NJ_DISPATCH(router.rows, L);
#undef L
  return hipGetLastError();
}

}  // namespace qmoe
