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
// (16 RM)-token x (16 RN)-expert tile, RM x RN outputs per thread (tokens
// ty + 16 i, experts tx + 16 j), staging KB-wide k slices (KB divides H) of x
// and of the router in LDS with k contiguous; the next slice is loaded raw into
// registers while the current one is multiplied.  Every output sums its
// products in h order, so the result equals the row-wise kernel's bit for bit.
template <int FMT, int RM, int RN, int KB>
__global__ void __launch_bounds__(256) router_tiled_kernel(const float *__restrict__ x, int T, int H,
                                                           const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ s, int E,
                                                           float *__restrict__ logits) {
#pragma clang fp contract(off)
  constexpr int TM = 16 * RM, TN = 16 * RN, LD = KB + 4;
  __shared__ __align__(16) float xs[TM][LD];
  __shared__ __align__(16) float ws[TN][LD];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int t0 = blockIdx.y * TM, e0 = blockIdx.x * TN;
  constexpr int EPC = Chunk<FMT>::kElems;
  constexpr int CPR = KB / EPC;                        // 16-byte router chunks per row per slice
  constexpr int NXP = TM * KB / 4, NWP = TN * CPR;     // float4 pieces of x, router chunks per slice
  constexpr int XPT = (NXP + 255) / 256, WPT = (NWP + 255) / 256;
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
  const int nsc = H / kGroup;

  // this thread's pieces of a slice: x piece p -> row p / (KB / 4), float4
  // (p % (KB / 4)); router chunk q -> row q / CPR, chunk q % CPR.  Rows are
  // clamped in bounds and the loads are unconditional (x_ok / w_ok zero the
  // stores), so the wait counts of the pipelined loads stay exact.
  const float *xsrc[XPT];
  bool x_in[XPT], x_ok[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int p = tid + 256 * i;
    const int r = min(p / (KB / 4), TM - 1);
    x_in[i] = p < NXP;
    x_ok[i] = x_in[i] && t0 + r < T;
    xsrc[i] = x + (size_t)min(t0 + r, T - 1) * H + (p % (KB / 4)) * 4;
  }
  const uint8_t *wrow[WPT];
  const uint16_t *wsrow[WPT];
  bool w_in[WPT], w_ok[WPT];
#pragma unroll
  for (int i = 0; i < WPT; i++) {
    const int q = tid + 256 * i;
    const int r = min(q / CPR, TN - 1);
    w_in[i] = q < NWP;
    w_ok[i] = w_in[i] && e0 + r < E;
    wrow[i] = w + (size_t)min(e0 + r, E - 1) * row_bytes;
    wsrow[i] = fmt_quant(FMT) ? s + (size_t)min(e0 + r, E - 1) * nsc : nullptr;
  }
  float4 xv[XPT];
  uint4 wraw[WPT];
  uint16_t wsc[WPT];
#pragma unroll
  for (int i = 0; i < WPT; i++) wsc[i] = 0;
  auto load_slice = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XPT; i++) xv[i] = *reinterpret_cast<const float4 *>(xsrc[i] + k0);
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int chunk = k0 / EPC + (tid + 256 * i) % CPR;
      wraw[i] = *reinterpret_cast<const uint4 *>(wrow[i] + (size_t)chunk * 16);
      if constexpr (fmt_quant(FMT)) wsc[i] = wsrow[i][(chunk * EPC) / kGroup];
    }
  };

  float acc[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; i++)
#pragma unroll
    for (int j = 0; j < RN; j++) acc[i][j] = 0.0f;
  load_slice(0);
  for (int k0 = 0; k0 < H; k0 += KB) {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int p = tid + 256 * i;
      if (x_in[i])
        *reinterpret_cast<float4 *>(&xs[p / (KB / 4)][(p % (KB / 4)) * 4]) =
            x_ok[i] ? xv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      if (!w_in[i]) continue;
      const int q = tid + 256 * i, r = q / CPR, c = q % CPR;
      float wv[EPC];
      widen_chunk<FMT>(wraw[i], wsc[i], wv);
#pragma unroll
      for (int q2 = 0; q2 < EPC; q2 += 4)
        *reinterpret_cast<float4 *>(&ws[r][c * EPC + q2]) =
            w_ok[i] ? make_float4(wv[q2], wv[q2 + 1], wv[q2 + 2], wv[q2 + 3]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    load_slice(min(k0 + KB, H - KB));
#pragma unroll
    for (int kk = 0; kk < KB; kk += 4) {
      float4 av[RM], bv[RN];
#pragma unroll
      for (int i = 0; i < RM; i++) av[i] = *reinterpret_cast<const float4 *>(&xs[ty + 16 * i][kk]);
#pragma unroll
      for (int j = 0; j < RN; j++) bv[j] = *reinterpret_cast<const float4 *>(&ws[tx + 16 * j][kk]);
#pragma unroll
      for (int i = 0; i < RM; i++)
#pragma unroll
        for (int j = 0; j < RN; j++) {
          acc[i][j] = acc[i][j] + av[i].x * bv[j].x;
          acc[i][j] = acc[i][j] + av[i].y * bv[j].y;
          acc[i][j] = acc[i][j] + av[i].z * bv[j].z;
          acc[i][j] = acc[i][j] + av[i].w * bv[j].w;
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < RM; i++) {
    const int t = t0 + ty + 16 * i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < RN; j++) {
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
    // 2x2 outputs per lane while that still fills 256 CUs four waves deep,
    // else one output per lane and four times the workgroups
    const bool wide = (int64_t)T * E >= (int64_t)4 * 256 * 256;
    const dim3 b(256), g11((E + 15) / 16, (T + 15) / 16), g22((E + 31) / 32, (T + 31) / 32);
    if (H % 64 == 0) {
      if (wide)
        QMOE_LAUNCH((router_tiled_kernel<FMT, 2, 2, 64>), g22, b, 0, st, x, T, H, r.w, r.s, E, logits);
      else
        QMOE_LAUNCH((router_tiled_kernel<FMT, 1, 1, 64>), g11, b, 0, st, x, T, H, r.w, r.s, E, logits);
    } else {
      if (wide)
        QMOE_LAUNCH((router_tiled_kernel<FMT, 2, 2, 32>), g22, b, 0, st, x, T, H, r.w, r.s, E, logits);
      else
        QMOE_LAUNCH((router_tiled_kernel<FMT, 1, 1, 32>), g11, b, 0, st, x, T, H, r.w, r.s, E, logits);
    }
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
  __shared__ int s_list[64];
  const int t = blockIdx.x;
  const int E = router.rows, H = router.cols;
  float *xs = reinterpret_cast<float *>(smem);
  float *lt = xs + H;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    double S[NJ], B[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int e = lane + 64 * j;
      const double2 v = e < E ? reinterpret_cast<const double2 *>(sb + (size_t)t * E * 2)[e] : make_double2(-INFINITY, 0.0);
      S[j] = v.x;
      B[j] = v.y;
    }
    double kth_lo = 0.0;
    bool c = certified_select_regs<NJ>(S, B, E, k, scope, ids + (size_t)t * k, weights + (size_t)t * k, nullptr,
                                       nullptr, -1, nullptr, &kth_lo);
    if (!c) {
      // exact logits for the few candidates in doubt first
      for (int i = lane; i < H; i += 64) xs[i] = x[(size_t)t * H + i];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
#define R(F)                                                                                                     \
  c = refine_select<F, NJ>(S, B, kth_lo, E, k, scope, xs, H, router.w, router.s, s_list, ids + (size_t)t * k, \
                           weights + (size_t)t * k, nullptr, nullptr)
      switch (router.fmt) {
      case kF32: R(kF32); break;
      case kBF16: R(kBF16); break;
      case kINT8: R(kINT8); break;
      default: R(kINT4); break;
      }
#undef R
      if (c && lane == 0) atomicAdd(fallbacks + 1, 1u);
    }
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
