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
#include "norm_common.hpp"
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
// With xb, workgroups past the token tiles (blockIdx.y >= ceil(T / TM), last
// in dispatch order) only store x rounded to bf16 (the batched GEMMs' A
// operand), TM tokens each, on the CUs the VALU-bound logit tiles release at
// their end instead of in a launch of their own.
template <int FMT, int RM, int RN, int KB>
__global__ void __launch_bounds__(256) router_tiled_kernel(const float *__restrict__ x, int T, int H,
                                                           const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ s, int E,
                                                           float *__restrict__ logits, uint16_t *__restrict__ xb) {
#pragma clang fp contract(off)
  constexpr int TM = 16 * RM, TN = 16 * RN, LD = KB + 4;
  __shared__ __align__(16) float xs[TM][LD];
  __shared__ __align__(16) float ws[TN][LD];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int t0 = blockIdx.y * TM, e0 = blockIdx.x * TN;
  const int ntok = (T + TM - 1) / TM;
  if ((int)blockIdx.y >= ntok) {
    const int c0 = ((blockIdx.y - ntok) * gridDim.x + blockIdx.x) * TM;  // first token of this block
    const int rows = min(TM, T - c0);
    for (int i = tid * 4; i < rows * H; i += 256 * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)c0 * H + i);
      *reinterpret_cast<uint2 *>(xb + (size_t)c0 * H + i) =
          make_uint2((uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16),
                     (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16));
    }
    return;
  }
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
static hipError_t router_logits_fmt(const float *x, int T, const DevMat &r, float *logits, uint16_t *xb,
                                    hipStream_t st) {
  const int H = r.cols, E = r.rows;
  if (T <= 32) {
    dim3 grid((E + 63) / 64, T);
    QMOE_LAUNCH(router_rowwise_kernel<FMT>, grid, dim3(64), (size_t)H * sizeof(float), st, x,
                       T, H, r.w, r.s, E, logits);
  } else {
    // two experts of one token per lane (two waves per SIMD at T x E = 2^18:
    // C3 router 64 -> 50 us against 2x2 outputs per lane at one wave per
    // SIMD, 54 us at one output per lane); 2x2 per lane only once that still
    // gives every CU four workgroups
    const bool wide = (int64_t)T * E >= (int64_t)16 * 256 * 256;
    // the x conversion rows: ceil(T / TM) blocks of TM tokens after the token tiles
    auto xrows = [&](int gx, int tm) { return xb ? ((T + tm - 1) / tm + gx - 1) / gx : 0; };
    const int gx11 = (E + 15) / 16, gx22 = (E + 31) / 32;
    const dim3 b(256), g11(gx11, (T + 15) / 16 + xrows(gx11, 16)), g22(gx22, (T + 31) / 32 + xrows(gx22, 32)),
        g12(gx22, (T + 15) / 16 + xrows(gx22, 16));
    if (H % 64 == 0) {
      if (wide)
        QMOE_LAUNCH((router_tiled_kernel<FMT, 2, 2, 64>), g22, b, 0, st, x, T, H, r.w, r.s, E, logits, xb);
      else if (E >= 32)
        QMOE_LAUNCH((router_tiled_kernel<FMT, 1, 2, 64>), g12, b, 0, st, x, T, H, r.w, r.s, E, logits, xb);
      else
        QMOE_LAUNCH((router_tiled_kernel<FMT, 1, 1, 64>), g11, b, 0, st, x, T, H, r.w, r.s, E, logits, xb);
    } else {
      if (wide)
        QMOE_LAUNCH((router_tiled_kernel<FMT, 2, 2, 32>), g22, b, 0, st, x, T, H, r.w, r.s, E, logits, xb);
      else
        QMOE_LAUNCH((router_tiled_kernel<FMT, 1, 1, 32>), g11, b, 0, st, x, T, H, r.w, r.s, E, logits, xb);
    }
  }
  return hipGetLastError();
}

hipError_t launch_router_logits(const float *x, int T, const DevMat &router, float *logits, uint16_t *xb,
                                hipStream_t st) {
  if (xb && T <= 32) return hipErrorInvalidValue;  // only the tiled kernels (T > 32) store xb
  switch (router.fmt) {
  case kF32: return router_logits_fmt<kF32>(x, T, router, logits, xb, st);
  case kBF16: return router_logits_fmt<kBF16>(x, T, router, logits, xb, st);
  case kINT8: return router_logits_fmt<kINT8>(x, T, router, logits, xb, st);
  default: return router_logits_fmt<kINT4>(x, T, router, logits, xb, st);
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
// also initialises out[t] when zero_out != nullptr (the fused expert kernel
// accumulates into it): to resid[t], the residual stream, when given, else 0.
// With n.w (the post-attention norm) x is the residual stream: every block
// normalises its token into LDS first (certified as in norm.hip) and block
// (0, t) stores the normed token into n.xn for the expert kernel.
template <int FMT, int CPL>
__global__ void __launch_bounds__(256) router_sb_kernel(const float *__restrict__ x, int H,
                                                        const uint8_t *__restrict__ w,
                                                        const uint16_t *__restrict__ s, int E,
                                                        double *__restrict__ sb, float *zero_out,
                                                        const float *resid, RouterNorm n) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float xl[];  // (H) the normed token, when n.w
  const int t = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  const float *xt = x + (size_t)t * H;
  if (n.w) {
    __shared__ double s_part[4];
    __shared__ float s_inv;
    double sq = 0.0;
    for (int i = threadIdx.x * 4; i < H; i += 1024) {
      const float4 v = *reinterpret_cast<const float4 *>(xt + i);
      *reinterpret_cast<float4 *>(xl + i) = v;
      sq += (double)v.x * (double)v.x;
      sq += (double)v.y * (double)v.y;
      sq += (double)v.z * (double)v.z;
      sq += (double)v.w * (double)v.w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_down(sq, off, 64);
    if (lane == 0) s_part[wave] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
      const double sp = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
      float inv;
      if (!norm_certify(sp, H, n.eps, &inv) || n.force_seq) {
        double q = 0.0;
        for (int i = 0; i < H; i++) q += (double)xl[i] * (double)xl[i];
        inv = norm_inv(q, H, n.eps);
        if (blockIdx.x == 0 && n.redo) atomicAdd(n.redo, 1u);
      }
      s_inv = inv;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = threadIdx.x * 4; i < H; i += 1024) {
      float4 v = *reinterpret_cast<const float4 *>(xl + i);
      const float4 g = *reinterpret_cast<const float4 *>(n.w + i);
      v.x = (v.x * inv) * (1.0f + g.x);
      v.y = (v.y * inv) * (1.0f + g.y);
      v.z = (v.z * inv) * (1.0f + g.z);
      v.w = (v.w * inv) * (1.0f + g.w);
      *reinterpret_cast<float4 *>(xl + i) = v;
      if (blockIdx.x == 0) *reinterpret_cast<float4 *>(n.xn + (size_t)t * H + i) = v;
    }
    __syncthreads();
    xt = xl;
  }
  if (zero_out && blockIdx.x == 0)
    for (int i = threadIdx.x; i < H; i += 256) zero_out[(size_t)t * H + i] = resid ? resid[(size_t)t * H + i] : 0.0f;
  if (e >= E) return;
  const uint8_t *row = w + (size_t)e * fmt_matrix_bytes(FMT, 1, H);
  const uint16_t *srow = fmt_quant(FMT) ? s + (size_t)e * (H / kGroup) : nullptr;
  double S, B;
  router_sb_wave<FMT, CPL>(xt, H, row, srow, S, B);
  if (lane == 0) {
    double *d = sb + ((size_t)t * E + e) * 2;
    d[0] = S;
    d[1] = B;
  }
}

template <int FMT>
static bool sb_fmt(const float *x, int T, const DevMat &r, double *sb, float *zero_out, const float *resid,
                   const RouterNorm &n, hipStream_t st) {
  constexpr int EPC = Chunk<FMT>::kElems;
  const int H = r.cols, E = r.rows;
  const int cpl = (H / EPC + 63) / 64;
  dim3 grid((E + 3) / 4, T);
  const size_t lds = n.w ? (size_t)H * 4 : 0;
#define L(C) \
  QMOE_LAUNCH((router_sb_kernel<FMT, C>), grid, dim3(256), lds, st, x, H, r.w, r.s, E, sb, zero_out, resid, n)
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
                            const float *resid, const RouterNorm &n, hipStream_t st) {
  switch (router.fmt) {
  case kF32: sb_fmt<kF32>(x, T, router, sb, zero_out, resid, n, st); break;
  case kBF16: sb_fmt<kBF16>(x, T, router, sb, zero_out, resid, n, st); break;
  case kINT8: sb_fmt<kINT8>(x, T, router, sb, zero_out, resid, n, st); break;
  default: sb_fmt<kINT4>(x, T, router, sb, zero_out, resid, n, st); break;
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

// ---- certified router partials for many tokens on the matrix cores (bf16
// router, H a multiple of 64 and at most 8192)
//
// x is split exactly into three bf16 parts, x = x1 + x2 + x3 (truncations:
// each remainder is exact in f32 and the last has at most 8 significant
// bits), plus |x| rounded up to bf16.  The matrix cores then give, per
// 64-wide k block, the block sum of the exact products x_p * w of all three
// parts (one f32 accumulator, 192 terms) and of |x|up * |w|.  Per (token,
// expert) the kernel keeps in f32 the running estimate S (block by block),
// A = the sum of |S| at the block ends, and P = the running sum of the |.|
// products, and writes {S, B} with B a rigorous bound on
// |reference logit - S|:
//   errS = 1.004 g193 P' + u A'                 (MFMA sums of 193 terms, the
//                                                 running sum)
//   sum_h |S_h| <= 64 (A' + nb errS) + 64 P' + H u P'   (prefix sums inside a
//                                                 block bounded by the last
//                                                 block end plus the block's
//                                                 |products|)
//   B = u (1 + 2Hu + 1e-9) sum_h |S_h| + u (1 + u) P' + errS + 1e-25
// with u = 2^-24, gn = nu / (1 - nu), nb = H / 64, and A', P' the f32 sums
// scaled up by their own rounding (and P' by the MFMA's).  The first term is
// the reference's sequential f32 sum (model/tensors.go:77-89) as the decode
// router bounds it; u P' covers its product roundings.  Pieces: planes of T*H
// bf16, in the order x1, x2, x3, |x|up.
constexpr int kCertPitch = 72;  // LDS row pitch of a 64-wide bf16 piece row (no bank conflicts)

// Piece p of x (as bf16 bits): x1, x2, x3 = the successive bf16
// truncations (each remainder is exact in f32; the third has at most 8
// significant bits), p = 3: |x| rounded up to bf16.
template <int P>
__device__ __forceinline__ uint32_t x_piece(float v) {
  const uint32_t b = __float_as_uint(v);
  if constexpr (P == 3) return ((b & 0x7fffffffu) + 0xffffu) >> 16;
  const float r1 = v - __uint_as_float(b & 0xffff0000u);  // exact
  if constexpr (P == 0) return b >> 16;
  const uint32_t b1 = __float_as_uint(r1);
  if constexpr (P == 1) return b1 >> 16;
  const float r2 = r1 - __uint_as_float(b1 & 0xffff0000u);  // exact
  return __float_as_uint(r2) >> 16;
}

typedef __bf16 cert_bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float cert_f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
// native 16-byte vectors: the HIP uint4 struct is copied through private
// memory in these register arrays
typedef unsigned int cert_u32x4 __attribute__((ext_vector_type(4)));

// The MFMAs of one 64-wide k block (four 16-wide steps, the three x parts
// against w into acc[0], |x|up against |w| into acc[1]); the first step
// takes a zero accumulator operand, so acc needs no clearing between blocks.
__device__ __forceinline__ void cert_mfma_block(const uint16_t *as, int l32, int hi, const cert_u32x4 (&wc)[4],
                                                cert_f32x16 (&acc)[2]) {
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
    const int ko = l32 * kCertPitch + 16 * ks + 8 * hi;
    const cert_u32x4 wa = wc[ks] & 0x7fff7fffu;
    const cert_bf16x8 bw = __builtin_bit_cast(cert_bf16x8, wc[ks]);
    const cert_bf16x8 bwa = __builtin_bit_cast(cert_bf16x8, wa);
    cert_bf16x8 av[4];
#pragma unroll
    for (int p = 0; p < 4; p++) av[p] = *reinterpret_cast<const cert_bf16x8 *>(as + p * 32 * kCertPitch + ko);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[0], bw, ks ? acc[0] : cert_f32x16{}, 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[3], bwa, ks ? acc[1] : cert_f32x16{}, 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[1], bw, acc[0], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[2], bw, acc[0], 0, 0, 0);
  }
}

// Piece P of 8 consecutive x values, as packed bf16 pairs (element 2i in
// the low half of word i).
template <int P>
__device__ __forceinline__ cert_u32x4 cert_piece8(const float4 (&v)[2]) {
  cert_u32x4 out;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    out[2 * i] = x_piece<P>(v[i].x) | (x_piece<P>(v[i].y) << 16);
    out[2 * i + 1] = x_piece<P>(v[i].z) | (x_piece<P>(v[i].w) << 16);
  }
  return out;
}

// A block's sums folded into S, A, P.
__device__ __forceinline__ void cert_fold(cert_f32x16 (&acc)[2], float (&S)[16], float (&A)[16], float (&P)[16]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 16; i++) {
    S[i] = S[i] + acc[0][i];
    A[i] = A[i] + fabsf(S[i]);
    P[i] = P[i] + acc[1][i];
  }
}

// One workgroup: 32 tokens x 128 experts, wave v the experts 128 bx + 32 v +
// (lane % 32).  The 32 x 64 piece tiles of a k block are staged in LDS once
// for the four waves (double buffered, one barrier per block): each thread
// loads 8 f32 of x (two blocks ahead) and stores those 8 elements of all four
// pieces; each wave keeps its router fragments in registers, loaded two blocks
// ahead.
// With qzero, workgroup (0, 0) also clears the selection's exact queue (its
// count and the first nq per-token workgroup counts) for the launches after it.
__global__ void __launch_bounds__(256, 1) router_cert_mfma_kernel(const float *__restrict__ x, int T, int H,
                                                               const uint16_t *__restrict__ w, int E,
                                                               double *__restrict__ sb, int *__restrict__ fbl,
                                                               uint32_t *__restrict__ qcnt, int nq) {
#pragma clang fp contract(off)
  __shared__ __align__(16) uint16_t at[2][4][32 * kCertPitch];
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  if (fbl && blockIdx.x == 0 && blockIdx.y == 0) {
    if (tid == 0) fbl[0] = 0;
    for (int i = tid; i < nq; i += 256) qcnt[i] = 0;
  }
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.y * 32;
  const int ew0 = blockIdx.x * 128 + wv * 32;  // first expert of this wave (uniform)
  const bool live = ew0 < E;
  const int e = ew0 + l32;
  const uint16_t *wrow = w + (size_t)min(e, E - 1) * H + 8 * hi;
  // A staging: thread -> row tid / 8, elements [8 (tid % 8), +8) of the k block
  const int sr = tid >> 3, sc = tid & 7;
  const float *asrc = x + (size_t)min(t0 + sr, T - 1) * H + sc * 8;
  // two register sets, loaded two blocks ahead (block indices clamped; the
  // loads past the end are never used)
  const int nb = H / 64;
  float4 an0[2], an1[2];
  cert_u32x4 wn0[4], wn1[4];  // the two register sets, named apart
  cert_f32x16 acc[2];
  float S[16], A[16], P[16];
#pragma unroll
  for (int i = 0; i < 16; i++) S[i] = A[i] = P[i] = 0.0f;
  // block blk's loads into register set (AN, WN) (block clamped: loads past
  // the end are never used)
#define CERT_LOAD(AN, WN, blk)                                                                  \
  do {                                                                                          \
    const int k0_ = min((blk), nb - 1) * 64;                                                    \
    _Pragma("unroll") for (int i_ = 0; i_ < 2; i_++)                                            \
        AN[i_] = *reinterpret_cast<const float4 *>(asrc + k0_ + 4 * i_);                         \
    _Pragma("unroll") for (int ks_ = 0; ks_ < 4; ks_++)                                         \
        WN[ks_] = *reinterpret_cast<const cert_u32x4 *>(wrow + k0_ + 16 * ks_);                  \
  } while (0)
  // block blk from register set (AN, WN) through LDS buffer BUF, then the
  // set's loads for block blk + 2
#define CERT_BLOCK(AN, WN, BUF, blk)                                                            \
  do {                                                                                          \
    *reinterpret_cast<cert_u32x4 *>(&at[BUF][0][sr * kCertPitch + sc * 8]) = cert_piece8<0>(AN); \
    *reinterpret_cast<cert_u32x4 *>(&at[BUF][1][sr * kCertPitch + sc * 8]) = cert_piece8<1>(AN); \
    *reinterpret_cast<cert_u32x4 *>(&at[BUF][2][sr * kCertPitch + sc * 8]) = cert_piece8<2>(AN); \
    *reinterpret_cast<cert_u32x4 *>(&at[BUF][3][sr * kCertPitch + sc * 8]) = cert_piece8<3>(AN); \
    cert_u32x4 wc_[4];                                                                          \
    _Pragma("unroll") for (int ks_ = 0; ks_ < 4; ks_++) wc_[ks_] = WN[ks_];                     \
    CERT_LOAD(AN, WN, (blk) + 2);                                                               \
    __syncthreads();                                                                            \
    if (live) {                                                                                 \
      cert_mfma_block(&at[BUF][0][0], l32, hi, wc_, acc);                                       \
      cert_fold(acc, S, A, P);                                                                  \
    }                                                                                           \
  } while (0)
  CERT_LOAD(an0, wn0, 0);
  CERT_LOAD(an1, wn1, 1);
  for (int b = 0; b < nb; b += 2) {
    CERT_BLOCK(an0, wn0, 0, b);
    if (b + 1 < nb) CERT_BLOCK(an1, wn1, 1, b + 1);
  }
#undef CERT_BLOCK
#undef CERT_LOAD
  if (!live || e >= E) return;
  const double u = 0x1p-24, g65 = 65.0 * u / (1.0 - 65.0 * u), g193 = 193.0 * u / (1.0 - 193.0 * u);
  const double fs = 1.0 + 2.0 * nb * u;  // an f32 running sum of nb terms
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int t = t0 + 8 * (i >> 2) + 4 * hi + (i & 3);
    if (t >= T) continue;
    const double Pp = (double)P[i] * fs * (1.0 + 2.0 * g65), Ap = (double)A[i] * fs;
    const double errS = 1.004 * g193 * Pp + u * Ap;
    const double sumSh = 64.0 * (Ap + nb * errS) + 64.0 * Pp + H * u * Pp;
    const double Bv = u * (1.0 + 2.0 * H * u + 1e-9) * sumSh + u * (1.0 + u) * Pp + errS + 1e-25;
    *reinterpret_cast<double2 *>(sb + ((size_t)t * E + e) * 2) = make_double2((double)S[i], Bv);
  }
}

bool router_cert_mfma_supported(const DevMat &router) {
  return router.fmt == kBF16 && router.cols % 64 == 0 && router.cols <= 8192 && router.rows <= kMaxE;
}

hipError_t launch_router_cert_mfma(const float *x, int T, const DevMat &router, double *sb, int *fbl,
                                   uint32_t *qcnt, hipStream_t st) {
  const int H = router.cols, E = router.rows;
  QMOE_LAUNCH(router_cert_mfma_kernel, dim3((E + 127) / 128, (T + 31) / 32), dim3(256), 0, st, x, T, H,
              reinterpret_cast<const uint16_t *>(router.w), E, sb, fbl, qcnt, fbl ? kExactQueueMax : 0);
  return hipGetLastError();
}

// Selection for many tokens from the matrix-core partials (bf16 router), one
// wavefront per token for everything but the exact logits.  lo_k = the k-th largest lower bound S - B among the
// experts of the scope; every expert of the scope whose upper bound S + B
// reaches it (the true top k of the scope are among them) gets its reference
// logit computed exactly, one per lane (the sequential f32 sum of
// model/tensors.go:77-89 on x in LDS).  So does every expert, in the scope or
// not, whose upper bound reaches the largest lower bound over all E: the
// reference's softmax subtracts the largest of all E logits
// (tensors.go:106-121), which can lie outside the scope (scope = k is the
// reference's own selection, moe.go:45-53), and the roundings below are
// sized from it.  The scope's candidates are ranked by (logit desc, index
// asc), which is the reference's order (moe.go:44-57) whenever consecutive
// ranks are equal or apart by more than the f32 roundings of the softmax can
// merge (4 ulps of their distance to the max plus 2^-20), the k-th is that far
// above every other upper bound in the scope and no probability is
// subnormal; otherwise, or with more than 64 candidates, the token is queued
// in fbl ({count, tokens...}) for the exact path (all logits, exact softmax),
// which select_exact_kernel runs with a row per thread.
// Weights: e_r = fl(exp(fl(L_r - max))) as the reference rounds it, divided by
// the f64 softmax sum of the partials over all E, renormalised with moe.go:63's
// 1e-9.
// Two tokens per workgroup, one wave each for the bounds, the candidates and
// the certification; the exact logits of both tokens' candidates are computed
// lane-packed in between (by wave 0 alone when they fit 64 lanes), since a
// wave's VALU instructions cost the same however few lanes run the chains.
constexpr int kCandTokens = 2;
template <int NJ>
__global__ void __launch_bounds__(64 * kCandTokens) __attribute__((amdgpu_waves_per_eu(4)))
    select_candidates_kernel(const float *__restrict__ x, int T, DevMat router, int k, int scope,
                             const double *__restrict__ sb, int32_t *__restrict__ ids, float *__restrict__ weights,
                             int *__restrict__ fbl) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int list_all[kCandTokens][64], sorted_e_all[kCandTokens][64], ncand[kCandTokens];
  __shared__ float sorted_l_all[kCandTokens][64], cand_l[kCandTokens][64];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kCandTokens + wv;
  const bool live = t < T;
  const int E = router.rows, H = router.cols;
  int *list = list_all[wv], *sorted_e = sorted_e_all[wv];
  float *sorted_l = sorted_l_all[wv];
  float *xs = reinterpret_cast<float *>(smem) + (size_t)wv * H;
  if (live)
    for (int i = lane * 4; i < H; i += 256)
      *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + (size_t)t * H + i);
  double S[NJ], B[NJ];
  float key[NJ];       // lower bounds in the scope, rounded down to f32
  double glo = -INFINITY;  // the largest lower bound over all E
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    const double2 v = live && e < E ? reinterpret_cast<const double2 *>(sb + (size_t)t * E * 2)[e]
                                    : make_double2(-INFINITY, 0.0);
    S[j] = v.x;
    B[j] = v.y;
    const double lo = S[j] - B[j];
    if (e < E) glo = fmax(glo, lo);
    float f = (float)lo;
    if ((double)f > lo) {  // one f32 step down (f is finite here)
      const uint32_t u = __float_as_uint(f);
      f = f == 0.0f ? -0x1p-149f : __uint_as_float(f > 0.0f ? u - 1u : u + 1u);
    }
    key[j] = e < scope ? f : -INFINITY;
  }
  glo = wave_max_f64(glo);
  // lo_k: k rounds of a wavefront max over each lane's sorted keys
  float hk[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) hk[j] = key[j];
#pragma unroll
  for (int size = 2; size <= NJ; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < NJ; i++) {
        const int l = i ^ stride;
        if (l > i) {
          const bool sw = (i & size) == 0 ? hk[l] > hk[i] : hk[l] < hk[i];
          const float a = hk[i];
          hk[i] = sw ? hk[l] : hk[i];
          hk[l] = sw ? a : hk[l];
        }
      }
  float lo_k = -INFINITY;
  for (int r = 0; r < k; r++) {
    lo_k = wave_max_f32(hk[0]);
    const uint64_t win = __ballot(hk[0] == lo_k);
    const int wl = win ? __ffsll((unsigned long long)win) - 1 : 0;
    if (lane == wl) {
#pragma unroll
      for (int j = 0; j + 1 < NJ; j++) hk[j] = hk[j + 1];
      hk[NJ - 1] = -INFINITY;
    }
  }
  // candidates, compacted into list: in the scope with upper bound >= lo_k,
  // or (any index) with upper bound >= glo, which includes the maximum's expert
  int n = 0;
  double uo = -INFINITY;  // the largest upper bound among the scope's others
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    const double up = S[j] + B[j];
    const bool in = e < E && ((e < scope && up >= (double)lo_k) || up >= glo);
    const uint64_t m = __ballot(in);
    const int idx = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (in && idx < 64) list[idx] = e;
    n += __popcll(m);
    if (!in && e < scope && e < E) uo = fmax(uo, up);
  }
  uo = wave_max_f64(uo);
  bool ok = live && n <= 64;
  if (lane == 0) ncand[wv] = ok ? n : 0;
  __syncthreads();  // every wave's x, list and count
  // the exact reference logits of every candidate, lane-packed over the block
  {
    int g = threadIdx.x, tw = -1;
#pragma unroll
    for (int q = 0; q < kCandTokens; q++) {
      if (tw < 0 && g < ncand[q]) tw = q;
      else if (tw < 0) g -= ncand[q];
    }
    if (tw >= 0)
      cand_l[tw][g] = exact_row_logit<kBF16>(reinterpret_cast<const float *>(smem) + (size_t)tw * H, H,
                                            router.w + (size_t)list_all[tw][g] * H * 2, nullptr);
  }
  __syncthreads();
  if (ok) {
    float L = -INFINITY;
    int ce = 0x7fffffff;
    if (lane < n) {
      ce = list[lane];
      L = cand_l[wv][lane];
    }
    // the reference's maximum over all E logits (its expert is listed)
    const float Lmax = wave_max_f32(L);
    // rank among the scope's candidates: (logit desc, index asc)
    const bool ranked = lane < n && ce < scope;
    int rank = 0;
    for (int j = 0; j < n; j++) {
      const float Lj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(L), j));
      const int ej = __builtin_amdgcn_readlane(ce, j);
      rank += (ej < scope && (Lj > L || (Lj == L && ej < ce))) ? 1 : 0;
    }
    const int nsc = __popcll(__ballot(ranked));
    if (ranked) {
      sorted_l[rank] = L;
      sorted_e[rank] = ce;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    ok = nsc >= k;
    bool bad = false;
    if (ok && lane < k) {
      const float Lr = sorted_l[lane];
      // the next one down: the next candidate, and below the k-th the others' upper bounds
      const double nxt = lane + 1 < nsc ? (double)sorted_l[lane + 1] : -INFINITY;
      const double below = lane == k - 1 ? fmax(nxt, uo) : nxt;
      const double X = (double)Lmax - fmin((double)Lr, below > -INFINITY ? below : (double)Lr);
      if (!((double)Lmax - (double)Lr < 80.0)) bad = true;
      if (below > -INFINITY && (double)Lr != below && !((double)Lr - below > f32_4ulps(X) + 0x1p-20)) bad = true;
      if (lane == k - 1 && uo > -INFINITY && !((double)Lr - uo > f32_4ulps(X) + 0x1p-20)) bad = true;
    }
    ok = ok && !__ballot(bad);
    if (ok) {
      // softmax sum of the partials over all E (the 1e-9 of moe.go:63 is relative to it)
      double z = 0.0;
#pragma unroll
      for (int j = 0; j < NJ; j++)
        if (lane + 64 * j < E) z += exp(fmin(S[j], (double)Lmax) - (double)Lmax);
      z = wave_sum_f64(z);
      const float er = lane < k ? (float)exp((double)(sorted_l[lane] - Lmax)) : 0.0f;
      double esum = 0.0;
      for (int r = 0; r < k; r++)
        esum += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(er), r));
      if (lane < k) {
        ids[(size_t)t * k + lane] = sorted_e[lane];
        weights[(size_t)t * k + lane] = (float)(((double)er / z) / (esum / z + 1e-9));
      }
      return;
    }
  }
  // queued for the exact path
  if (live && lane == 0) fbl[1 + atomicAdd(fbl, 1)] = t;
}

// The exact path for the queued tokens: every logit (the sequential f32 sum,
// one row per lane), then the exact softmax and selection (select_exact_nj).
// A queued token's E rows are split over kQSplit workgroups of one wave, so
// that one token costs about one row's chain instead of every row streamed by
// one workgroup (C5: 512 rows on one CU took up to 80 us).  Each workgroup
// stores its logits into the entry's row of qlt and counts itself in
// qcnt[entry] (release); the last one (acquire) selects.  Entry q is taken by
// workgroups [kQSplit (q % kQPar), +kQSplit); entries from kQMax on (more than
// any call queues in practice) are routed whole by one workgroup.
constexpr int kQSplit = 16, kQPar = 16, kQMax = kExactQueueMax;
template <int NJ>
__global__ void __launch_bounds__(64) select_exact_kernel(const float *__restrict__ x, DevMat router, int k,
                                                          int scope, const int *__restrict__ fbl,
                                                          float *__restrict__ qlt, uint32_t *__restrict__ qcnt,
                                                          int32_t *__restrict__ ids, float *__restrict__ weights,
                                                          unsigned int *__restrict__ fallbacks) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_last;
  const int E = router.rows, H = router.cols, n = fbl[0], lane = threadIdx.x;
  float *xs = reinterpret_cast<float *>(smem);
  float *lt = xs + H;
  const int part = blockIdx.x % kQSplit, slot = blockIdx.x / kQSplit;
  const int per = (E + kQSplit - 1) / kQSplit;  // rows of a part (<= 64: E <= 1024)
  auto load_x = [&](int t) {
    __syncthreads();  // the previous entry's LDS reads are done
    for (int i = lane * 4; i < H; i += 256)
      *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + (size_t)t * H + i);
    __syncthreads();
  };
  for (int q = slot; q < n; q += kQPar) {
    const int t = fbl[1 + q];
    int32_t *gi = ids + (size_t)t * k;
    float *gw = weights + (size_t)t * k;
    if (q >= kQMax) {  // whole token in one workgroup (part 0)
      if (part != 0) continue;
      load_x(t);
      for (int e = lane; e < E; e += 64) lt[e] = exact_row_logit<kBF16, 16>(xs, H, router.w + (size_t)e * H * 2, nullptr);
      __syncthreads();
      select_exact_nj<NJ>(lt, E, k, scope, gi, gw, nullptr, nullptr);
      if (lane == 0) atomicAdd(fallbacks, 1u);
      continue;
    }
    load_x(t);
    const int e = part * per + lane;
    if (lane < per && e < E)
      qlt[(size_t)q * E + e] = exact_row_logit<kBF16, 16>(xs, H, router.w + (size_t)e * H * 2, nullptr);
    __threadfence();  // release this part's logits
    if (lane == 0) s_last = atomicAdd(qcnt + q, 1u) == kQSplit - 1;
    __syncthreads();
    if (s_last) {
      __threadfence();  // acquire every part's logits
      for (int i = lane; i < E; i += 64) lt[i] = __hip_atomic_load(qlt + (size_t)q * E + i, __ATOMIC_RELAXED,
                                                                      __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      select_exact_nj<NJ>(lt, E, k, scope, gi, gw, nullptr, nullptr);
      if (lane == 0) atomicAdd(fallbacks, 1u);
    }
  }
}

hipError_t launch_select_candidates(const float *x, int T, const DevMat &router, int k, int scope, const double *sb,
                                    int32_t *ids, float *weights, int *fbl, float *qlt, uint32_t *qcnt,
                                    unsigned int *fallbacks, hipStream_t st) {
  const size_t lds = (size_t)router.cols * 4 * kCandTokens;
#define L(NJ) QMOE_LAUNCH(select_candidates_kernel<NJ>, dim3((T + kCandTokens - 1) / kCandTokens), \
                          dim3(64 * kCandTokens), lds, st, x, T, router, k, scope, sb, ids, weights, fbl)
  QMOE_NJ_DISPATCH(router.rows, L);
#undef L
  const size_t lds2 = (size_t)router.cols * 4 + (size_t)router.rows * 4;
#define L(NJ) QMOE_LAUNCH(select_exact_kernel<NJ>, dim3(kQSplit * kQPar), dim3(64), lds2, st, x, router, k, scope, \
                          fbl, qlt, qcnt, ids, weights, fallbacks)
  QMOE_NJ_DISPATCH(router.rows, L);
#undef L
  return hipGetLastError();
}

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
