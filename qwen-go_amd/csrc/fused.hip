// fused.hip -- the expert products of a decode-sized forward in one kernel.
//
// Each token's k * I routed intermediate rows (plus the Is rows of the shared
// expert, model/moe.go:86-97) are split evenly over about one block per CU; a
// block holds at most two runs of rows (a run = consecutive rows of one expert).
// Eight waves; wave 0 is also the control wave:
//   control: the certified selection from the router partials (select.hpp):
//            after the round of rank r it publishes that rank's tentative expert
//            in LDS, then finishes the rounds, certifies the order and computes
//            the renormalised weights while the data waves stream.  With
//            precomputed routing it just reads it.  For a shared-expert run it
//            computes the scalar gate sigmoid(sharedGate . x).
//   all:     each lane group owns a contiguous range of the block's rows and
//            streams, two rows ahead, each row's gate and up rows and its row of
//            the transposed (I, H) down matrix into registers; per row it forms
//            act = silu(g) * u in f32 (model/moe.go:64-75) and accumulates
//            act * down_row in registers, flushing the sum into the run's LDS
//            accumulator (f32 LDS atomics) when the run -- or, for the group-32
//            formats, the 32-row scale group -- changes.
// The routing weight (or the shared gate) multiplies a run's accumulator once,
// at the end, so the data waves can start on the tentative experts before the
// weights are known; a run whose final expert differs from the tentative one
// is recomputed.  When certification fails the whole block computes the
// token's exact sequential logits and selects on them.  The block's result is
// added into out with f32 atomics (model/moe.go:76-84); out must be zero on
// entry.  The atomics make the order of the final f32 sums run-dependent
// (within f32 rounding of the reference's rank-ordered sum).
#include "gemv_common.hpp"
#include "norm_common.hpp"
#include "router_common.hpp"
#include "select.hpp"

namespace qmoe {

constexpr int kCtl = 64;                      // control wave (wave 0)
constexpr int kFusedBlock = 512;              // every wave, the control wave included, streams rows
constexpr int kData = kFusedBlock;
constexpr int kMaxRows = 192;                 // intermediate rows per block, at most

// LDS: x, two run accumulators, exact logits (fallback); then, for the burst
// mode, each data wave's down rows (kBurstKB KiB per wave).
constexpr int kBurstKB = 16;
__host__ __device__ inline size_t fused_head_bytes(int H, int E) {
  return ((size_t)(3 * H + E) * 4 + 15) / 16 * 16;
}
constexpr uint64_t kRankGapTicks = 40;         // 0.4 us at the 100 MHz s_memrealtime clock
constexpr size_t kLdsLimit = 160 * 1024 - 2048;  // static LDS < 1 KiB

// Waits until the n tagged words (one per workgroup, saying that its slice of
// out is zero) carry `tag` (false: timed out after `budget` s_memrealtime
// ticks; a zero budget gives up at once, without polling).
__device__ __forceinline__ bool poll_zero_flags(const uint32_t *ztag, int n, uint32_t tag, uint64_t budget) {
  if (budget == 0) return false;
  const int lane = threadIdx.x & 63;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    bool mine = true;
    for (int i = lane; i < n; i += 64)
      mine = mine && __hip_atomic_load(ztag + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
    if (__all(mine)) return true;
    if (__builtin_amdgcn_s_memrealtime() - t0 > budget) return false;
  }
}

// Polls the E tagged router words of this call (one per expert, sb_word)
// until every one carries `tag` (or the wait times out after `budget` ticks,
// or at once for a zero budget: false).  Lane l receives expert l + 64 j in
// S[j], B[j] (S = -inf, B = 0 past E).
template <int NJ>
__device__ __forceinline__ bool poll_router_words(const uint64_t *rtag, int E, uint32_t tag, double (&S)[NJ],
                                                  double (&B)[NJ], uint64_t budget) {
  if (budget == 0) return false;
  const int lane = threadIdx.x & 63;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    bool mine = true;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int e = lane + 64 * j;
      S[j] = -INFINITY;
      B[j] = 0.0;
      if (e < E) {
        const uint64_t w = __hip_atomic_load(rtag + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mine = mine && (w & 0xffu) == tag;
        sb_unword(w, S[j], B[j]);
      }
    }
    if (__all(mine)) return true;
    if (__builtin_amdgcn_s_memrealtime() - t0 > budget) return false;
  }
}
__host__ inline size_t fused_burst_bytes() { return (size_t)(kData / 64) * kBurstKB * 1024; }
__host__ inline bool fused_burst_fits(int H, int E) { return fused_head_bytes(H, E) + fused_burst_bytes() <= kLdsLimit; }
__host__ inline size_t fused_lds_bytes(int H, int E) {
  return fused_head_bytes(H, E) + (fused_burst_fits(H, E) ? fused_burst_bytes() : 0);
}

// acc[0..EPC) += a * w for one 16-byte chunk of stored weights (INT formats:
// the raw codes; the group scale is applied when the sum is flushed).
template <int FMT>
__device__ __forceinline__ void chunk_axpy(const uint4 v, float a, float (&acc)[Chunk<FMT>::kElems]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if constexpr (FMT == kF32) {
#pragma unroll
    for (int q = 0; q < 4; q++) acc[q] = fmaf(a, __uint_as_float(u[q]), acc[q]);
  } else if constexpr (FMT == kBF16) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      acc[2 * q] = fmaf(a, __uint_as_float(u[q] << 16), acc[2 * q]);
      acc[2 * q + 1] = fmaf(a, __uint_as_float(u[q] & 0xffff0000u), acc[2 * q + 1]);
    }
  } else if constexpr (FMT == kINT8) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b++) acc[4 * q + b] = fmaf(a, (float)(int8_t)((u[q] >> (8 * b)) & 0xffu), acc[4 * q + b]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t byte = (u[q] >> (8 * b)) & 0xffu;  // (2c: high nibble, 2c+1: low)
        acc[8 * q + 2 * b] = fmaf(a, (float)((int)(byte >> 4) - 8), acc[8 * q + 2 * b]);
        acc[8 * q + 2 * b + 1] = fmaf(a, (float)((int)(byte & 0xfu) - 8), acc[8 * q + 2 * b + 1]);
      }
  }
}

// Rows whose loads are in flight per lane group: two while they fit the
// register budget of a 512-thread block.
template <int ITER>
constexpr int prefetch_rows() {
  return ITER > 0 && ITER <= 4 ? 2 : 1;
}
// Burst mode: a lane group (one wave) owning at most this many rows issues all
// of them at once -- gate and up rows into registers, down rows into the wave's
// LDS region -- so the whole block's data is in flight together.
template <int FMT, int ITER>
constexpr int burst_rows() {
  return ITER <= 0 ? 0 : ITER * Chunk<FMT>::kElems > 32 ? 2 : (kBurstKB / ITER < 4 ? kBurstKB / ITER : 4);
}
// Up to 32 outputs per lane the row sums stay in registers between flushes;
// wider rows add each row's products straight into the LDS run sums.
template <int FMT, int ITER>
constexpr bool accumulate_in_registers() {
  return ITER > 0 && ITER * Chunk<FMT>::kElems <= 32;
}

// Phase timeline of the decode kernel, built only into the instrumented
// library (make libqmoe_timeline.so, -DQMOE_TIMELINE): one s_memrealtime
// stamp (100 MHz) per (workgroup, point) from the first lane of the named
// wave, read back with qmoe_timeline_read.  The product library compiles the
// stamps away.
#ifdef QMOE_TIMELINE
constexpr int kStampsPerBlock = 16;
__device__ uint64_t g_timeline[kMaxExchangeBlocks * kStampsPerBlock];
#define QMOE_STAMP(i, wave)                                                                \
  do {                                                                                     \
    if (threadIdx.x == (wave) * 64)                                                        \
      g_timeline[blockIdx.x * kStampsPerBlock + (i)] = __builtin_amdgcn_s_memrealtime();  \
  } while (0)
#define QMOE_STAMP_DRAINED(i, wave)                                                        \
  do {                                                                                     \
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                     \
    QMOE_STAMP(i, wave);                                                                   \
  } while (0)
#else
#define QMOE_STAMP(i, wave) do { } while (0)
#define QMOE_STAMP_DRAINED(i, wave) do { } while (0)
#endif

template <int FMT, int ITER, int NJ>
__global__ void __launch_bounds__(kFusedBlock) expert_fused_kernel(FusedArgs a) {
  constexpr int EPC = Chunk<FMT>::kElems;
  constexpr int IT = ITER > 0 ? ITER : 1;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ids[64];
  __shared__ float s_w[64];
  __shared__ int s_spec[64];  // tentative expert + 1 per rank, 0 = not yet
  __shared__ int s_list[64];  // candidates of a certification rescue
  __shared__ float s_sg;
  __shared__ int s_exact;
  __shared__ int s_xready;  // data waves whose share of x is in LDS
  const int H = a.H;
  float *xs = reinterpret_cast<float *>(smem);
  float *red = xs + H;        // (2, H): the block's two runs
  float *lt = red + 2 * H;    // exact logits (fallback)
  unsigned char *burst_lds = smem + fused_head_bytes(H, a.E);
  QMOE_STAMP(0, 0);
  QMOE_STAMP(1, 1);

  // ---- the post-attention norm in the prologue (T = 1, a.norm_w given):
  // every workgroup normalises x into xs itself (gemmaRMSNormApply,
  // model/tensors.go:147-157, certified as in norm.hip), so the router
  // partials and the rows read the normed x without a launch of its own.
  const bool fnorm = a.norm_w != nullptr;
  if (fnorm) {
    __shared__ double s_part[kFusedBlock / 64];
    __shared__ float s_inv;
    double sq = 0.0;
    for (int i = threadIdx.x * 4; i < H; i += kFusedBlock * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(a.x + i);
      *reinterpret_cast<float4 *>(xs + i) = v;
      sq += (double)v.x * (double)v.x;
      sq += (double)v.y * (double)v.y;
      sq += (double)v.z * (double)v.z;
      sq += (double)v.w * (double)v.w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_down(sq, off, 64);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
      double sp = 0.0;
      for (int i = 0; i < kFusedBlock / 64; i++) sp += s_part[i];
      float inv;
      if (!norm_certify(sp, H, a.norm_eps, &inv) || a.norm_force_seq) {
        double q = 0.0;
        for (int i = 0; i < H; i++) q += (double)xs[i] * (double)xs[i];
        inv = norm_inv(q, H, a.norm_eps);
        if (blockIdx.x == 0 && a.norm_redo) atomicAdd(a.norm_redo, 1u);
      }
      s_inv = inv;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = threadIdx.x * 4; i < H; i += kFusedBlock * 4) {
#pragma clang fp contract(off)
      float4 v = *reinterpret_cast<const float4 *>(xs + i);
      const float4 g = *reinterpret_cast<const float4 *>(a.norm_w + i);
      v.x = (v.x * inv) * (1.0f + g.x);
      v.y = (v.y * inv) * (1.0f + g.y);
      v.z = (v.z * inv) * (1.0f + g.z);
      v.w = (v.w * inv) * (1.0f + g.w);
      *reinterpret_cast<float4 *>(xs + i) = v;
    }
    __syncthreads();
  }
  const float *xsrc = fnorm ? xs : a.x;  // x of token 0 for the router partials

  // ---- router partials computed in-kernel (T = 1): waves 1..7 of the
  // workgroups take one expert each (expert e: workgroup e % G, wave
  // 1 + e / G) and publish {S, B} as one tagged word (sb_word), which carries
  // its own validity.  Wave 7 of every workgroup initialises its slice of out
  // (to the residual stream when given, else 0) and then
  // (release) tags a per-workgroup word; every workgroup waits for all of
  // those (acquire) before its atomics into out -- off the critical path,
  // since that is long after the start.
  if (a.fused_router && threadIdx.x >= kCtl) {
    const int G = gridDim.x;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x + (wv - 1) * G;
    if (e < a.E) {
      const uint8_t *row = a.rw + (size_t)e * fmt_matrix_bytes(kBF16, 1, H);
      double S, B;
      if (a.fused_router == 1) router_sb_wave<kBF16, 1>(xsrc, H, row, nullptr, S, B);
      else if (a.fused_router == 2) router_sb_wave<kBF16, 2>(xsrc, H, row, nullptr, S, B);
      else router_sb_wave<kBF16, 4>(xsrc, H, row, nullptr, S, B);
      if (lane == 0)
        __hip_atomic_store(a.rtag + e, sb_word(S, B, a.epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (wv == 1) QMOE_STAMP_DRAINED(2, 1);
    }
    if (wv == kFusedBlock / 64 - 1) {
      // The zeros are agent-scope stores, which write through the L2; once
      // this wave's stores have completed (vmcnt(0)) they are visible device
      // wide, so the flag needs no L2 writeback (a release fence here would
      // write back the whole L2 and stall the router rows' loads).
      const int Z = (H + G - 1) / G;
      for (int j = blockIdx.x * Z + lane; j < min(H, (int)blockIdx.x * Z + Z); j += 64)
        __hip_atomic_store(a.out + j, a.resid ? a.resid[j] : 0.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane == 0) __hip_atomic_store(a.ztag + blockIdx.x, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- block -> (token, rows [u0, u1) of the token's flattened rows)
  const int t = blockIdx.x / a.nb;
  if (t >= a.T) return;
  const int U = a.k_routed * a.I + (a.with_shared ? a.Is : 0);
  const int u0 = (blockIdx.x % a.nb) * a.rb;
  const int u1 = min(U, u0 + a.rb);
  if (u0 >= u1) return;
  const int nrows = u1 - u0;
  const int KR = a.k_routed * a.I;
  // runs: at most two, since rb <= the smaller expert's rows.  Rank k = shared.
  int rank0, i00, n0, rank1 = 0, i01 = 0, n1 = 0;
  {
    int end0;
    if (u0 < KR) {
      rank0 = u0 / a.I;
      i00 = u0 % a.I;
      end0 = min(u1, (rank0 + 1) * a.I);
    } else {
      rank0 = a.k;
      i00 = u0 - KR;
      end0 = u1;
    }
    n0 = end0 - u0;
    if (end0 < u1) {
      rank1 = end0 < KR ? end0 / a.I : a.k;
      i01 = end0 < KR ? end0 % a.I : end0 - KR;
      n1 = u1 - end0;
    }
  }
  const int nruns = n1 > 0 ? 2 : 1;
  auto run_rank = [&](int q) { return q ? rank1 : rank0; };
  const bool ctl = threadIdx.x < kCtl;
  const int dt = threadIdx.x;  // row-streaming thread index (all threads)
  const bool writer = blockIdx.x % a.nb == 0 && (a.sb || a.fused_router) && a.k_routed > 0;

  // ---- geometry of a row: nch 16-byte chunks, lpr lanes per row
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);  // gate/up rows and transposed down rows
  const int gnsc = H / kGroup;
  const int nch = H / EPC;
  // The run sums are stored element-major: output j = ch * EPC + e sits at
  // e * nch + ch, so a lane-parallel update of element e of each lane's chunk
  // touches consecutive words (no LDS bank conflicts).
  auto pos = [&](int ch, int e) { return e * nch + ch; };
  const int lpr = lanes_per_row(nch);
  // burst mode (block-uniform): the lane groups are waves 1..7 -- the control
  // wave, busy with the selection until late, takes no rows -- each with at
  // most burst_rows rows, and the LDS holds the burst regions
  constexpr int kBurstGroups = kData / 64 - 1;
  const bool use_burst = a.burst && lpr == 64 &&
                         (nrows + kBurstGroups - 1) / kBurstGroups <= burst_rows<FMT, ITER>() &&
                         2 * H * 4 <= kBurstKB * 1024;
  const int groups = use_burst ? kBurstGroups : kData / lpr;
  const int g = use_burst ? dt / 64 - 1 : dt / lpr, sl = dt % lpr;  // g = -1: no rows
  // Burst run sums sit in output order; for EPC >= 16 (the group-32 formats)
  // with the 16-byte granules of each 256-byte row XOR-swizzled by the row
  // index: a lane's EPC consecutive outputs (float4 stores, lanes EPC floats
  // apart: a 4- or 8-way bank conflict per 16 lanes in plain order) then spread
  // over the banks, and 64 consecutive outputs (the final sums) still fill them
  // once.  (Measured: int4 30.1 -> 28.2 us, int8 25.7 -> 25.4 us; bf16, 2-way
  // in plain order, no better.)
  const bool pswz = EPC >= 16 && H % 64 == 0;
  auto part_idx = [&](int j) { return pswz ? j ^ (((j >> 6) & 15) << 2) : j; };
  // Burst mode with that swizzle: the data waves also store x, swizzled the
  // same way, into red (the burst keeps its sums elsewhere; a recompute clears
  // red first), where each lane's EPC consecutive x values read without bank
  // conflicts.
  const bool xcopy = use_burst && pswz && !fnorm;

  if (threadIdx.x < 64) s_spec[threadIdx.x] = 0;
  if (threadIdx.x == 0) s_xready = fnorm ? (kFusedBlock - kCtl) / 64 : 0;  // the prologue filled xs
  for (int j = threadIdx.x; j < 2 * H; j += kFusedBlock) red[j] = 0.0f;
  __syncthreads();
  // Waves 1..7 load x[t] into LDS and count themselves done in s_xready; the
  // control wave starts the selection at once, without x.
  if (!ctl && !fnorm) {
    for (int i = (threadIdx.x - kCtl) * 4; i < H; i += (kFusedBlock - kCtl) * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
      *reinterpret_cast<float4 *>(xs + i) = v;
      if (xcopy) *reinterpret_cast<float4 *>(red + part_idx(i)) = v;
    }
    if ((threadIdx.x & 63) == 0)
      __hip_atomic_fetch_add(&s_xready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  auto wait_x = [&]() {
    while (__hip_atomic_load(&s_xready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (kFusedBlock - kCtl) / 64)
      __builtin_amdgcn_s_sleep(1);
  };

  const int rs = g < 0 ? 0 : (int)((int64_t)g * nrows / groups);
  const int re = g < 0 ? 0 : (int)((int64_t)(g + 1) * nrows / groups);

  // expert of run q: tentative (published in s_spec, for the data waves) or
  // final (s_ids); both live in LDS in either routing mode
  auto run_expert = [&](int q, bool tentative) -> int {
    const int rk = run_rank(q);
    if (rk == a.k) return 0;
    return tentative ? s_spec[rk] - 1 : s_ids[rk];
  };

  // Rows [rs, re) of this lane group for the runs in `mask`, experts e0/e1.
  auto process_rows = [&](int e0_in, int e1_in, int mask, bool burst) {
    const int e0 = __builtin_amdgcn_readfirstlane(e0_in), e1 = __builtin_amdgcn_readfirstlane(e1_in);
    struct RowPtr {
      const uint8_t *g, *u, *d;
      const uint16_t *gs, *us, *ds;  // INT: gate/up scale rows; down scale row of the 32-row group
      int q, grp;
    };
    auto row_ptr = [&](int rho) -> RowPtr {
      RowPtr p;
      p.q = rho < n0 ? 0 : 1;
      const int i = p.q ? i01 + rho - n0 : i00 + rho;
      const bool sh = run_rank(p.q) == a.k;
      const int e = p.q ? e1 : e0;
      const uint8_t *gb = sh ? a.sgate : a.gu + (size_t)e * a.gu_bytes;
      const uint8_t *ub = sh ? a.sup : gb + (size_t)a.I * row_bytes;
      p.g = gb + (size_t)i * row_bytes;
      p.u = ub + (size_t)i * row_bytes;
      p.d = (sh ? a.sdown : a.dn + (size_t)e * a.dn_bytes) + (size_t)i * row_bytes;
      p.grp = i / kGroup;
      p.gs = p.us = p.ds = nullptr;
      if constexpr (fmt_quant(FMT)) {
        const uint16_t *gsb = sh ? a.sgate_s : a.gu_s + (size_t)e * a.gu_scales;
        const uint16_t *usb = sh ? a.sup_s : gsb + (size_t)a.I * gnsc;
        p.gs = gsb + (size_t)i * gnsc;
        p.us = usb + (size_t)i * gnsc;
        p.ds = (sh ? a.sdown_s : a.dn_s + (size_t)e * a.dn_scales) + (size_t)p.grp * H;
      }
      return p;
    };
    // per-lane running sum of act * down for the current (run, scale group)
    constexpr bool kAcc = accumulate_in_registers<FMT, ITER>();
    constexpr int AIT = kAcc ? IT : 1;
    float acc[AIT][EPC];
#pragma unroll
    for (int c = 0; c < AIT; c++)
#pragma unroll
      for (int e = 0; e < EPC; e++) acc[c][e] = 0.0f;
    int cur_q = -1, cur_grp = -1;
    const uint16_t *cur_ds = nullptr;
    auto flush = [&]() {
      if (!kAcc || cur_q < 0) return;
      float *rq = red + cur_q * H;
#pragma unroll
      for (int c = 0; c < AIT; c++) {
        const int ch = sl + c * lpr;
#pragma unroll
        for (int e = 0; e < EPC; e++) {
          float v = acc[c][e];
          if constexpr (fmt_quant(FMT)) v *= f16_to_f32(cur_ds[ch * EPC + e]);
          atomicAdd(rq + pos(ch, e), v);
          acc[c][e] = 0.0f;
        }
      }
    };
    auto act_of = [&](float gv, float uv) {
      gv = group_sum(gv, lpr);
      uv = group_sum(uv, lpr);
      return silu_ref(gv) * uv;
    };
    auto begin_row = [&](const RowPtr &p) {
      const bool same = p.q == cur_q && (!fmt_quant(FMT) || p.grp == cur_grp);
      if (!same) {
        flush();
        cur_q = p.q;
        cur_grp = p.grp;
        cur_ds = p.ds;
      }
    };
    constexpr int BR = burst_rows<FMT, ITER>();
    if constexpr (BR > 0) {
      if (burst && mask == 3) {
        // Burst: every row of this wave in flight at once -- down rows into the
        // wave's LDS region, gate and up rows (and, for the group-32 formats,
        // the row's down scales) into registers.  The per-run sums stay in
        // registers and are stored, without atomics, into the same LDS region
        // once the down rows have been consumed.  One lane group = one wave, so
        // rows and experts are wave-uniform and the row bases scalar.
        unsigned char *wl = burst_lds + (size_t)(dt >> 6) * kBurstKB * 1024;
        // Nothing of this wave is in flight here.  Saying so with a real
        // s_waitcnt vmcnt(0) (the builtin, which the compiler's wait
        // insertion sees, unlike asm) clears the loads it believes pending
        // from other paths into registers this code reuses; otherwise it
        // waits for a count before each row's loads, which here means
        // waiting for the first rows' data before issuing the fourth.
        __builtin_amdgcn_s_waitcnt(0x0f70);
        constexpr int SV = fmt_quant(FMT) ? IT * EPC / 8 : 1;  // 16-byte pieces of a lane's fp16 down scales
        uint4 bg[BR][IT], bu[BR][IT], bs[BR][SV];
        uint32_t bgs[BR][IT], bus[BR][IT];  // group-32 formats: the gate/up scales of the lane's chunks
        RowPtr bp[BR];
        const int n = __builtin_amdgcn_readfirstlane(re - rs);
        const int rs_u = __builtin_amdgcn_readfirstlane(rs);
#pragma unroll
        for (int r = 0; r < BR; r++)  // every pointer first, then every load
          if (r < n) bp[r] = row_ptr(rs_u + r);
        // row r starts a new set of down scales (run or scale group changes)
        auto newset = [&](int r) { return r == 0 || bp[r].q != bp[r - 1].q || bp[r].grp != bp[r - 1].grp; };
#pragma unroll
        for (int r = 0; r < BR; r++) {
          if (r < n) {
#pragma unroll
            for (int c = 0; c < IT; c++)
              dma16_nt(bp[r].d + (size_t)(sl + c * lpr) * 16, wl + (r * IT + c) * 1024);
          }
        }
#pragma unroll
        for (int r = 0; r < BR; r++) {
          if (r < n) {
#pragma unroll
            for (int c = 0; c < IT; c++) {
              const size_t off = (size_t)(sl + c * lpr) * 16;
              bg[r][c] = load_nt(bp[r].g + off);
              bu[r][c] = load_nt(bp[r].u + off);
            }
            if constexpr (fmt_quant(FMT)) {
              // loaded with the rows: past wait_x (an atomic spin) the
              // compiler would issue them only where they are used; the
              // empty asm after wait_x keeps their conversion (and its
              // wait) from being hoisted between the rows' loads
#pragma unroll
              for (int c = 0; c < IT; c++) {
                const int ch = sl + c * lpr;
                bgs[r][c] = bp[r].gs[(ch * EPC) / kGroup];
                bus[r][c] = bp[r].us[(ch * EPC) / kGroup];
              }
              // the down scales of the lane's outputs (chunk c covers EPC
              // consecutive outputs), once per run of rows sharing a run and
              // a 32-row scale group
              if (newset(r)) {
#pragma unroll
                for (int v = 0; v < SV; v++) {
                  const int c = v / (EPC / 8), part = v % (EPC / 8);
                  bs[r][v] = *reinterpret_cast<const uint4 *>(bp[r].ds + (sl + c * lpr) * EPC + part * 8);
                }
              }
            }
          }
        }
        wait_x();
        if constexpr (fmt_quant(FMT)) {
#pragma unroll
          for (int r = 0; r < BR; r++)
#pragma unroll
            for (int c = 0; c < IT; c++) asm volatile("" : "+v"(bgs[r][c]), "+v"(bus[r][c]));
        }
        // this lane's x chunks, read once for all its rows
        const float *xb = xcopy ? red : xs;
        float xl[IT][EPC];
#pragma unroll
        for (int c = 0; c < IT; c++) {
          const int j0 = (sl + c * lpr) * EPC;
#pragma unroll
          for (int q = 0; q < EPC / 4; q++) {
            const int xi = xcopy ? part_idx(j0 + 4 * q) : j0 + 4 * q;
            const float4 v = *reinterpret_cast<const float4 *>(xb + xi);
            xl[c][4 * q] = v.x;
            xl[c][4 * q + 1] = v.y;
            xl[c][4 * q + 2] = v.z;
            xl[c][4 * q + 3] = v.w;
          }
        }
        float act[BR];
#pragma unroll
        for (int r = 0; r < BR; r++) {
          act[r] = 0.0f;
          if (r < n) {
            float gv = 0.0f, uv = 0.0f;
#pragma unroll
            for (int c = 0; c < IT; c++) {
              float dg = chunk_dot<FMT>(bg[r][c], xl[c]);
              float du = chunk_dot<FMT>(bu[r][c], xl[c]);
              if constexpr (fmt_quant(FMT)) {
                dg *= f16_to_f32((uint16_t)bgs[r][c]);
                du *= f16_to_f32((uint16_t)bus[r][c]);
              }
              gv += dg;
              uv += du;
            }
            act[r] = act_of(gv, uv);
          }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the down rows have landed in LDS
        QMOE_STAMP(6, 1);
        QMOE_STAMP(13, 7);
        float acc0[IT][EPC], acc1[IT][EPC];
#pragma unroll
        for (int c = 0; c < IT; c++)
#pragma unroll
          for (int e = 0; e < EPC; e++) acc0[c][e] = acc1[c][e] = 0.0f;
        if constexpr (fmt_quant(FMT) && IT * EPC > 32) {
          // wide rows (no registers for a set's sum): scale each row's products
          uint4 sv[SV];
#pragma unroll
          for (int v = 0; v < SV; v++) sv[v] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
          for (int r = 0; r < BR; r++) {
            if (r < n) {
              if (newset(r)) {
#pragma unroll
                for (int v = 0; v < SV; v++) sv[v] = bs[r][v];
              }
#pragma unroll
              for (int c = 0; c < IT; c++) {
                float w[EPC];
#pragma unroll
                for (int e = 0; e < EPC; e++) w[e] = 0.0f;
                chunk_axpy<FMT>(*reinterpret_cast<const uint4 *>(wl + (r * IT + c) * 1024 + sl * 16), act[r], w);
#pragma unroll
                for (int e = 0; e < EPC; e++) {
                  const int k = c * EPC + e;  // the lane's k-th output
                  const uint32_t word = (&sv[k / 8].x)[(k % 8) / 2];
                  const float sc = f16_to_f32((uint16_t)((k & 1) ? (word >> 16) : (word & 0xffffu)));
                  if (bp[r].q == 0) acc0[c][e] = fmaf(w[e], sc, acc0[c][e]);
                  else acc1[c][e] = fmaf(w[e], sc, acc1[c][e]);
                }
              }
            }
          }
        } else if constexpr (fmt_quant(FMT)) {
          // sum act * code over the rows of one scale set, then scale once
          float tmp[IT][EPC];
          uint4 sv[SV];
          int tq = 0;
#pragma unroll
          for (int c = 0; c < IT; c++)
#pragma unroll
            for (int e = 0; e < EPC; e++) tmp[c][e] = 0.0f;
#pragma unroll
          for (int v = 0; v < SV; v++) sv[v] = make_uint4(0u, 0u, 0u, 0u);
          auto flush_set = [&]() {
#pragma unroll
            for (int c = 0; c < IT; c++)
#pragma unroll
              for (int e = 0; e < EPC; e++) {
                const int k = c * EPC + e;  // the lane's k-th output
                const uint32_t word = (&sv[k / 8].x)[(k % 8) / 2];
                const float sc = f16_to_f32((uint16_t)((k & 1) ? (word >> 16) : (word & 0xffffu)));
                if (tq == 0) acc0[c][e] = fmaf(tmp[c][e], sc, acc0[c][e]);
                else acc1[c][e] = fmaf(tmp[c][e], sc, acc1[c][e]);
                tmp[c][e] = 0.0f;
              }
          };
#pragma unroll
          for (int r = 0; r < BR; r++) {
            if (r < n) {
              if (newset(r)) {
                if (r > 0) flush_set();
#pragma unroll
                for (int v = 0; v < SV; v++) sv[v] = bs[r][v];
                tq = bp[r].q;
              }
#pragma unroll
              for (int c = 0; c < IT; c++)
                chunk_axpy<FMT>(*reinterpret_cast<const uint4 *>(wl + (r * IT + c) * 1024 + sl * 16), act[r], tmp[c]);
            }
          }
          flush_set();
        } else {
#pragma unroll
          for (int r = 0; r < BR; r++) {
            if (r < n) {
#pragma unroll
              for (int c = 0; c < IT; c++) {
                const uint4 v = *reinterpret_cast<const uint4 *>(wl + (r * IT + c) * 1024 + sl * 16);
                if (bp[r].q == 0) chunk_axpy<FMT>(v, act[r], acc0[c]);
                else chunk_axpy<FMT>(v, act[r], acc1[c]);
              }
            }
          }
        }
        // the wave's run sums, in (swizzled) output order, into its own region
        float *part = reinterpret_cast<float *>(wl);
#pragma unroll
        for (int c = 0; c < IT; c++) {
          const int j0 = (sl + c * lpr) * EPC;
#pragma unroll
          for (int e = 0; e < EPC; e += 4) {
            *reinterpret_cast<float4 *>(part + part_idx(j0 + e)) =
                make_float4(acc0[c][e], acc0[c][e + 1], acc0[c][e + 2], acc0[c][e + 3]);
            *reinterpret_cast<float4 *>(part + H + part_idx(j0 + e)) =
                make_float4(acc1[c][e], acc1[c][e + 1], acc1[c][e + 2], acc1[c][e + 3]);
          }
        }
        return;
      }
    }
    if constexpr (ITER > 0) {
      constexpr int PD = prefetch_rows<ITER>();
      struct RowData {
        uint4 g[IT], u[IT], d[IT];
      };
      RowData buf[PD];
      RowPtr ptr[PD];
      auto load = [&](int slot, int rho) {
        ptr[slot] = row_ptr(rho);
#pragma unroll
        for (int c = 0; c < IT; c++) {
          const size_t off = (size_t)(sl + c * lpr) * 16;
          buf[slot].g[c] = *reinterpret_cast<const uint4 *>(ptr[slot].g + off);
          buf[slot].u[c] = *reinterpret_cast<const uint4 *>(ptr[slot].u + off);
          buf[slot].d[c] = *reinterpret_cast<const uint4 *>(ptr[slot].d + off);
        }
      };
      auto consume = [&](int slot) {
        const RowPtr &p = ptr[slot];
        float gv = 0.0f, uv = 0.0f;
#pragma unroll
        for (int c = 0; c < IT; c++) {
          const int ch = sl + c * lpr;
          float dg = chunk_dot<FMT>(buf[slot].g[c], xs + ch * EPC);
          float du = chunk_dot<FMT>(buf[slot].u[c], xs + ch * EPC);
          if constexpr (fmt_quant(FMT)) {
            dg *= f16_to_f32(p.gs[(ch * EPC) / kGroup]);
            du *= f16_to_f32(p.us[(ch * EPC) / kGroup]);
          }
          gv += dg;
          uv += du;
        }
        const float act = act_of(gv, uv);
        if constexpr (kAcc) {
          begin_row(p);
#pragma unroll
          for (int c = 0; c < IT; c++) chunk_axpy<FMT>(buf[slot].d[c], act, acc[AIT > 1 ? c : 0]);
        } else {
          float *rq = red + p.q * H;
#pragma unroll
          for (int c = 0; c < IT; c++) {
            const int ch = sl + c * lpr;
            float w[EPC];
#pragma unroll
            for (int e = 0; e < EPC; e++) w[e] = 0.0f;
            chunk_axpy<FMT>(buf[slot].d[c], act, w);
#pragma unroll
            for (int e = 0; e < EPC; e++) {
              float v = w[e];
              if constexpr (fmt_quant(FMT)) v *= f16_to_f32(p.ds[ch * EPC + e]);
              atomicAdd(rq + pos(ch, e), v);
            }
          }
        }
      };
      // rows of runs outside `mask` are skipped (they are only loaded)
      auto wanted = [&](int rho) { return (mask >> (rho < n0 ? 0 : 1)) & 1; };
#pragma unroll
      for (int s = 0; s < PD; s++)
        if (rs + s < re) load(s, rs + s);
      wait_x();
      for (int rho = rs; rho < re; rho += PD) {
#pragma unroll
        for (int s = 0; s < PD; s++) {
          if (rho + s < re) {
            if (wanted(rho + s)) consume(s);
            if (rho + s + PD < re) load(s, rho + s + PD);
          }
        }
      }
    } else {
      wait_x();
      for (int rho = rs; rho < re; rho++) {
        if (!((mask >> (rho < n0 ? 0 : 1)) & 1)) continue;
        const RowPtr p = row_ptr(rho);
        const float act = act_of(row_dot_rt<FMT>(p.g, p.gs, xs, sl, lpr, nch),
                                 row_dot_rt<FMT>(p.u, p.us, xs, sl, lpr, nch));
        float *rq = red + p.q * H;
        for (int c = sl; c < nch; c += lpr) {
          float w[EPC];
#pragma unroll
          for (int e = 0; e < EPC; e++) w[e] = 0.0f;
          chunk_axpy<FMT>(*reinterpret_cast<const uint4 *>(p.d + (size_t)c * 16), act, w);
#pragma unroll
          for (int e = 0; e < EPC; e++) {
            float v = w[e];
            if constexpr (fmt_quant(FMT)) v *= f16_to_f32(p.ds[c * EPC + e]);
            atomicAdd(rq + pos(c, e), v);
          }
        }
      }
    }
    flush();
  };

  bool need_exact = false;
  int te0 = 0, te1 = 0;  // tentative experts of the two runs
  if (ctl) {
    // ---- control wave: routing; the shared gate for a shared run
    const bool has_routed = rank0 != a.k;
    double S[NJ], B[NJ], kth_lo = 0.0;
    bool rescue = false;  // certification failed: try exact logits of the candidates in doubt
    int32_t *gi = nullptr;
    float *gw = nullptr;
    if (a.fused_router) {
      if (has_routed) {
        gi = writer ? a.ids : nullptr;
        gw = writer ? a.weights : nullptr;
        if (poll_router_words<NJ>(a.rtag, a.E, a.epoch, S, B, a.xchg_ticks)) {
          QMOE_STAMP(3, 0);
          rescue = !certified_select_regs<NJ>(S, B, a.E, a.k, a.scope, gi, gw, s_ids, s_w, -2, s_spec, &kth_lo);
          QMOE_STAMP(4, 0);
        } else {
          // timed out: flag it for the host (the call's result is not
          // trustworthy), stream expert 0 tentatively and route this
          // workgroup with the exact logits so that every wave still finishes
          if (threadIdx.x == 0) __hip_atomic_store(a.xchg_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          if (threadIdx.x < a.k)
            __hip_atomic_store(&s_spec[threadIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          need_exact = true;
        }
      }
    } else if (has_routed && a.sb) {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int e = threadIdx.x + 64 * j;
        const double2 v =
            e < a.E ? reinterpret_cast<const double2 *>(a.sb + (size_t)t * a.E * 2)[e] : make_double2(-INFINITY, 0.0);
        S[j] = v.x;
        B[j] = v.y;
      }
      gi = writer ? a.ids + (size_t)t * a.k : nullptr;
      gw = writer ? a.weights + (size_t)t * a.k : nullptr;
      rescue = !certified_select_regs<NJ>(S, B, a.E, a.k, a.scope, gi, gw, s_ids, s_w, -2, s_spec, &kth_lo);
    }
    if (rescue) {
      // a bf16 router (the in-kernel router is one): exact logits of the few
      // candidates in doubt, while the data waves stream the tentative
      // experts; other formats, or a failed rescue: the exact path
      bool ok = false;
      if (a.rfmt == kBF16) {
        wait_x();
        ok = refine_select<kBF16, NJ>(S, B, kth_lo, a.E, a.k, a.scope, xs, H, a.rw, nullptr, s_list, gi, gw, s_ids,
                                      s_w);
        if (ok && writer && threadIdx.x == 0) atomicAdd(a.fallbacks + 1, 1u);
      }
      need_exact = !ok;
    }
    if (!a.fused_router && !a.sb && has_routed && threadIdx.x < a.k) {  // precomputed routing
      const int id = a.ids[(size_t)t * a.k + threadIdx.x];
      s_ids[threadIdx.x] = id;
      s_w[threadIdx.x] = a.weights[(size_t)t * a.k + threadIdx.x];
      __hip_atomic_store(&s_spec[threadIdx.x], id + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if ((nruns > 1 ? rank1 : rank0) == a.k) {
      wait_x();
      float sgv = 0.0f;  // shared-expert gate, model/moe.go:89-93
      for (int i = threadIdx.x; i < H; i += 64) sgv = fmaf(xs[i], a.shared_gate[i], sgv);
      sgv = group_sum(sgv, 64);
      if (threadIdx.x == 0) s_sg = 1.0f / (1.0f + (float)exp(-(double)sgv));
    }
  }
  // ---- every wave: wait for the tentative experts of the block's runs (the
  // control wave has published them already) and stream its rows
  for (int q = 0; q < nruns; q++) {
    const int rk = run_rank(q);
    if (rk == a.k) continue;
    while (__hip_atomic_load(&s_spec[rk], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
      __builtin_amdgcn_s_sleep(1);
  }
  // T = 1: a rank's bursts start rank * rank_gap ticks after its expert is
  // known, spreading the ranks' reads beyond the selection rounds' own spacing
  if (a.rank_gap && rank0 != a.k) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime(), d = (uint64_t)rank0 * a.rank_gap;
    while (__builtin_amdgcn_s_memrealtime() - t0 < d) __builtin_amdgcn_s_sleep(1);
  }
  QMOE_STAMP(5, 1);
  QMOE_STAMP(12, 7);
  te0 = run_expert(0, true);
  te1 = nruns > 1 ? run_expert(1, true) : 0;
  process_rows(te0, te1, 3, use_burst);
  QMOE_STAMP(7, 1);
  QMOE_STAMP(14, 7);
  if (ctl && a.fused_router) {
    // out's zeros, every workgroup's slice, before this workgroup's atomics
    if (poll_zero_flags(a.ztag, gridDim.x, a.epoch, a.xchg_ticks)) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    else if (threadIdx.x == 0) __hip_atomic_store(a.xchg_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  QMOE_STAMP(8, 0);
  if (threadIdx.x == 0) s_exact = need_exact;
  __syncthreads();  // run sums, s_ids/s_w (when certified), s_sg, s_exact
  QMOE_STAMP(9, 0);
  if (s_exact) {
    // certification failed: the whole block computes the exact routing
    exact_logits_block(xs, H, a.rw, a.rs, a.rfmt, a.E, lt, kFusedBlock);
    __syncthreads();
    if (ctl) {
      select_exact_nj<NJ>(lt, a.E, a.k, a.scope, writer ? a.ids + (size_t)t * a.k : nullptr,
                          writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w);
      if (writer && threadIdx.x == 0) atomicAdd(a.fallbacks, 1u);
    }
    __syncthreads();
  }
  const int e0 = run_expert(0, false);
  const int e1 = nruns > 1 ? run_expert(1, false) : 0;
  // runs whose tentative expert was not the final one are recomputed
  int redo = 0;
  if (rank0 != a.k && e0 != s_spec[rank0] - 1) redo |= 1;
  if (nruns > 1 && rank1 != a.k && e1 != s_spec[rank1] - 1) redo |= 2;
  if (redo) {
    // recompute the runs in `redo` into red (streaming mode); their burst
    // partial sums are dropped
    for (int j = threadIdx.x; j < H; j += kFusedBlock) {
      if ((redo & 1) || use_burst) red[j] = 0.0f;  // burst mode: red holds nothing (x, with xcopy)
      if ((redo & 2) || use_burst) red[H + j] = 0.0f;
      if (use_burst)
        for (int w = 0; w < kFusedBlock / 64; w++) {
          float *part = reinterpret_cast<float *>(burst_lds + (size_t)w * kBurstKB * 1024);
          if (redo & 1) part[j] = 0.0f;
          if (redo & 2) part[H + j] = 0.0f;
        }
    }
    __syncthreads();
    process_rows(e0, e1, redo, false);
    __syncthreads();
  }
  // ---- out[t] += w_run * run sum (the routing weight, or the shared gate)
  const float w0 = rank0 == a.k ? s_sg : s_w[rank0];
  const float w1 = nruns > 1 ? (rank1 == a.k ? s_sg : s_w[rank1]) : 0.0f;
  float *out_t = a.out + (size_t)t * H;
  // output order: the global atomics of a wave then cover 256 contiguous bytes
  const int rot = H % 64 == 0 ? (int)(blockIdx.x % (H / 64)) * 64 : 0;
  // In burst mode red holds only recomputed runs: read it only then (its
  // element-major reads in output order put EPC consecutive outputs in one
  // LDS bank, an EPC-way conflict)
  const bool red_live = !use_burst || redo != 0;
  for (int j0 = threadIdx.x; j0 < H; j0 += kFusedBlock) {
    const int j = j0 + rot < H ? j0 + rot : j0 + rot - H;
    float s0 = 0.0f, s1 = 0.0f;
    if (red_live) {
      const int pj = pos(j / EPC, j % EPC);
      s0 = red[pj];
      s1 = red[H + pj];
    }
    if (use_burst)  // burst sums are stored in (swizzled) output order
      for (int w = 0; w < kFusedBlock / 64; w++) {
        const float *part = reinterpret_cast<const float *>(burst_lds + (size_t)w * kBurstKB * 1024);
        s0 += part[part_idx(j)];
        s1 += part[H + part_idx(j)];
      }
    float v = w0 * s0;
    if (nruns > 1) v = fmaf(w1, s1, v);
    atomicAdd(out_t + j, v);
  }
  QMOE_STAMP_DRAINED(10, 0);
}

// Splits each token's k*I (+ Is) intermediate rows evenly over about one
// wave of blocks per CU, at most kMaxRows rows and two experts per block:
// fills a.rb and a.nb, returns the grid size.
static int fused_grid(FusedArgs &a) {
  const int U = a.k_routed * a.I + (a.with_shared ? a.Is : 0);
  const int rmax = min(kMaxRows, min(a.k_routed ? a.I : a.Is, a.with_shared ? a.Is : a.I));
  int nb = max(1, (a.n_cu + a.T - 1) / a.T);
  nb = max(nb, (U + rmax - 1) / rmax);
  a.rb = (U + nb - 1) / nb;
  a.nb = (U + a.rb - 1) / a.rb;
  return a.T * a.nb;
}

template <int FMT, int ITER, int NJ>
static void fused_launch(const FusedArgs &a0, hipStream_t st) {
  FusedArgs a = a0;
  const int blocks = fused_grid(a);
  a.burst = fused_burst_fits(a.H, a.E);
  // Same-box A/B of the gap (0.1 us steps): at T = 1 with the in-kernel router
  // and ranks of several MB (Qwen3-30B-A3B: bf16 9.4 MB, int8 4.7 MB per rank)
  // 0.4 us ends the data phase sooner (bf16 29.8 -> 28.9 us, int8 26.8 -> 26.2);
  // with 1.5 MB ranks (int4, E = 512) or at T = 8 any gap is slower.
  a.rank_gap = a.fused_router && a.T == 1 && fmt_matrix_bytes(a.fmt, 3 * a.I, a.H) >= (int64_t)(4 << 20)
                   ? kRankGapTicks : 0;
  const size_t lds = fused_lds_bytes(a.H, a.E);
  if (a.occ_out) {
    *a.occ_out = 0;
    (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(a.occ_out, expert_fused_kernel<FMT, ITER, NJ>, kFusedBlock, lds);
    return;
  }
  // dynamic LDS above 64 KiB has to be allowed per kernel (once per size)
  static size_t allowed = 64 * 1024;
  if (lds > allowed) {
    if (hipFuncSetAttribute((const void *)expert_fused_kernel<FMT, ITER, NJ>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return;  // the error stays set; launch_expert_fused reports it
    allowed = lds;
  }
  QMOE_LAUNCH((expert_fused_kernel<FMT, ITER, NJ>), dim3(blocks), dim3(kFusedBlock), lds, st, a);
}

template <int FMT, int ITER>
static void fused_nj(const FusedArgs &a, hipStream_t st) {
#define L(NJ) fused_launch<FMT, ITER, NJ>(a, st)
  QMOE_NJ_DISPATCH(a.E, L);
#undef L
}

// Rows of more than 64 elements per lane take the run-time chunk loop (the
// unrolled loads would not fit the registers).
template <int FMT, int ITER>
constexpr int usable_iter() {
  return ITER * Chunk<FMT>::kElems > 64 ? 0 : ITER;
}

template <int FMT, int ITER>
static void fused_iter(const FusedArgs &a, hipStream_t st) {
  if constexpr (usable_iter<FMT, ITER>() == ITER) fused_nj<FMT, ITER>(a, st);
  else fused_nj<FMT, 0>(a, st);
}

template <int FMT>
static void fused_fmt(const FusedArgs &a, hipStream_t st) {
  switch (iter_of(FMT, a.H)) {
  case 1: fused_iter<FMT, 1>(a, st); break;
  case 2: fused_iter<FMT, 2>(a, st); break;
  case 4: fused_iter<FMT, 4>(a, st); break;
  case 8: fused_iter<FMT, 8>(a, st); break;
  default: fused_nj<FMT, 0>(a, st); break;
  }
}

int fused_exchange_blocks(const FusedArgs &a0, int *resident) {
  FusedArgs a = a0;
  const int blocks = fused_grid(a);
  int per_cu = 0;
  a.occ_out = &per_cu;
  switch (a.fmt) {
  case kF32: fused_fmt<kF32>(a, nullptr); break;
  case kBF16: fused_fmt<kBF16>(a, nullptr); break;
  case kINT8: fused_fmt<kINT8>(a, nullptr); break;
  default: fused_fmt<kINT4>(a, nullptr); break;
  }
  *resident = per_cu * a.n_cu;
  return blocks;
}

bool fused_supported(int fmt, int H, int E) {
  (void)fmt;
  return fused_lds_bytes(H, E) <= kLdsLimit;
}

__global__ void __launch_bounds__(256) zero_kernel(float *__restrict__ p, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) *reinterpret_cast<float4 *>(p + i) = make_float4(0.f, 0.f, 0.f, 0.f);
  else
    for (int64_t q = i; q < n; q++) p[q] = 0.0f;
}

hipError_t launch_zero(float *p, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  QMOE_LAUNCH(zero_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

hipError_t launch_expert_fused(const FusedArgs &a, hipStream_t st) {
  if (a.fused_router) {
    // the in-kernel router needs one expert per wave of waves 1..7 and one
    // zero flag per workgroup
    FusedArgs g = a;
    const int blocks = fused_grid(g);
    if (a.T != 1 || blocks > kMaxExchangeBlocks || a.E > 7 * blocks) return hipErrorInvalidConfiguration;
  }
  switch (a.fmt) {
  case kF32: fused_fmt<kF32>(a, st); break;
  case kBF16: fused_fmt<kBF16>(a, st); break;
  case kINT8: fused_fmt<kINT8>(a, st); break;
  default: fused_fmt<kINT4>(a, st); break;
  }
  return hipGetLastError();
}

}  // namespace qmoe

#ifdef QMOE_TIMELINE
// The instrumented library's read-out of the stamps: n words from the start.
extern "C" int qmoe_timeline_read(uint64_t *host, int n) {
  if (!host || n < 0 || n > qmoe::kMaxExchangeBlocks * qmoe::kStampsPerBlock) return 1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(qmoe::g_timeline), (size_t)n * 8, 0, hipMemcpyDeviceToHost) ==
                 hipSuccess
             ? 0
             : 4;
}
#endif
