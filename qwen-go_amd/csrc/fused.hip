// fused.hip -- the expert products for one forward in a single kernel.
//
// Block = (token t, rank r, chunk c of 32 intermediate rows); a launch covers
// the routed ranks, the shared expert (model/moe.go:86-97), or both.  One
// control wave and eight data waves:
//   control: picks the block's expert.  From the router partials it runs the
//            certified selection (select.hpp): as soon as the round of rank r
//            ends it publishes that tentative expert through LDS, then
//            finishes the remaining rounds and the certification while the
//            data waves stream.  With precomputed routing it just reads it.
//            For the shared expert it computes sigmoid(shared_gate . x).
//   data:    issue every load of the block at once -- gate and up rows
//            [32c, 32c+32) of the expert into registers, and rows [32c, 32c+32)
//            of its down matrix, stored transposed (I, H) so that they are one
//            contiguous region, straight into LDS (global_load_lds) -- then
//            compute act = silu(g) * u (model/moe.go:64-75) and
//            w_r * (down[:, 32c:32c+32] . act), added into out[t] with f32
//            atomics (model/moe.go:76-84).
// The certification result is checked before any atomic; if the final expert
// differs from the tentative one, the block recomputes with the final one.
// When certification fails the whole block computes the exact sequential
// logits of the token (the reference's bits) and selects on them.
// Splitting the intermediate dimension across blocks removes the dependency
// between the gate_up and the down products, so the layer needs no second
// launch and no in-kernel handoff between blocks.  out must be zero on entry.
// The atomics make the order of the final f32 sums run-dependent (within f32
// rounding of the reference's rank-ordered sum).
//
// Work to blocks, XCD-aware: workgroups go to the 8 XCDs round-robin by linear
// id; the chunks of one expert are given ids that spread evenly over them.
#include "gemv_common.hpp"
#include "select.hpp"

namespace qmoe {

constexpr int kCtl = 64;                      // control wave
constexpr int kData = 448;                    // data threads (7 waves)
constexpr int kFusedBlock = kCtl + kData;
constexpr int kMaxRows = 192;                 // intermediate rows per block, at most
constexpr int kDownLds = 128 * 1024;          // LDS bytes for down-slice staging
constexpr int kMaxRowsPerGroup = 4;

// Rows per lane group whose loads are in flight together: as many as fit the
// register budget of 512-thread blocks (the quantised dot products unpack
// more per chunk).
// Output chunks per data thread in the down product: two where a row of the
// hidden size can have more 16-byte chunks than there are data threads.
template <int FMT>
constexpr int kDownPasses = FMT == kINT4 ? 1 : 2;

template <int FMT, int ITER>
constexpr int rows_in_flight() {
  return (FMT == kINT4 && ITER >= 4) ? 1 : (fmt_quant(FMT) && ITER >= 4) ? 2 : kMaxRowsPerGroup;
}

// Rows of the transposed down slice staged per LDS pass.
template <int FMT>
__host__ __device__ inline int stage_rows(int H) {
  const int64_t row = fmt_matrix_bytes(FMT, 1, H);
  int r = (int)(kDownLds / row);
  return r >= 32 ? 32 : (r >= 16 ? 16 : (r >= 8 ? 8 : 0));
}
template <int FMT>
__host__ inline size_t fused_lds_bytes(int H, int E) {
  const size_t head = ((size_t)(H + kMaxRows + E) * 4 + 15) / 16 * 16;
  // stage_slice writes whole passes of kData x 16 bytes
  const size_t pass = (size_t)kData * 16;
  const size_t slice = ((size_t)stage_rows<FMT>(H) * fmt_matrix_bytes(FMT, 1, H) + pass - 1) / pass * pass;
  const int epc = Chunk<FMT>::kElems;
  const int jc = H / epc;
  const int ig = jc >= kData ? 1 : kData / jc;
  const size_t part = (size_t)ig * H * 4;
  return head + (slice > part ? slice : part);
}

// Issues the loads of `rows` contiguous stored down rows (each row_bytes) into
// dsl (LDS), 16 bytes per data lane per instruction.
__device__ __forceinline__ void stage_slice(const uint8_t *__restrict__ src, int64_t bytes, unsigned char *dsl,
                                            int dt) {
  const int64_t n16 = bytes / 16;
  for (int64_t p = 0; p * kData < n16; p++) {
    int64_t q = p * kData + dt;
    q = q < n16 ? q : n16 - 1;  // the tail reloads a valid piece that is never used
    auto *dst = (__attribute__((address_space(3))) void *)(dsl + ((size_t)p * kData + (dt & ~63)) * 16);
    __builtin_amdgcn_global_load_lds(src + q * 16, dst, 16, 0, 0);
  }
}

// acc[0..EPC) += a * w for one 16-byte chunk of stored weights.
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

// acc[q] += (a * sc[q]) * w[q]: one chunk of a quantised row whose group
// scales differ per output.
template <int FMT>
__device__ __forceinline__ void chunk_axpy_scaled(const uint4 v, float a, const float (&sc)[Chunk<FMT>::kElems],
                                                  float (&acc)[Chunk<FMT>::kElems]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if constexpr (FMT == kINT8) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b++)
        acc[4 * q + b] = fmaf(a * sc[4 * q + b], (float)(int8_t)((u[q] >> (8 * b)) & 0xffu), acc[4 * q + b]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t byte = (u[q] >> (8 * b)) & 0xffu;
        acc[8 * q + 2 * b] = fmaf(a * sc[8 * q + 2 * b], (float)((int)(byte >> 4) - 8), acc[8 * q + 2 * b]);
        acc[8 * q + 2 * b + 1] = fmaf(a * sc[8 * q + 2 * b + 1], (float)((int)(byte & 0xfu) - 8), acc[8 * q + 2 * b + 1]);
      }
  }
}

// One intermediate row of the block: which expert it belongs to and where.
struct RowRef {
  int seg;  // 0 or 1: the block's first or second run of rows
  int i;    // intermediate index within the expert
};

template <int FMT, int ITER, int NJ>
__global__ void __launch_bounds__(kFusedBlock) expert_fused_kernel(FusedArgs a) {
  constexpr int EPC = Chunk<FMT>::kElems;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ids[64];
  __shared__ float s_w[64];
  __shared__ int s_spec[64];  // tentative expert + 1 per rank, 0 = not yet
  __shared__ float s_sg;
  __shared__ int s_exact;
  __shared__ int s_xready;  // data waves whose share of x is in LDS
  const int H = a.H;
  float *xs = reinterpret_cast<float *>(smem);
  float *act = xs + H;                      // kMaxRows (act scaled by the routing weight)
  float *lt = act + kMaxRows;
  unsigned char *dsl = smem + ((size_t)(H + kMaxRows + a.E) * 4 + 15) / 16 * 16;

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
  const int dt = threadIdx.x - kCtl;
  const bool writer = blockIdx.x % a.nb == 0 && a.sb && a.k_routed > 0;

  if (threadIdx.x < 64) s_spec[threadIdx.x] = a.sb ? 0 : 1;
  if (threadIdx.x == 0) s_xready = 0;
  __syncthreads();
  // The data waves load x[t] into LDS and count themselves done in s_xready;
  // the control wave starts the selection at once, without x.
  if (!ctl) {
    for (int i = dt * 4; i < H; i += kData * 4)
      *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
    if ((dt & 63) == 0) __hip_atomic_fetch_add(&s_xready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  auto wait_x = [&]() {
    while (__hip_atomic_load(&s_xready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < kData / 64)
      __builtin_amdgcn_s_sleep(1);
  };

  // ---- geometry
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);  // gate/up rows and transposed down rows
  const int gnsc = H / kGroup;
  const int nch = H / EPC;
  const int lpr = lanes_per_row(nch);
  const int groups = kData / lpr;
  const int g = dt / lpr, sl = dt % lpr;
  const int SR = stage_rows<FMT>(H);

  // expert of run q (tentative for data waves until certification ends)
  auto run_expert = [&](int q, bool tentative) -> int {
    const int rk = run_rank(q);
    if (rk == a.k) return 0;
    if (!a.sb) return a.ids[(size_t)t * a.k + rk];
    return tentative ? s_spec[rk] - 1 : s_ids[rk];
  };
  auto gate_ptr = [&](int q, int e, int i, const uint8_t *&gr, const uint8_t *&ur, const uint16_t *&gsr,
                      const uint16_t *&usr) {
    const bool sh = run_rank(q) == a.k;
    const uint8_t *gb = sh ? a.sgate : a.gu + (size_t)e * a.gu_bytes;
    const uint8_t *ub = sh ? a.sup : gb + (size_t)a.I * row_bytes;
    gr = gb + (size_t)i * row_bytes;
    ur = ub + (size_t)i * row_bytes;
    gsr = usr = nullptr;
    if constexpr (fmt_quant(FMT)) {
      const uint16_t *gs = sh ? a.sgate_s : a.gu_s + (size_t)e * a.gu_scales;
      const uint16_t *us = sh ? a.sup_s : gs + (size_t)a.I * gnsc;
      gsr = gs + (size_t)i * gnsc;
      usr = us + (size_t)i * gnsc;
    }
  };
  auto down_row = [&](int q, int e, int i) -> const uint8_t * {
    const bool sh = run_rank(q) == a.k;
    return (sh ? a.sdown : a.dn + (size_t)e * a.dn_bytes) + (size_t)i * row_bytes;
  };
  auto down_scales = [&](int q, int e, int i) -> const uint16_t * {  // scale row of i's group
    const bool sh = run_rank(q) == a.k;
    return (sh ? a.sdown_s : a.dn_s + (size_t)e * a.dn_scales) + (size_t)(i / kGroup) * H;
  };
  auto row_of = [&](int rho) -> RowRef { return rho < n0 ? RowRef{0, i00 + rho} : RowRef{1, i01 + rho - n0}; };

  // Stage rows [r0, r0 + n) of the block's rows (down, transposed) into LDS.
  auto stage = [&](int r0, int n, int e0, int e1) {
    const int per_row = (int)(row_bytes / 16);
    const int total = n * per_row;
    for (int p = 0; p * kData < total; p++) {
      int qd = p * kData + dt;
      qd = qd < total ? qd : total - 1;  // the tail reloads a valid piece that is never used
      const RowRef rr = row_of(r0 + qd / per_row);
      const uint8_t *src = down_row(rr.seg, rr.seg ? e1 : e0, rr.i) + (size_t)(qd % per_row) * 16;
      auto *dst = (__attribute__((address_space(3))) void *)(dsl + ((size_t)p * kData + (dt & ~63)) * 16);
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
  };

  // gate_up of the block's rows: act[rho] = silu(g) * u, loads in batches of
  // kMaxRowsPerGroup rows per lane group, all issued before the dots.
  auto gate_up = [&](int e0, int e1) {
    constexpr int RIF = rows_in_flight<FMT, ITER>();
    for (int b0 = g; b0 < nrows; b0 += RIF * groups) {
      if constexpr (ITER > 0) {
        uint4 vg[RIF][ITER], vu[RIF][ITER];
        const uint16_t *sgp[RIF], *sup[RIF];
#pragma unroll
        for (int qq = 0; qq < RIF; qq++) {
          const int rho = b0 + qq * groups;
          if (rho < nrows) {
            const RowRef rr = row_of(rho);
            const uint8_t *gr, *ur;
            gate_ptr(rr.seg, rr.seg ? e1 : e0, rr.i, gr, ur, sgp[qq], sup[qq]);
#pragma unroll
            for (int c = 0; c < ITER; c++) {
              vg[qq][c] = *reinterpret_cast<const uint4 *>(gr + (size_t)(sl + c * lpr) * 16);
              vu[qq][c] = *reinterpret_cast<const uint4 *>(ur + (size_t)(sl + c * lpr) * 16);
            }
          }
        }
        wait_x();
#pragma unroll
        for (int qq = 0; qq < RIF; qq++) {
          const int rho = b0 + qq * groups;
          float gv = 0.0f, uv = 0.0f;
          if (rho < nrows) {
#pragma unroll
            for (int c = 0; c < ITER; c++) {
              const int ch = sl + c * lpr;
              float dg = chunk_dot<FMT>(vg[qq][c], xs + ch * EPC);
              float du = chunk_dot<FMT>(vu[qq][c], xs + ch * EPC);
              if constexpr (fmt_quant(FMT)) {
                dg *= f16_to_f32(sgp[qq][(ch * EPC) / kGroup]);
                du *= f16_to_f32(sup[qq][(ch * EPC) / kGroup]);
              }
              gv += dg;
              uv += du;
            }
          }
          gv = group_sum(gv, lpr);
          uv = group_sum(uv, lpr);
          if (sl == 0 && rho < nrows) act[rho] = silu_ref(gv) * uv;
        }
      } else {
        wait_x();
#pragma unroll 1
        for (int qq = 0; qq < RIF; qq++) {
          const int rho = b0 + qq * groups;
          if (rho >= nrows) break;
          const RowRef rr = row_of(rho);
          const uint8_t *gr, *ur;
          const uint16_t *gsr, *usr;
          gate_ptr(rr.seg, rr.seg ? e1 : e0, rr.i, gr, ur, gsr, usr);
          float gv = row_dot_rt<FMT>(gr, gsr, xs, sl, lpr, nch);
          float uv = row_dot_rt<FMT>(ur, usr, xs, sl, lpr, nch);
          gv = group_sum(gv, lpr);
          uv = group_sum(uv, lpr);
          if (sl == 0) act[rho] = silu_ref(gv) * uv;
        }
      }
    }
  };

  bool need_exact = false;
  int te0 = 0, te1 = 0;  // tentative experts of the two runs (data waves)
  if (ctl) {
    // ---- control wave: routing; the shared gate for a shared run
    const bool has_routed = rank0 != a.k;
    if (has_routed && a.sb) {
      const bool ok = certified_select_nj<NJ>(a.sb + (size_t)t * a.E * 2, a.E, a.k, a.scope,
                                              writer ? a.ids + (size_t)t * a.k : nullptr,
                                              writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w, -2,
                                              s_spec);
      need_exact = !ok;
    } else if (has_routed && threadIdx.x < a.k) {
      s_ids[threadIdx.x] = a.ids[(size_t)t * a.k + threadIdx.x];
      s_w[threadIdx.x] = a.weights[(size_t)t * a.k + threadIdx.x];
    }
    if ((nruns > 1 ? rank1 : rank0) == a.k) {
      wait_x();
      float sgv = 0.0f;  // shared-expert gate, model/moe.go:89-93
      for (int i = threadIdx.x; i < H; i += 64) sgv = fmaf(xs[i], a.shared_gate[i], sgv);
      sgv = group_sum(sgv, 64);
      if (threadIdx.x == 0) s_sg = 1.0f / (1.0f + (float)exp(-(double)sgv));
    }
  } else {
    // ---- data waves: wait for the tentative experts of the block's runs
    for (int q = 0; q < nruns; q++) {
      const int rk = run_rank(q);
      if (rk == a.k || !a.sb) continue;
      while (__hip_atomic_load(&s_spec[rk], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
        __builtin_amdgcn_s_sleep(1);
    }
    te0 = run_expert(0, true);
    te1 = nruns > 1 ? run_expert(1, true) : 0;
    stage(0, min(SR, nrows), te0, te1);
    gate_up(te0, te1);
  }
  if (threadIdx.x == 0) s_exact = need_exact;
  __syncthreads();  // act, s_ids/s_w (when certified), s_sg, s_exact
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
  // data waves recompute when a tentative expert was not the final one
  const bool redo = a.sb && ((rank0 != a.k && e0 != s_spec[rank0] - 1) ||
                             (nruns > 1 && rank1 != a.k && e1 != s_spec[rank1] - 1));
  if (redo) {
    if (!ctl) __builtin_amdgcn_s_waitcnt(0);  // earlier LDS-direct loads have landed
    __syncthreads();
    if (!ctl) {
      stage(0, min(SR, nrows), e0, e1);
      gate_up(e0, e1);
    }
    __syncthreads();
  }
  // fold the routing weight (or the shared gate) into act
  for (int rho = threadIdx.x; rho < nrows; rho += kFusedBlock) {
    const int rk = rho < n0 ? rank0 : rank1;
    act[rho] *= rk == a.k ? s_sg : s_w[rk];
  }

  // ---- down: out[t, j] += sum_rho act[rho] * downT[row rho][j].  Thread
  // (ig, jc) owns the outputs of chunk jc (and of chunk jc + kData when the
  // row has more chunks than there are data threads) over rows ig, ig + IG, ...
  constexpr int NP = kDownPasses<FMT>;
  const int JC = nch;
  const int IG = JC >= kData ? 1 : kData / JC;
  const int jc = dt % JC, ig = dt / JC;  // threads with ig >= IG idle here
  float acc[NP][EPC];
#pragma unroll
  for (int pp = 0; pp < NP; pp++)
#pragma unroll
    for (int q = 0; q < EPC; q++) acc[pp][q] = 0.0f;
  for (int s0 = 0; s0 < nrows; s0 += SR) {
    const int srows = min(SR, nrows - s0);
    if (s0 > 0 && !ctl) stage(s0, srows, e0, e1);
    if (!ctl) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the whole stage is in LDS (and act is scaled)
    if (!ctl && ig < IG) {
#pragma unroll
      for (int pp = 0; pp < NP; pp++) {
        const int jcp = jc + pp * kData;
        if (jcp >= JC) break;
        if constexpr (fmt_quant(FMT)) {
          // per row: the scales of its (expert, 32-row group) for these outputs
          int cur = -1;
          float sc[EPC];
          for (int i = ig; i < srows; i += IG) {
            const RowRef rr = row_of(s0 + i);
            const int key = rr.seg * 65536 + rr.i / kGroup;
            if (key != cur) {
              const uint16_t *sp = down_scales(rr.seg, rr.seg ? e1 : e0, rr.i) + jcp * EPC;
#pragma unroll
              for (int q = 0; q < EPC; q++) sc[q] = f16_to_f32(sp[q]);
              cur = key;
            }
            const uint4 v = *reinterpret_cast<const uint4 *>(dsl + (size_t)i * row_bytes + (size_t)jcp * 16);
            chunk_axpy_scaled<FMT>(v, act[s0 + i], sc, acc[pp]);
          }
        } else {
          const unsigned char *col = dsl + (size_t)jcp * 16;
          int i = ig;
          for (; i + 3 * IG < srows; i += 4 * IG) {  // four LDS reads in flight
            uint4 v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = *reinterpret_cast<const uint4 *>(col + (size_t)(i + r * IG) * row_bytes);
#pragma unroll
            for (int r = 0; r < 4; r++) chunk_axpy<FMT>(v[r], act[s0 + i + r * IG], acc[pp]);
          }
          for (; i < srows; i += IG)
            chunk_axpy<FMT>(*reinterpret_cast<const uint4 *>(col + (size_t)i * row_bytes), act[s0 + i], acc[pp]);
        }
      }
    }
    __syncthreads();  // before the next stage (or the partials) overwrite LDS
  }
  // combine the IG partial sums of each output through LDS, add to out
  float *part = reinterpret_cast<float *>(dsl);
  if (!ctl && ig < IG) {
#pragma unroll
    for (int pp = 0; pp < NP; pp++) {
      const int jcp = jc + pp * kData;
      if (jcp < JC) {
#pragma unroll
        for (int q = 0; q < EPC; q++) part[(size_t)ig * H + jcp * EPC + q] = acc[pp][q];
      }
    }
  }
  __syncthreads();
  float *out_t = a.out + (size_t)t * H;
  for (int j = threadIdx.x; j < H; j += kFusedBlock) {
    float v = 0.0f;
    for (int q = 0; q < IG; q++) v += part[(size_t)q * H + j];
    atomicAdd(out_t + j, v);
  }
}

template <int FMT, int ITER, int NJ>
static void fused_launch(const FusedArgs &a0, hipStream_t st) {
  FusedArgs a = a0;
  // split each token's k*I (+ Is) intermediate rows evenly over about one
  // wave of blocks per CU, at most kMaxRows rows and two experts per block
  const int U = a.k_routed * a.I + (a.with_shared ? a.Is : 0);
  const int rmax = min(kMaxRows, min(a.k_routed ? a.I : a.Is, a.with_shared ? a.Is : a.I));
  int nb = max(1, (a.n_cu + a.T - 1) / a.T);
  nb = max(nb, (U + rmax - 1) / rmax);
  a.rb = (U + nb - 1) / nb;
  a.nb = (U + a.rb - 1) / a.rb;
  const int blocks = a.T * a.nb;
  const size_t lds = fused_lds_bytes<FMT>(a.H, a.E);
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

template <int FMT>
static void fused_fmt(const FusedArgs &a, hipStream_t st) {
  switch (iter_of(FMT, a.H)) {
  case 1: fused_nj<FMT, 1>(a, st); break;
  case 2: fused_nj<FMT, 2>(a, st); break;
  case 4: fused_nj<FMT, 4>(a, st); break;
  default: fused_nj<FMT, 0>(a, st); break;
  }
}

bool fused_supported(int fmt, int H, int E) {
  size_t lds = 0;
  int sr = 0;
  switch (fmt) {
  case kF32: lds = fused_lds_bytes<kF32>(H, E); sr = stage_rows<kF32>(H); break;
  case kBF16: lds = fused_lds_bytes<kBF16>(H, E); sr = stage_rows<kBF16>(H); break;
  case kINT8: lds = fused_lds_bytes<kINT8>(H, E); sr = stage_rows<kINT8>(H); break;
  default: lds = fused_lds_bytes<kINT4>(H, E); sr = stage_rows<kINT4>(H); break;
  }
  const int epc = fmt == kF32 ? 4 : fmt == kBF16 ? 8 : fmt == kINT8 ? 16 : 32;
  const int passes = fmt == kINT4 ? 1 : 2;
  return sr > 0 && H / epc <= passes * kData && lds <= 160 * 1024 - 2048;  // static LDS < 1 KiB
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
  switch (a.fmt) {
  case kF32: fused_fmt<kF32>(a, st); break;
  case kBF16: fused_fmt<kBF16>(a, st); break;
  case kINT8: fused_fmt<kINT8>(a, st); break;
  default: fused_fmt<kINT4>(a, st); break;
  }
  return hipGetLastError();
}

}  // namespace qmoe
