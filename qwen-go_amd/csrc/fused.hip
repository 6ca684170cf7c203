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
constexpr int kData = 512;                    // data threads (8 waves)
constexpr int kFusedBlock = kCtl + kData;
constexpr int kCH = 32;                       // intermediate rows per block
constexpr int kDownLds = 128 * 1024;          // LDS bytes for down-slice staging
constexpr int kMaxRowsPerGroup = 4;

// Rows of the transposed down slice staged per LDS pass.
template <int FMT>
__host__ __device__ inline int stage_rows(int H) {
  const int64_t row = fmt_matrix_bytes(FMT, 1, H);
  int r = (int)(kDownLds / row);
  return r >= kCH ? kCH : (r >= 16 ? 16 : (r >= 8 ? 8 : 0));
}
template <int FMT>
__host__ inline size_t fused_lds_bytes(int H, int E) {
  const size_t head = ((size_t)(H + kCH + E) * 4 + 15) / 16 * 16;
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

template <int FMT, int ITER>
struct GateUpPipe {
  uint4 g[kMaxRowsPerGroup][ITER > 0 ? ITER : 1];
  uint4 u[kMaxRowsPerGroup][ITER > 0 ? ITER : 1];
};

template <int FMT, int ITER, int NJ>
__global__ void __launch_bounds__(kFusedBlock) expert_fused_kernel(FusedArgs a) {
  constexpr int EPC = Chunk<FMT>::kElems;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ids[64];
  __shared__ float s_w[64];
  __shared__ float s_sg;
  __shared__ int s_spec;
  const int H = a.H;
  float *xs = reinterpret_cast<float *>(smem);
  float *act = xs + H;
  float *lt = act + kCH;
  unsigned char *dsl = smem + ((size_t)(H + kCH + a.E) * 4 + 15) / 16 * 16;

  // ---- (t, r, chunk) from the linear block id: consecutive ids walk the
  // chunks of one (t, r), so each expert's chunks spread over all XCDs
  const int L = blockIdx.x;
  const int per_t = a.ranks * a.nchunks;
  const int t = L / per_t;
  if (t >= a.T) return;
  const int r = (L % per_t) / a.nchunks;
  const int chunk = L % a.nchunks;
  const bool shared = a.with_shared && r == a.k_routed;
  const int K = shared ? a.Is : a.I;  // intermediate rows of this expert
  const int o0 = chunk * kCH;
  if (o0 >= K) return;
  const int nrows = min(kCH, K - o0);
  const bool ctl = threadIdx.x < kCtl;
  const int dt = threadIdx.x - kCtl;
  const bool writer = !shared && r == 0 && chunk == 0 && a.sb;

  if (threadIdx.x == 0) s_spec = (shared || !a.sb) ? 1 : 0;
  for (int i = threadIdx.x * 4; i < H; i += kFusedBlock * 4)
    *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
  __syncthreads();

  // ---- geometry
  const int64_t gu_row = fmt_matrix_bytes(FMT, 1, H);
  const int gnsc = H / kGroup;
  const int nch = H / EPC;
  const int lpr = lanes_per_row(nch);
  const int groups = kData / lpr;
  const int g = dt / lpr, sl = dt % lpr;
  const int SR = stage_rows<FMT>(H);          // down rows per LDS stage
  const int64_t dn_row = gu_row;              // a transposed down row holds H values

  auto expert_ptrs = [&](int e, const uint8_t *&gb, const uint8_t *&ub, const uint16_t *&gs, const uint16_t *&us,
                         const uint8_t *&db, const uint16_t *&ds) {
    gb = shared ? a.sgate : a.gu + (size_t)e * a.gu_bytes;
    ub = shared ? a.sup : gb + (size_t)a.I * gu_row;
    db = (shared ? a.sdown : a.dn + (size_t)e * a.dn_bytes) + (size_t)o0 * dn_row;
    gs = us = ds = nullptr;
    if constexpr (fmt_quant(FMT)) {
      gs = shared ? a.sgate_s : a.gu_s + (size_t)e * a.gu_scales;
      us = shared ? a.sup_s : gs + (size_t)a.I * gnsc;
      ds = (shared ? a.sdown_s : a.dn_s + (size_t)e * a.dn_scales) + (size_t)(o0 / kGroup) * H;
    }
  };

  // gate_up for the data waves: loads for all row pairs first, then the dots.
  auto gate_up = [&](const uint8_t *gb, const uint8_t *ub, const uint16_t *gs, const uint16_t *us) {
    if constexpr (ITER > 0) {
      GateUpPipe<FMT, ITER> pp;
#pragma unroll
      for (int q = 0; q < kMaxRowsPerGroup; q++) {
        const int i = g + q * groups;
        if (i < nrows) {
#pragma unroll
          for (int c = 0; c < ITER; c++) {
            pp.g[q][c] = *reinterpret_cast<const uint4 *>(gb + (size_t)(o0 + i) * gu_row + (size_t)(sl + c * lpr) * 16);
            pp.u[q][c] = *reinterpret_cast<const uint4 *>(ub + (size_t)(o0 + i) * gu_row + (size_t)(sl + c * lpr) * 16);
          }
        }
      }
#pragma unroll
      for (int q = 0; q < kMaxRowsPerGroup; q++) {
        const int i = g + q * groups;
        float gv = 0.0f, uv = 0.0f;
        if (i < nrows) {
#pragma unroll
          for (int c = 0; c < ITER; c++) {
            const int ch = sl + c * lpr;
            float dg = chunk_dot<FMT>(pp.g[q][c], xs + ch * EPC);
            float du = chunk_dot<FMT>(pp.u[q][c], xs + ch * EPC);
            if constexpr (fmt_quant(FMT)) {
              const int si = (o0 + i) * gnsc + (ch * EPC) / kGroup;
              dg *= f16_to_f32(gs[si]);
              du *= f16_to_f32(us[si]);
            }
            gv += dg;
            uv += du;
          }
        }
        gv = group_sum(gv, lpr);
        uv = group_sum(uv, lpr);
        if (sl == 0 && i < nrows) act[i] = silu_ref(gv) * uv;
      }
    } else {
      for (int i = g; i < nrows; i += groups) {
        float gv = row_dot_rt<FMT>(gb + (size_t)(o0 + i) * gu_row, gs ? gs + (size_t)(o0 + i) * gnsc : nullptr, xs,
                                   sl, lpr, nch);
        float uv = row_dot_rt<FMT>(ub + (size_t)(o0 + i) * gu_row, us ? us + (size_t)(o0 + i) * gnsc : nullptr, xs,
                                   sl, lpr, nch);
        gv = group_sum(gv, lpr);
        uv = group_sum(uv, lpr);
        if (sl == 0) act[i] = silu_ref(gv) * uv;
      }
    }
    for (int i = nrows + dt; i < kCH; i += kData) act[i] = 0.0f;
  };

  int e_spec = 0;
  const uint8_t *gb = nullptr, *ub = nullptr, *db = nullptr;
  const uint16_t *gs = nullptr, *us = nullptr, *ds = nullptr;
  bool need_exact = false;
  if (ctl) {
    // ---- control wave: routing (or the shared gate)
    if (shared) {
      float sgv = 0.0f;  // shared-expert gate, model/moe.go:89-93
      for (int i = threadIdx.x; i < H; i += 64) sgv = fmaf(xs[i], a.shared_gate[i], sgv);
      sgv = group_sum(sgv, 64);
      if (threadIdx.x == 0) s_sg = 1.0f / (1.0f + (float)exp(-(double)sgv));
    } else if (a.sb) {
      const bool ok = certified_select_nj<NJ>(a.sb + (size_t)t * a.E * 2, a.E, a.k, a.scope,
                                              writer ? a.ids + (size_t)t * a.k : nullptr,
                                              writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w, r,
                                              &s_spec);
      need_exact = !ok;
    } else if (threadIdx.x < a.k) {
      s_ids[threadIdx.x] = a.ids[(size_t)t * a.k + threadIdx.x];
      s_w[threadIdx.x] = a.weights[(size_t)t * a.k + threadIdx.x];
    }
  } else {
    // ---- data waves: wait for the tentative expert, then stream
    int v;
    while ((v = __hip_atomic_load(&s_spec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
      __builtin_amdgcn_s_sleep(1);
    if (!shared) e_spec = a.sb ? v - 1 : a.ids[(size_t)t * a.k + r];
    expert_ptrs(e_spec, gb, ub, gs, us, db, ds);
    stage_slice(db, (int64_t)min(SR, nrows) * dn_row, dsl, dt);
    gate_up(gb, ub, gs, us);
  }
  // certification failed: the whole block recomputes the token's routing
  __shared__ int s_exact;
  if (threadIdx.x == 0) s_exact = need_exact;
  __syncthreads();  // act, s_ids/s_w (when certified), s_sg, s_exact
  if (s_exact) {
    exact_logits_block(xs, H, a.rw, a.rs, a.rfmt, a.E, lt, kFusedBlock);
    __syncthreads();
    if (ctl) {
      select_exact_nj<NJ>(lt, a.E, a.k, a.scope, writer ? a.ids + (size_t)t * a.k : nullptr,
                          writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w);
      if (writer && threadIdx.x == 0) atomicAdd(a.fallbacks, 1u);
    }
    __syncthreads();
  }
  const int e = shared ? 0 : s_ids[r];
  const float wgt = shared ? s_sg : s_w[r];
  const bool redo = !shared && a.sb && e != s_spec - 1;
  // every thread (the control wave included) needs the final expert's down
  // pointers: the combine below reads its scales
  if (ctl || !redo) expert_ptrs(e, gb, ub, gs, us, db, ds);
  if (redo) {
    // the tentative expert was not the final one: redo with the final expert
    if (!ctl) {
      __builtin_amdgcn_s_waitcnt(0);  // earlier LDS-direct loads have landed
      expert_ptrs(e, gb, ub, gs, us, db, ds);
    }
    __syncthreads();
    if (!ctl) {
      stage_slice(db, (int64_t)min(SR, nrows) * dn_row, dsl, dt);
      gate_up(gb, ub, gs, us);
    }
    __syncthreads();
  }

  // ---- down: out[t, j] += w * sum_i act[i] * downT[o0 + i][j] over the
  // block's rows i; thread (ig, jc) owns outputs [jc*EPC, jc*EPC + EPC) and
  // rows i = ig, ig + IG, ...
  const int JC = nch;                       // 16-byte chunks per stored row
  const int IG = JC >= kData ? 1 : kData / JC;
  const int jc = dt % JC, ig = dt / JC;
  float acc[EPC];
#pragma unroll
  for (int q = 0; q < EPC; q++) acc[q] = 0.0f;
  for (int s0 = 0; s0 < nrows; s0 += SR) {
    const int srows = min(SR, nrows - s0);
    if (s0 > 0 && !ctl) stage_slice(db + (size_t)s0 * dn_row, (int64_t)srows * dn_row, dsl, dt);
    if (!ctl) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the whole stage is in LDS
    if (!ctl && ig < IG && jc < JC) {
      for (int i = ig; i < srows; i += IG) {
        const uint4 v = *reinterpret_cast<const uint4 *>(dsl + (size_t)i * dn_row + (size_t)jc * 16);
        chunk_axpy<FMT>(v, act[s0 + i], acc);
      }
    }
    __syncthreads();  // before the next stage (or the partials) overwrite LDS
  }
  // combine the IG partial sums of each output through LDS, scale, add to out
  float *part = reinterpret_cast<float *>(dsl);
  if (!ctl && ig < IG) {
#pragma unroll
    for (int q = 0; q < EPC; q++) part[(size_t)ig * H + jc * EPC + q] = acc[q];
  }
  __syncthreads();
  float *out_t = a.out + (size_t)t * H;
  for (int j = threadIdx.x; j < H; j += kFusedBlock) {
    float v = 0.0f;
    for (int q = 0; q < IG; q++) v += part[(size_t)q * H + j];
    if constexpr (fmt_quant(FMT)) v *= f16_to_f32(ds[j]);  // one group: rows o0..o0+31
    atomicAdd(out_t + j, wgt * v);
  }
}

template <int FMT, int ITER, int NJ>
static void fused_launch(const FusedArgs &a0, hipStream_t st) {
  FusedArgs a = a0;
  a.nchunks = (max(a.k_routed ? a.I : 0, a.with_shared ? a.Is : 0) + kCH - 1) / kCH;
  a.ranks = a.k_routed + (a.with_shared ? 1 : 0);
  const int blocks = a.T * a.ranks * a.nchunks;
  const size_t lds = fused_lds_bytes<FMT>(a.H, a.E);
  // dynamic LDS above 64 KiB has to be allowed per kernel (once per size)
  static size_t allowed = 64 * 1024;
  if (lds > allowed) {
    if (hipFuncSetAttribute((const void *)expert_fused_kernel<FMT, ITER, NJ>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return;  // the error stays set; launch_expert_fused reports it
    allowed = lds;
  }
  hipLaunchKernelGGL((expert_fused_kernel<FMT, ITER, NJ>), dim3(blocks), dim3(kFusedBlock), lds, st, a);
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
  return sr > 0 && H / epc <= kData && lds <= 160 * 1024 - 2048;  // static LDS < 1 KiB
}

__global__ void __launch_bounds__(256) zero_kernel(float *__restrict__ p, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) *reinterpret_cast<float4 *>(p + i) = make_float4(0.f, 0.f, 0.f, 0.f);
  else
    for (int64_t q = i; q < n; q++) p[q] = 0.0f;
}

hipError_t launch_zero(float *p, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, p, n);
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
