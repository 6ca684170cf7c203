// fused.hip -- the decode path (T <= 8): one kernel per forward after the
// router partials.
//
// Block = (token t, rank r, chunk c of 32 intermediate rows).  It
//   1. selects the token's experts from the router partials (certified, with
//      the exact sequential fallback; select.hpp), rank k being the shared
//      expert whose weight is sigmoid(shared_gate . x) (model/moe.go:86-97);
//   2. computes gate and up rows [32c, 32c+32) of its expert against x in LDS
//      and keeps act = silu(g) * u (model/moe.go:64-75) in LDS;
//   3. streams the matching 32 columns of the expert's down matrix for all H
//      output rows and adds w_r * (down[:, 32c:32c+32] . act) into out[t] with
//      f32 atomics (model/moe.go:76-84).  out is zeroed by the router kernel.
// Splitting the intermediate dimension across blocks removes the dependency
// between the gate_up and the down products, so the layer needs no second
// launch and no in-kernel handoff between blocks.  The atomics make the order
// of the final f32 sums run-dependent (within f32 rounding of the reference's
// rank-ordered sum); the f32 path with rank-ordered sums is the mid-T path.
//
// Work to blocks, XCD-aware: one 32-column slice of a down row covers 16-128
// bytes, so G = 128 B / slice consecutive chunks share the down matrix's cache
// lines.  Workgroups go to the 8 XCDs round-robin by linear id, so the G
// chunks of a line group are given linear ids that share an XCD (and its L2).
#include "gemv_common.hpp"
#include "select.hpp"

namespace qmoe {

constexpr int kFusedBlock = 512;
constexpr int kCH = 32;     // intermediate rows per block
constexpr int kXcds = 8;

template <int FMT>
__host__ __device__ constexpr int line_group() {
  // bytes of one 32-column slice: f32 128, bf16 64, int8 32, int4 16
  return 128 / (kCH * fmt_bytes_x2(FMT) / 2);
}

template <int FMT, int ITER, int NJ>
__global__ void __launch_bounds__(kFusedBlock) expert_fused_kernel(FusedArgs a) {
  constexpr int G = line_group<FMT>();
  constexpr int EPC = Chunk<FMT>::kElems;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ids[64];
  __shared__ float s_w[64];
  __shared__ int s_ok;
  __shared__ float s_sg;
  const int H = a.H;
  float *xs = reinterpret_cast<float *>(smem);
  float *act = xs + H;
  float *lt = act + kCH;

  // ---- decode (t, r, chunk) from the linear block id
  const int L = blockIdx.x;
  const int xcd = L % kXcds, slot = L / kXcds;
  const int h = slot % G;
  const int P = (slot / G) * kXcds + xcd;
  const int per_t = a.ranks * a.ng;
  const int t = P / per_t;
  if (t >= a.T) return;
  const int r = (P % per_t) / a.ng;
  const int chunk = (P % a.ng) * G + h;
  const bool shared = r == a.k;
  const int K = shared ? a.Is : a.I;  // intermediate rows of this expert
  const int o0 = chunk * kCH;
  if (o0 >= K) return;

  for (int i = threadIdx.x * 4; i < H; i += kFusedBlock * 4)
    *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
  __syncthreads();

  // ---- 1. routing
  const bool writer = r == 0 && chunk == 0;
  if (!shared) {
    if (threadIdx.x < 64) {
      const bool ok = certified_select_nj<NJ>(a.sb + (size_t)t * a.E * 2, a.E, a.k, a.scope,
                                              writer ? a.ids + (size_t)t * a.k : nullptr,
                                              writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w);
      if (threadIdx.x == 0) s_ok = ok;
    }
    __syncthreads();
    if (!s_ok) {
      exact_logits_block(xs, H, a.rw, a.rs, a.rfmt, a.E, lt);
      __syncthreads();
      if (threadIdx.x < 64)
        select_exact_nj<NJ>(lt, a.E, a.k, a.scope, writer ? a.ids + (size_t)t * a.k : nullptr,
                            writer ? a.weights + (size_t)t * a.k : nullptr, s_ids, s_w);
      if (writer && threadIdx.x == 0) atomicAdd(a.fallbacks, 1u);
    }
  } else if (threadIdx.x < 64) {
    float g = 0.0f;  // shared-expert gate, model/moe.go:89-93
    for (int i = threadIdx.x; i < H; i += 64) g = fmaf(xs[i], a.shared_gate[i], g);
    g = group_sum(g, 64);
    if (threadIdx.x == 0) s_sg = 1.0f / (1.0f + (float)exp(-(double)g));
  }
  __syncthreads();
  const int e = shared ? 0 : s_ids[r];
  const float wgt = shared ? s_sg : s_w[r];

  // ---- 2. gate_up rows [o0, o0 + kCH) -> act (LDS)
  {
    const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
    const int nsc = H / kGroup;
    const uint8_t *gbase = shared ? a.sgate : a.gu + (size_t)e * a.gu_bytes;
    const uint8_t *ubase = shared ? a.sup : gbase + (size_t)a.I * row_bytes;
    const uint16_t *gsb = nullptr, *usb = nullptr;
    if constexpr (fmt_quant(FMT)) {
      gsb = shared ? a.sgate_s : a.gu_s + (size_t)e * a.gu_scales;
      usb = shared ? a.sup_s : gsb + (size_t)a.I * nsc;
    }
    const int nch = H / EPC;
    const int lpr = lanes_per_row(nch);
    const int groups = kFusedBlock / lpr;
    const int g = threadIdx.x / lpr, sl = threadIdx.x % lpr;
    const int nrows = min(kCH, K - o0);
    for (int i0 = g; i0 < nrows; i0 += 2 * groups) {
      const int i1 = i0 + groups;
      const int oa = o0 + i0, ob = o0 + min(i1, nrows - 1);
      // two row pairs in flight per lane group
      float ga = row_dot_any<FMT, ITER>(gbase + (size_t)oa * row_bytes, gsb ? gsb + (size_t)oa * nsc : nullptr, xs,
                                        sl, lpr, nch);
      float ua = row_dot_any<FMT, ITER>(ubase + (size_t)oa * row_bytes, usb ? usb + (size_t)oa * nsc : nullptr, xs,
                                        sl, lpr, nch);
      float gb = 0.0f, ub = 0.0f;
      if (i1 < nrows) {
        gb = row_dot_any<FMT, ITER>(gbase + (size_t)ob * row_bytes, gsb ? gsb + (size_t)ob * nsc : nullptr, xs, sl,
                                    lpr, nch);
        ub = row_dot_any<FMT, ITER>(ubase + (size_t)ob * row_bytes, usb ? usb + (size_t)ob * nsc : nullptr, xs, sl,
                                    lpr, nch);
      }
      ga = group_sum(ga, lpr);
      ua = group_sum(ua, lpr);
      gb = group_sum(gb, lpr);
      ub = group_sum(ub, lpr);
      if (sl == 0) {
        act[i0] = silu_ref(ga) * ua;
        if (i1 < nrows) act[i1] = silu_ref(gb) * ub;
      }
    }
    for (int i = nrows + threadIdx.x; i < kCH; i += kFusedBlock) act[i] = 0.0f;
  }
  __syncthreads();

  // ---- 3. down columns [o0, o0 + kCH) for all H rows, scaled, into out[t]
  {
    constexpr int SEG = kCH * fmt_bytes_x2(FMT) / 2;  // bytes of the slice
    constexpr int LPS = SEG / 16;                      // lanes per row
    constexpr int RPP = kFusedBlock / LPS;             // rows per pass
    constexpr int U = LPS >= 4 ? 8 : 4;                // passes in flight
    const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, K);
    const uint8_t *dbase = (shared ? a.sdown : a.dn + (size_t)e * a.dn_bytes) + (size_t)o0 * fmt_bytes_x2(FMT) / 2;
    const uint16_t *dsb = nullptr;
    if constexpr (fmt_quant(FMT)) dsb = (shared ? a.sdown_s : a.dn_s + (size_t)e * a.dn_scales) + o0 / kGroup;
    const int nsc = K / kGroup;
    const int sl = threadIdx.x % LPS;
    const int jr = threadIdx.x / LPS;
    float *out_t = a.out + (size_t)t * H;
    const float *ac = act + sl * EPC;
    for (int j0 = 0; j0 < H; j0 += U * RPP) {
      uint4 v[U];
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int j = j0 + u * RPP + jr;
        if (j < H) {
          v[u] = *reinterpret_cast<const uint4 *>(dbase + (size_t)j * row_bytes + sl * 16);
          if constexpr (fmt_quant(FMT)) sc[u] = f16_to_f32(dsb[(size_t)j * nsc]);
        } else {
          v[u] = make_uint4(0, 0, 0, 0);
          sc[u] = 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int j = j0 + u * RPP + jr;
        float d = chunk_dot<FMT>(v[u], ac);
        if constexpr (fmt_quant(FMT)) d *= sc[u];
        d = group_sum(d, LPS);
        if (sl == 0 && j < H) atomicAdd(out_t + j, wgt * d);
      }
    }
  }
}

template <int FMT, int ITER, int NJ>
static void fused_launch(const FusedArgs &a0, hipStream_t st) {
  FusedArgs a = a0;
  constexpr int G = line_group<FMT>();
  const int nchunks = (max(a.I, a.Is) + kCH - 1) / kCH;
  a.ng = (nchunks + G - 1) / G;
  a.ranks = a.k + (a.Is ? 1 : 0);
  const int tasks = a.T * a.ranks * a.ng;
  const int blocks = kXcds * G * ((tasks + kXcds - 1) / kXcds);
  const size_t lds = (size_t)(a.H + kCH + a.E) * sizeof(float);
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
