// gate_up.hip -- expert gate_up GEMV with fused SwiGLU (bandwidth-bound, decode-sized T).
//
// Weight rows stream from HBM once per (token, rank) with 16-byte per-lane
// loads along K: a group of `lpr` lanes covers 16*lpr contiguous bytes, and
// each lane issues all ITER of its loads for a row before any arithmetic, so a
// wave keeps ITER*1 KiB in flight.  Elements are widened / dequantised in
// registers and dotted with f32 activations staged in LDS.  Accumulation is f32
// FMA: the reference sums sequentially, so these outputs match it within f32
// rounding (the tolerance path), not bit for bit.
//
// gate_up (model/moe.go:64-75, shared expert model/model.go:350-358): a lane
//   group computes gate row o and up row o of one expert for one token and
//   writes silu(g) * u; the shared expert rides in the same launch as rank k
//   (grid.y == k), and also produces sigmoid(shared_gate . x) (moe.go:89-93).
#include "gemv_common.hpp"

namespace qmoe {

// Rows [o_begin, o_end) of one gate/up pair of matrices for one token.
template <int FMT, int ITER>
__device__ __forceinline__ void gate_up_rows(const uint8_t *gbase, const uint8_t *ubase, const uint16_t *gsb,
                                             const uint16_t *usb, const float *xs, int H, int o_begin,
                                             int o_end, float *act_row) {
  constexpr int EPC = Chunk<FMT>::kElems;
  const int nch = H / EPC;
  const int lpr = lanes_per_row(nch);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per_wave = 64 / lpr;
  const int sub = lane / lpr, sl = lane % lpr;
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
  const int nsc = H / kGroup;
  for (int o = o_begin + wave * per_wave + sub; o < o_end; o += (kBlock / 64) * per_wave) {
    float g = row_dot_any<FMT, ITER>(gbase + (size_t)o * row_bytes, gsb ? gsb + (size_t)o * nsc : nullptr, xs, sl,
                                     lpr, nch);
    float u = row_dot_any<FMT, ITER>(ubase + (size_t)o * row_bytes, usb ? usb + (size_t)o * nsc : nullptr, xs, sl,
                                     lpr, nch);
    g = group_sum(g, lpr);
    u = group_sum(u, lpr);
    if (sl == 0) act_row[o] = silu_ref(g) * u;
  }
}

// The shared expert's projections share K = H with the routed experts, so
// its compile-time chunk count is the routed one when the formats agree.
template <int EFMT, int EITER, int SFMT, int SITER = (SFMT == EFMT ? EITER : 0)>
__global__ void __launch_bounds__(kBlock) gate_up_kernel(GateUpArgs a, int rows_per_block, int srows_per_block) {
  extern __shared__ __align__(16) float xs[];
  const int t = blockIdx.z;
  const int r = blockIdx.y;
  const int H = a.H;
  const bool shared = r == a.k;
  const int rows = shared ? a.Is : a.I;
  const int rpb = shared ? srows_per_block : rows_per_block;
  const int o_begin = blockIdx.x * rpb;
  if (o_begin >= rows) return;  // shared expert has fewer row blocks
  for (int i = threadIdx.x * 4; i < H; i += kBlock * 4)
    *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
  __syncthreads();
  const int o_end = min(o_begin + rpb, rows);
  if (!shared) {
    const int p = t * a.k + r;
    const int e = a.ids[p];
    const uint8_t *gbase = a.gate + (size_t)e * a.expert_bytes;
    const uint16_t *gsb = fmt_quant(EFMT) ? a.gate_s + (size_t)e * a.expert_scales : nullptr;
    const uint8_t *ubase = gbase + fmt_matrix_bytes(EFMT, a.I, H);
    const uint16_t *usb = gsb ? gsb + (size_t)a.I * (H / kGroup) : nullptr;
    gate_up_rows<EFMT, EITER>(gbase, ubase, gsb, usb, xs, H, o_begin, o_end, a.act + (size_t)p * a.I);
  } else {
    if (blockIdx.x == 0 && threadIdx.x < 64) {
      // shared-expert gate, model/moe.go:89-93
      const int lane = threadIdx.x;
      float g = 0.0f;
      for (int i = lane; i < H; i += 64) g = fmaf(xs[i], a.shared_gate[i], g);
      g = group_sum(g, 64);
      if (lane == 0) a.sg[t] = 1.0f / (1.0f + (float)exp(-(double)g));
    }
    gate_up_rows<SFMT, SITER>(a.sgate, a.sup, a.sgate_s, a.sup_s, xs, H, o_begin, o_end,
                              a.act_s + (size_t)t * a.Is);
  }
}

template <int EFMT, int EITER, int SFMT>
static void gate_up_launch(const GateUpArgs &a, hipStream_t st) {
  const int rpb = rows_per_block_of(EFMT, a.H);
  const int srpb = a.Is ? rows_per_block_of(SFMT, a.H) : 1;
  const int bx = max((a.I + rpb - 1) / rpb, a.Is ? (a.Is + srpb - 1) / srpb : 0);
  dim3 grid(bx, a.k + (a.Is ? 1 : 0), a.T);
  hipLaunchKernelGGL((gate_up_kernel<EFMT, EITER, SFMT>), grid, dim3(kBlock), (size_t)a.H * sizeof(float), st, a,
                     rpb, srpb);
}

template <int EFMT, int EITER>
static void gate_up_sf(const GateUpArgs &a, hipStream_t st) {
  switch (a.Is ? a.sfmt : EFMT) {
  case kF32: gate_up_launch<EFMT, EITER, kF32>(a, st); break;
  case kBF16: gate_up_launch<EFMT, EITER, kBF16>(a, st); break;
  case kINT8: gate_up_launch<EFMT, EITER, kINT8>(a, st); break;
  default: gate_up_launch<EFMT, EITER, kINT4>(a, st); break;
  }
}

template <int EFMT>
static void gate_up_e(const GateUpArgs &a, hipStream_t st) {
  switch (iter_of(EFMT, a.H)) {
#define C(F, I) case I: gate_up_sf<EFMT, I>(a, st); break;
    QMOE_ITER_CASES(EFMT, C)
#undef C
  default: gate_up_sf<EFMT, 0>(a, st); break;
  }
}

hipError_t launch_gate_up_gemv(const GateUpArgs &a, hipStream_t st) {
  switch (a.fmt) {
  case kF32: gate_up_e<kF32>(a, st); break;
  case kBF16: gate_up_e<kBF16>(a, st); break;
  case kINT8: gate_up_e<kINT8>(a, st); break;
  default: gate_up_e<kINT4>(a, st); break;
  }
  return hipGetLastError();
}

}  // namespace qmoe
