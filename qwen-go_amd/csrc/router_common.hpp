// router_common.hpp -- the certified router partials of one (token, expert),
// shared by the router kernels and the decode kernel that computes them itself.
//
// The reference sums each logit sequentially in f32,
//   s = 0; for h in 0..H-1: s = fl(s + fl(x[h] * w[e][h]))
// (matmulVec model/tensors.go:77-89, matvecRange model/model.go:167-176,
// quantLinear.forward model/moe.go:159-162).  One wavefront forms the same
// products p_h = fl(x_h * w_h) and sums them in f64 across its lanes, giving
// S ~ the exact sum; the reference's sequential f32 sum differs from S by at
// most
//   B = u (1 + 2 H u) sum_h |S_h|,   u = 2^-24, S_h the exact prefix sums
// (each f32 add rounds with relative error <= u; the f64 prefix sums come from
// a wavefront scan).  Selection then certifies every rank on {S, B} and falls
// back to the exact sequential logits when it cannot.
#pragma once

#include "common.hpp"
#include "select.hpp"

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

__device__ __forceinline__ double seq_sum_bound(double babs, double pabs, int H) {
  const double u = 0x1p-24;
  return u * (1.0 + 2.0 * H * u + 1e-9) * babs + 1e-12 * pabs;
}

// {S, B} of one router row against one token row xt (global or LDS), computed
// by the calling wavefront; lane l owns chunks [l * CPL, (l + 1) * CPL).  Every
// lane receives S and B.
template <int FMT, int CPL>
__device__ __forceinline__ void router_sb_wave(const float *__restrict__ xt, int H, const uint8_t *__restrict__ row,
                                               const uint16_t *__restrict__ srow, double &S, double &B) {
#pragma clang fp contract(off)
  constexpr int EPC = Chunk<FMT>::kElems;
  constexpr int NP = CPL * EPC;  // products per lane
  const int lane = threadIdx.x & 63;
  const int nch = H / EPC;
  float p[NP];
#pragma unroll
  for (int c = 0; c < CPL; c++) {
    const int ch = lane * CPL + c;
    float wv[EPC];
    if (ch < nch) {
      router_chunk<FMT>(row, srow, ch, wv);
#pragma unroll
      for (int i = 0; i < EPC; i += 4) {
        const float4 xv = *reinterpret_cast<const float4 *>(xt + ch * EPC + i);
        p[c * EPC + i + 0] = xv.x * wv[i + 0];
        p[c * EPC + i + 1] = xv.y * wv[i + 1];
        p[c * EPC + i + 2] = xv.z * wv[i + 2];
        p[c * EPC + i + 3] = xv.w * wv[i + 3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < EPC; i++) p[c * EPC + i] = 0.0f;
    }
  }
  double tot = 0.0, pabs = 0.0;
#pragma unroll
  for (int i = 0; i < NP; i++) {
    tot += (double)p[i];
    pabs += fabs((double)p[i]);
  }
  const double inc = wave_incl_scan_f64(tot);  // lane totals -> exact prefix sums
  double run = inc - tot, babs = 0.0;
#pragma unroll
  for (int i = 0; i < NP; i++) {
    run += (double)p[i];
    babs += fabs(run);
  }
  S = readlane_f64(inc, 63);
  babs = wave_sum_f64(babs);
  pabs = wave_sum_f64(pabs);
  B = seq_sum_bound(babs, pabs, H);
}

// Router partials exchanged between workgroups as 64-bit words whose low 8
// bits carry the call's tag (1..255), so that a reader can tell this call's
// words from the previous call's without a separate flag.  Dropping those 8
// bits moves S by less than 2^-43 |S|; the published bound covers that and is
// rounded up past its own dropped bits.
__device__ __forceinline__ uint64_t tag_word(double v, uint32_t tag) {
  return ((uint64_t)__double_as_longlong(v) & ~0xffull) | tag;
}
__device__ __forceinline__ double untag_word(uint64_t w) { return __longlong_as_double((long long)(w & ~0xffull)); }
__device__ __forceinline__ void tagged_sb(double S, double B, uint32_t tag, uint64_t &ws, uint64_t &wb) {
  ws = tag_word(S, tag);
  wb = tag_word((B + fabs(S) * 0x1p-42) * (1.0 + 0x1p-40), tag);
}

}  // namespace qmoe
