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
// The decode kernel's exchange packs {S, B} into one 64-bit word: S rounded
// to f32 in the high half; in the low half an f32 upper bound of B plus that
// rounding, whose low 8 bits carry the call's tag (setting them only raises
// the value after the bound is first raised by 256 f32 ulps).
__device__ __forceinline__ uint64_t sb_word(double S, double B, uint32_t tag) {
  const float s = (float)S;
  const double b = B + fabs(S - (double)s);
  const float bf = (float)b;
  uint32_t bb = __float_as_uint(bf) + ((double)bf < b ? 1u : 0u);  // b >= 0: rounded up
  bb = ((bb + 0x100u) & ~0xffu) | (tag & 0xffu);
  return ((uint64_t)__float_as_uint(s) << 32) | bb;
}
__device__ __forceinline__ void sb_unword(uint64_t w, double &S, double &B) {
  S = (double)__uint_as_float((uint32_t)(w >> 32));
  B = (double)__uint_as_float((uint32_t)w);
}

__device__ __forceinline__ uint64_t tag_word(double v, uint32_t tag) {
  return ((uint64_t)__double_as_longlong(v) & ~0xffull) | tag;
}
__device__ __forceinline__ double untag_word(uint64_t w) { return __longlong_as_double((long long)(w & ~0xffull)); }
__device__ __forceinline__ void tagged_sb(double S, double B, uint32_t tag, uint64_t &ws, uint64_t &wb) {
  ws = tag_word(S, tag);
  wb = tag_word((B + fabs(S) * 0x1p-42) * (1.0 + 0x1p-40), tag);
}

// A raw 16-byte router chunk widened to f32 exactly as router_chunk does.
template <int FMT>
__device__ inline void widen_chunk(const uint4 raw, uint16_t scale, float (&wv)[Chunk<FMT>::kElems]) {
  const uint32_t u[4] = {raw.x, raw.y, raw.z, raw.w};
  if constexpr (FMT == kF32) {
#pragma unroll
    for (int k = 0; k < 4; k++) wv[k] = __uint_as_float(u[k]);
  } else if constexpr (FMT == kBF16) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      wv[2 * k] = __uint_as_float(u[k] << 16);
      wv[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
    }
  } else if constexpr (FMT == kINT8) {
    const float sc = f16_to_f32(scale);
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int b = 0; b < 4; b++) wv[4 * k + b] = (float)(int8_t)((u[k] >> (8 * b)) & 0xffu) * sc;
  } else {
    const float sc = f16_to_f32(scale);
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t byte = (u[k] >> (8 * b)) & 0xffu;
        wv[8 * k + 2 * b] = (float)((int)(byte >> 4) - 8) * sc;
        wv[8 * k + 2 * b + 1] = (float)((int)(byte & 0xfu) - 8) * sc;
      }
  }
}

// The reference's logit of one router row against x in LDS: the sequential
// f32 sum of model/tensors.go:77-89 (model/model.go:167-176,
// model/moe.go:159-162), streaming the row in 16-byte chunks, G at a time,
// the next G in flight while the current ones are widened and summed.
template <int FMT, int G = 8>
__device__ __forceinline__ float exact_row_logit(const float *__restrict__ xs, int H, const uint8_t *__restrict__ row,
                                 const uint16_t *__restrict__ srow) {
#pragma clang fp contract(off)
  constexpr int EPC = Chunk<FMT>::kElems;
  const int nch = H / EPC;
  uint4 raw[2][G];
  uint16_t sc[2][G];
  auto fetch = [&](int g, int c0) {
#pragma unroll
    for (int c = 0; c < G; c++) {
      const int ch = min(c0 + c, nch - 1);
      raw[g][c] = *reinterpret_cast<const uint4 *>(row + (size_t)ch * 16);
      sc[g][c] = fmt_quant(FMT) ? srow[(ch * EPC) / kGroup] : (uint16_t)0;
    }
  };
  float L = 0.0f;
  fetch(0, 0);
  for (int c0 = 0; c0 < nch; c0 += 2 * G) {
    fetch(1, c0 + G);
#pragma unroll
    for (int c = 0; c < G; c++)
      if (c0 + c < nch) {
        float wv[EPC];
        widen_chunk<FMT>(raw[0][c], sc[0][c], wv);
#pragma unroll
        for (int i = 0; i < EPC; i++) L = L + xs[(c0 + c) * EPC + i] * wv[i];
      }
    fetch(0, c0 + 2 * G);
#pragma unroll
    for (int c = 0; c < G; c++)
      if (c0 + G + c < nch) {
        float wv[EPC];
        widen_chunk<FMT>(raw[1][c], sc[1][c], wv);
#pragma unroll
        for (int i = 0; i < EPC; i++) L = L + xs[(c0 + G + c) * EPC + i] * wv[i];
      }
  }
  return L;
}

// Exact logits of one token for every expert into lt, by the first nthreads
// threads of the block (the certification's last resort): a bf16 router, the
// format of every certified router in practice, streams its rows; the other
// formats take a plain element loop (same sums, fewer registers).
__device__ __forceinline__ void exact_logits_block(const float *__restrict__ xs, int H, const uint8_t *__restrict__ w,
                                                   const uint16_t *__restrict__ sc, int fmt, int E,
                                                   float *__restrict__ lt, int nthreads) {
#pragma clang fp contract(off)
  const int64_t row_bytes = fmt_matrix_bytes(fmt, 1, H);
  for (int e = threadIdx.x; e < E; e += nthreads) {
    const uint8_t *row = w + (size_t)e * row_bytes;
    const uint16_t *srow = fmt_quant(fmt) ? sc + (size_t)e * (H / kGroup) : nullptr;
    if (fmt == kBF16) {
      lt[e] = exact_row_logit<kBF16>(xs, H, row, nullptr);
      continue;
    }
    float acc = 0.0f;
    if (fmt == kF32) {
      for (int h = 0; h < H; h++) acc = acc + xs[h] * reinterpret_cast<const float *>(row)[h];
    } else if (fmt == kINT8) {
      for (int h = 0; h < H; h++) {
        const float wv = (float)(int8_t)row[h] * f16_to_f32(srow[h / kGroup]);
        acc = acc + xs[h] * wv;
      }
    } else {
      for (int h = 0; h < H; h++) {
        const uint8_t b = row[h / 2];
        const int nib = (h % 2 == 0) ? (b >> 4) : (b & 0xf);
        const float wv = ((float)nib - 8.0f) * f16_to_f32(srow[h / kGroup]);
        acc = acc + xs[h] * wv;
      }
    }
    lt[e] = acc;
  }
}

// Rescue of a failed certification (one full wavefront): the candidates
// whose upper bound reaches the k-th selected one's lower bound (less the f32
// rounding of the round keys) -- the only ones that can be in the top k or
// change its order -- get their reference logits computed exactly, one
// candidate per lane (the sequential f32 sum of model/tensors.go:77-89,
// model/moe.go:159-162 on x in LDS), and the selection is certified again with
// their bounds at zero.  S and B are updated in place.  Returns false (nothing
// written) when more than 64 candidates qualify or certification still fails,
// which takes a near or exact tie of reference logits.  list: 64 ints of LDS.
template <int FMT, int NJ>
__device__ __forceinline__ bool refine_select(double (&S)[NJ], double (&B)[NJ], double kth_lo, int E, int k, int scope,
                              const float *__restrict__ xs, int H, const uint8_t *__restrict__ rw,
                              const uint16_t *__restrict__ rs, int *list, int32_t *g_ids, float *g_w, int *s_ids,
                              float *s_w) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const double thr = kth_lo - fabs(kth_lo) * 0x1p-20 - 0x1p-60;
  bool in[NJ];
  int idx[NJ];
  int n = 0;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    in[j] = e < scope && e < E && S[j] + B[j] >= thr;
    const uint64_t m = __ballot(in[j]);
    idx[j] = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    n += __popcll(m);
  }
  if (n > 64) return false;
#pragma unroll
  for (int j = 0; j < NJ; j++)
    if (in[j]) list[idx[j]] = lane + 64 * j;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  float L = 0.0f;
  if (lane < n) {
    const int e = list[lane];
    L = exact_row_logit<FMT>(xs, H, rw + (size_t)e * fmt_matrix_bytes(FMT, 1, H),
                             fmt_quant(FMT) ? rs + (size_t)e * (H / kGroup) : nullptr);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const float Lj = __uint_as_float(__builtin_amdgcn_ds_bpermute(4 * (idx[j] & 63), __float_as_uint(L)));
    if (in[j]) {
      S[j] = (double)Lj;
      B[j] = 0.0;
    }
  }
  return certified_select_regs<NJ>(S, B, E, k, scope, g_ids, g_w, s_ids, s_w);
}

}  // namespace qmoe
