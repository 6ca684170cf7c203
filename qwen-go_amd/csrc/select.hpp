// select.hpp -- wavefront helpers for softmax + top-k selection (gfx950).
//
// Selection order is the reference's: a stable descending insertion sort of the
// first `scope` probabilities (model/moe.go:45-53), i.e. descending p with ties
// to the lower expert index.  Keys are packed into one u64 so that a single
// unsigned max over the wavefront yields the winner of a round.
#pragma once

#include "common.hpp"

#include <math.h>

namespace qmoe {

// DPP max of a u64 over each 16-lane row; every lane of the row gets the row max.
__device__ __forceinline__ uint64_t row_max_u64(uint64_t v) {
#define QMOE_DPP_STEP(CTRL)                                                                  \
  {                                                                                          \
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);                                     \
    uint32_t olo = __builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xf, 0xf, false);               \
    uint32_t ohi = __builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xf, 0xf, false);               \
    uint64_t o = ((uint64_t)ohi << 32) | olo;                                                \
    v = o > v ? o : v;                                                                       \
  }
  QMOE_DPP_STEP(0xB1)   // quad_perm [1,0,3,2]
  QMOE_DPP_STEP(0x4E)   // quad_perm [2,3,0,1]
  QMOE_DPP_STEP(0x124)  // row_ror:4
  QMOE_DPP_STEP(0x128)  // row_ror:8
#undef QMOE_DPP_STEP
  return v;
}

// Unsigned max of a u64 over the wavefront, returned uniformly.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = row_max_u64(v);
  uint64_t m = 0;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, 16 * r);
    uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), 16 * r);
    uint64_t o = ((uint64_t)hi << 32) | lo;
    m = o > m ? o : m;
  }
  return m;
}

// Probability key: larger p first, then lower index.  p >= 0 (or NaN, which
// ranks lowest); 0 means "not a candidate".
__device__ __forceinline__ uint64_t prob_key(float p, int e) {
  uint32_t hi = (p == p) ? __float_as_uint(p) + 2u : 1u;  // p in [0, 1]: bits monotone
  return ((uint64_t)hi << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}
__device__ __forceinline__ int key_index(uint64_t key) { return (int)(0xffffffffu - (uint32_t)key); }

// Order-preserving u64 image of a double (for max reductions).
__device__ __forceinline__ uint64_t dkey(double d) {
  uint64_t b = (uint64_t)__double_as_longlong(d);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ __forceinline__ double dkey_inv(uint64_t k) {
  uint64_t b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
  return __longlong_as_double((long long)b);
}

// Inclusive prefix sum of a double over the wavefront (DPP row shifts and
// row broadcasts; lanes outside a step's source range add 0).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
#define QMOE_SCAN_STEP(CTRL, ROWMASK)                                                              \
  {                                                                                                \
    const uint64_t b = (uint64_t)__double_as_longlong(v);                                          \
    const uint32_t lo = __builtin_amdgcn_update_dpp(0u, (uint32_t)b, CTRL, ROWMASK, 0xf, true);    \
    const uint32_t hi = __builtin_amdgcn_update_dpp(0u, (uint32_t)(b >> 32), CTRL, ROWMASK, 0xf, true); \
    v += __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));                             \
  }
  QMOE_SCAN_STEP(0x111, 0xf)  // row_shr:1
  QMOE_SCAN_STEP(0x112, 0xf)  // row_shr:2
  QMOE_SCAN_STEP(0x114, 0xf)  // row_shr:4
  QMOE_SCAN_STEP(0x118, 0xf)  // row_shr:8
  QMOE_SCAN_STEP(0x142, 0xa)  // row_bcast:15 -> rows 1, 3
  QMOE_SCAN_STEP(0x143, 0xc)  // row_bcast:31 -> rows 2, 3
#undef QMOE_SCAN_STEP
  return v;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum over the wavefront (every lane gets it).
__device__ __forceinline__ double wave_sum_f64(double v) { return readlane_f64(wave_incl_scan_f64(v), 63); }

// 4 ulps of an f32 of magnitude x >= 0 (x + 1 keeps it >= 4 ulps of 1).
__device__ __forceinline__ double f32_4ulps(double x) {
  const float f = (float)(x + 1.0) * 1.0000001f;
  const int ex = (int)((__float_as_uint(f) >> 23) & 0xffu) - 127;  // floor(log2 f)
  return __longlong_as_double((long long)((uint64_t)(ex - 21 + 1023) << 52));  // 2^(ex-23) * 4
}

// Exact softmax + selection + renormalisation for one token held by one full
// wavefront, E <= 64 * NJ.  lt: the token's exact f32 logits.  Results go to
// global (g_ids/g_w) and/or LDS (s_ids/s_w) when non-null.
template <int NJ>
__device__ __forceinline__ void select_exact_nj(const float *__restrict__ lt, int E, int k, int scope,
                                                int32_t *g_ids, float *g_w, int *s_ids, float *s_w) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float v[NJ];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lt[e] : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    if (e < E) v[j] = (float)exp((double)(v[j] - mx));
    else v[j] = 0.0f;
  }
  float sum = 0.0f;  // sequential, expert order (tensors.go:113-117)
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int n = min(64, E - 64 * j);
    if (n == 64) {  // a full column: constant lane indices, no loop overhead
#pragma unroll
      for (int l = 0; l < 64; l++) sum = sum + __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v[j]), l));
    } else {
      for (int l = 0; l < n; l++) sum = sum + __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v[j]), l));
    }
  }
  uint64_t key[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    v[j] = v[j] / sum;
    key[j] = e < scope ? prob_key(v[j], e) : 0ull;
  }
  float selp = 0.0f, wsum = 0.0f;
  int seli = 0;
  for (int r = 0; r < k; r++) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++) best = key[j] > best ? key[j] : best;
    best = wave_max_u64(best);
    const int c = key_index(best);
    float pc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      if (lane + 64 * j == c) key[j] = 0;
      if ((c >> 6) == j) pc = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v[j]), c & 63));
    }
    wsum = wsum + pc;  // moe.go:54-57, rank order
    if (lane == r) {
      selp = pc;
      seli = c;
    }
  }
  const float den = wsum + 1e-9f;  // moe.go:63
  if (lane < k) {
    const float w = selp / den;
    if (g_ids) {
      g_ids[lane] = seli;
      g_w[lane] = w;
    }
    if (s_ids) {
      s_ids[lane] = seli;
      s_w[lane] = w;
    }
  }
}

// Certified selection (one full wavefront) from sb = {S_e, B_e} pairs of one
// token: S_e ~ the exact sum of the reference's f32 products for expert e and
// B_e a rigorous bound on the reference's sequential-sum rounding error, so
// the reference's logit L_e lies in [S_e - B_e, S_e + B_e].
//
// Rounds pick the candidate with the largest S (ties to the lower index);
// every lane caches the best of its own candidates, so a round is one
// wavefront max.  Rank r is certified when its lower bound exceeds every
// remaining candidate's upper bound -- the later selected ones and all
// unselected ones -- by delta, enough that p = fl(fl(exp(fl(L - max))) / sum)
// (tensors.go:106-121) stays strictly ordered through its f32 roundings:
// 4 ulps of an f32 of the size of |L - max| plus 2^-20, with |L - max| < 80 so
// that no probability is subnormal.  Returns false (nothing written) when any
// rank fails.  Weights come from the f64 softmax of S.
// f32 max over the wavefront, returned uniformly (DPP within rows, then the
// four row maxima).
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x124, 0xf, 0xf, false)));
  v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x128, 0xf, 0xf, false)));
  const float a0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float a1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float a2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float a3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return fmaxf(fmaxf(a0, a1), fmaxf(a2, a3));
}

// f64 max over the wavefront (uniform).
__device__ __forceinline__ double wave_max_f64(double v) { return dkey_inv(wave_max_u64(dkey(v))); }

// Certified selection (one full wavefront) from sb = {S_e, B_e} pairs of one
// token: S_e ~ the exact sum of the reference's f32 products for expert e and
// B_e a rigorous bound on the reference's sequential-sum rounding error, so
// the reference's logit L_e lies in [S_e - B_e, S_e + B_e].
//
// Rounds pick the candidate with the largest S rounded to f32 (each lane
// sorts its own candidates once, so a round is one f32 wavefront max, a ballot
// for the lowest winning lane and a shift of the winner's list).  The order is then certified with the full bounds:
// rank r must beat every candidate still remaining after it -- the later
// selected ones and all unselected ones -- lower bound over upper bound by
// delta, enough that p = fl(fl(exp(fl(L - max))) / sum) (tensors.go:106-121)
// stays strictly ordered through its f32 roundings: 4 ulps of an f32 of the
// size of |L - max| plus 2^-20, with |L - max| < 80 so that no probability is
// subnormal.  An order that the f32 keys got wrong, or any near or exact tie,
// fails certification; the function then returns false and writes nothing.
// Weights come from the f64 softmax of S.  When spec_slot is given, the
// tentative expert of rank spec_rank is published there (as id + 1) as soon
// as its round ends, before certification.
// certified_select_regs takes the pairs already in registers: lane l holds
// expert l + 64 j in S[j], B[j] (S = -inf, B = 0 past E).
template <int NJ>
__device__ __forceinline__ bool certified_select_regs(const double (&S)[NJ], const double (&B)[NJ], int E, int k,
                                                      int scope, int32_t *g_ids, float *g_w, int *s_ids,
                                                      float *s_w, int spec_rank = -1, int *spec_slot = nullptr,
                                                      double *kth_lo = nullptr) {
  // spec_rank == -2: publish every rank's tentative expert to spec_slot[rank]
  const int lane = threadIdx.x & 63;
  float key[NJ];
  float mh = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    if (e < E) mh = fmaxf(mh, (float)(S[j] + B[j]));
    key[j] = e < scope ? (float)S[j] : -INFINITY;
  }
  // upper bound of the reference's max logit (f32 rounding covered by 2^-20)
  const double mh_all = (double)wave_max_f32(mh);
  const double mx_hi = mh_all + fabs(mh_all) * 0x1p-20 + 0x1p-60;
  // this lane's candidates sorted by key, descending, equal keys by lower
  // slot (the one a scan of the slots meets first): a bitonic network over
  // (key, slot), slot NJ marking an exhausted list
  static_assert((NJ & (NJ - 1)) == 0, "NJ is a power of two");
  float hk[NJ];
  int hj[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    hk[j] = key[j];
    hj[j] = j;
  }
#pragma unroll
  for (int size = 2; size <= NJ; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < NJ; i++) {
        const int l = i ^ stride;
        if (l > i) {
          const bool l_first = hk[l] > hk[i] || (hk[l] == hk[i] && hj[l] < hj[i]);
          const bool swap = (i & size) == 0 ? l_first : !l_first;
          const float tk = hk[i];
          const int tj = hj[i];
          hk[i] = swap ? hk[l] : hk[i];
          hj[i] = swap ? hj[l] : hj[i];
          hk[l] = swap ? tk : hk[l];
          hj[l] = swap ? tj : hj[l];
        }
      }
  int seli = 0;
  double myS = 0.0, myB = 0.0;
  for (int r = 0; r < k; r++) {
    const float m = wave_max_f32(hk[0]);
    const uint64_t win = __ballot(hk[0] != -INFINITY && hk[0] == m);
    const int wl = win ? __ffsll((unsigned long long)win) - 1 : 0;
    const int jw = __builtin_amdgcn_readlane(hj[0], wl);  // the winner's slot (uniform)
    const int c = wl + 64 * jw;
    // jw is uniform: an indexed register read, not a select over the slots
    const double sc = readlane_f64(S[jw], wl), bc = readlane_f64(B[jw], wl);
    if (lane == r) {
      seli = c;
      myS = sc;
      myB = bc;
    }
    if (lane == 0) {  // tentative expert of that rank (spec_slot is in LDS)
      if (spec_rank == -2)
        __hip_atomic_store(spec_slot + r, c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else if (r == spec_rank)
        __hip_atomic_store(spec_slot, c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (lane == wl) {  // the winner's lane retires the slot and drops its head
      key[jw] = -INFINITY;
#pragma unroll
      for (int j = 0; j + 1 < NJ; j++) {
        hk[j] = hk[j + 1];
        hj[j] = hj[j + 1];
      }
      hk[NJ - 1] = -INFINITY;
      hj[NJ - 1] = NJ;
    }
  }
  // largest upper bound among the candidates never selected
  double uout = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; j++)
    if (key[j] != -INFINITY) uout = fmax(uout, S[j] + B[j]);
  uout = wave_max_f64(uout);
  // certify ranks k-1 .. 0 against the running max of later upper bounds
  bool ok = true;
  double umax = uout;
  for (int r = k - 1; r >= 0; r--) {
    const double s_r = readlane_f64(myS, r), b_r = readlane_f64(myB, r);
    const double lo = s_r - b_r;
    const bool rival = umax > -INFINITY;  // none when scope == k and r == k - 1
    const double X = mx_hi - (rival ? fmin(lo, umax) : lo);
    if (!(X < 80.0)) ok = false;
    if (rival && !(lo - umax > f32_4ulps(X) + 0x1p-20)) ok = false;
    umax = fmax(umax, s_r + b_r);
  }
  if (!ok) {
    // for a rescue: the lower bound of the k-th selected candidate
    if (kth_lo) *kth_lo = readlane_f64(myS, k - 1) - readlane_f64(myB, k - 1);
    return false;
  }
  const double smax = mx_hi;  // >= every logit: exp never overflows
  double z = 0.0;
#pragma unroll
  for (int j = 0; j < NJ; j++)
    if (lane + 64 * j < E) z += exp(S[j] - smax);
  z = wave_sum_f64(z);
  const float myp = (float)(exp(myS - smax) / z);
  float wsum = 0.0f;  // moe.go:54-57, rank order
  for (int r = 0; r < k; r++) wsum = wsum + __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(myp), r));
  if (lane < k) {
    const float w = myp / (wsum + 1e-9f);
    if (g_ids) {
      g_ids[lane] = seli;
      g_w[lane] = w;
    }
    if (s_ids) {
      s_ids[lane] = seli;
      s_w[lane] = w;
    }
  }
  return true;
}

template <int NJ>
__device__ __forceinline__ bool certified_select_nj(const double *__restrict__ sb, int E, int k, int scope,
                                                    int32_t *g_ids, float *g_w, int *s_ids, float *s_w,
                                                    int spec_rank = -1, int *spec_slot = nullptr) {
  const int lane = threadIdx.x & 63;
  double S[NJ], B[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int e = lane + 64 * j;
    if (e < E) {
      const double2 v = reinterpret_cast<const double2 *>(sb)[e];
      S[j] = v.x;
      B[j] = v.y;
    } else {
      S[j] = -INFINITY;
      B[j] = 0.0;
    }
  }
  return certified_select_regs<NJ>(S, B, E, k, scope, g_ids, g_w, s_ids, s_w, spec_rank, spec_slot);
}

// Dispatch on the number of expert slots per lane.
#define QMOE_NJ_DISPATCH(E, CALL) \
  do {                            \
    if ((E) <= 64) {              \
      CALL(1);                    \
    } else if ((E) <= 128) {      \
      CALL(2);                    \
    } else if ((E) <= 256) {      \
      CALL(4);                    \
    } else if ((E) <= 512) {      \
      CALL(8);                    \
    } else {                      \
      CALL(16);                   \
    }                             \
  } while (0)


}  // namespace qmoe
