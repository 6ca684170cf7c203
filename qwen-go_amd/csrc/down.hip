// down.hip -- expert down GEMV with the rank-ordered weighted combine and the
// gated shared expert (bandwidth-bound, decode-sized T).  See gate_up.hip for
// the load scheme.
#include "gemv_common.hpp"

namespace qmoe {

// ------------------------------------------------------------------ down

// Block (chunk of kDownRows output rows, token t).  Items are (row, rank)
// pairs, rank k being the shared expert; lane groups compute two items at a
// time with all their loads in flight, write w * dot into LDS, and the block
// then sums each row's items in rank order (shared expert last), as
// model/moe.go:82-84 and :94-96 accumulate.  No cross-block communication.
template <int EFMT, int EITER, int SFMT, bool SAME>
__global__ void __launch_bounds__(kBlock) down_kernel(DownArgs a) {
  constexpr int SITER = SAME ? EITER : 0;
  extern __shared__ __align__(16) float as[];  // ranks x Kmax activations, then parts
  const int t = blockIdx.y, chunk = blockIdx.x;
  const int H = a.H, k = a.k, I = a.I, Is = a.Is;
  const int ranks = k + (Is ? 1 : 0);
  const int Kmax = max(I, Is);
  float *part = as + (size_t)ranks * Kmax;  // [rank][row]
  for (int i = threadIdx.x * 4; i < k * I; i += kBlock * 4) {
    const int rr = i / I, c = i % I;
    *reinterpret_cast<float4 *>(as + rr * Kmax + c) =
        *reinterpret_cast<const float4 *>(a.act + (size_t)t * k * I + i);
  }
  for (int i = threadIdx.x * 4; i < Is; i += kBlock * 4)
    *reinterpret_cast<float4 *>(as + k * Kmax + i) = *reinterpret_cast<const float4 *>(a.act_s + (size_t)t * Is + i);
  __syncthreads();
  const int j0 = chunk * kDownRows;
  const int nrows = min(kDownRows, H - j0);
  const int items = nrows * ranks;

  // routed experts: one lane-group layout for format EFMT
  {
    constexpr int EPC = Chunk<EFMT>::kElems;
    const int nch = I / EPC;
    const int lpr = lanes_per_row(nch);
    const int groups = kBlock / lpr;
    const int g = threadIdx.x / lpr, sl = threadIdx.x % lpr;
    const int64_t row_bytes = fmt_matrix_bytes(EFMT, 1, I);
    const int nsc = I / kGroup;
    const int nitems = nrows * k;
    for (int i0 = g; i0 < nitems; i0 += 2 * groups) {
      const int i1 = min(i0 + groups, nitems - 1);
      const int r0 = i0 / nrows, q0 = i0 % nrows, r1 = i1 / nrows, q1 = i1 % nrows;
      const int e0 = a.ids[(size_t)t * k + r0], e1 = a.ids[(size_t)t * k + r1];
      const uint8_t *b0 = a.down + (size_t)e0 * a.expert_bytes + (size_t)(j0 + q0) * row_bytes;
      const uint8_t *b1 = a.down + (size_t)e1 * a.expert_bytes + (size_t)(j0 + q1) * row_bytes;
      const uint16_t *s0 = nullptr, *s1 = nullptr;
      if constexpr (fmt_quant(EFMT)) {
        s0 = a.down_s + (size_t)e0 * a.expert_scales + (size_t)(j0 + q0) * nsc;
        s1 = a.down_s + (size_t)e1 * a.expert_scales + (size_t)(j0 + q1) * nsc;
      }
      float d0 = row_dot_any<EFMT, EITER>(b0, s0, as + r0 * Kmax, sl, lpr, nch);
      float d1 = row_dot_any<EFMT, EITER>(b1, s1, as + r1 * Kmax, sl, lpr, nch);
      d0 = group_sum(d0, lpr);
      d1 = group_sum(d1, lpr);
      if (sl == 0) {
        part[r0 * kDownRows + q0] = a.weights[(size_t)t * k + r0] * d0;
        if (i0 + groups < nitems) part[r1 * kDownRows + q1] = a.weights[(size_t)t * k + r1] * d1;
      }
    }
  }
  // shared expert rows
  if (Is) {
    constexpr int EPC = Chunk<SFMT>::kElems;
    const int nch = Is / EPC;
    const int lpr = lanes_per_row(nch);
    const int groups = kBlock / lpr;
    const int g = threadIdx.x / lpr, sl = threadIdx.x % lpr;
    const int64_t row_bytes = fmt_matrix_bytes(SFMT, 1, Is);
    const int nsc = Is / kGroup;
    for (int q = g; q < nrows; q += groups) {
      const uint8_t *b = a.sdown + (size_t)(j0 + q) * row_bytes;
      const uint16_t *sp = fmt_quant(SFMT) ? a.sdown_s + (size_t)(j0 + q) * nsc : nullptr;
      float d = row_dot_any<SFMT, SITER>(b, sp, as + k * Kmax, sl, lpr, nch);
      d = group_sum(d, lpr);
      if (sl == 0) part[k * kDownRows + q] = a.sg[t] * d;
    }
  }
  __syncthreads();
  (void)items;
  for (int q = threadIdx.x; q < nrows; q += kBlock) {
    float acc = 0.0f;
    for (int rr = 0; rr < ranks; rr++) acc += part[rr * kDownRows + q];
    a.out[(size_t)t * H + j0 + q] = acc;
  }
}

template <int EFMT, int EITER, int SFMT, bool SAME>
static void down_launch(const DownArgs &a, hipStream_t st) {
  const int chunks = (a.H + kDownRows - 1) / kDownRows;
  dim3 grid(chunks, a.T);
  const int ranks = a.k + (a.Is ? 1 : 0);
  const size_t lds = ((size_t)ranks * max(a.I, a.Is) + (size_t)ranks * kDownRows) * sizeof(float);
  hipLaunchKernelGGL((down_kernel<EFMT, EITER, SFMT, SAME>), grid, dim3(kBlock), lds, st, a);
}

template <int EFMT, int EITER>
static void down_sf(const DownArgs &a, hipStream_t st) {
  const int sf = a.Is ? a.sfmt : EFMT;
  if (sf == EFMT && (a.Is == 0 || a.Is == a.I)) {
    down_launch<EFMT, EITER, EFMT, true>(a, st);
    return;
  }
  switch (sf) {
  case kF32: down_launch<EFMT, EITER, kF32, false>(a, st); break;
  case kBF16: down_launch<EFMT, EITER, kBF16, false>(a, st); break;
  case kINT8: down_launch<EFMT, EITER, kINT8, false>(a, st); break;
  default: down_launch<EFMT, EITER, kINT4, false>(a, st); break;
  }
}

template <int EFMT>
static void down_e(const DownArgs &a, hipStream_t st) {
  switch (iter_of(EFMT, a.I)) {
#define C(F, I) case I: down_sf<EFMT, I>(a, st); break;
    QMOE_ITER_CASES(EFMT, C)
#undef C
  default: down_sf<EFMT, 0>(a, st); break;
  }
}

hipError_t launch_down_gemv(const DownArgs &a, hipStream_t st) {
  switch (a.fmt) {
  case kF32: down_e<kF32>(a, st); break;
  case kBF16: down_e<kBF16>(a, st); break;
  case kINT8: down_e<kINT8>(a, st); break;
  default: down_e<kINT4>(a, st); break;
  }
  return hipGetLastError();
}


}  // namespace qmoe
