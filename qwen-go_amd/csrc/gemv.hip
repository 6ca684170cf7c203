// gemv.hip -- bandwidth-bound expert GEMVs for decode-sized T on gfx950.
//
// Each weight row is streamed from HBM once per (token, rank) with 16-byte
// per-lane loads along K (coalesced: a group of `lpr` lanes covers 16*lpr
// contiguous bytes of the row), widened / dequantised in registers, and dotted
// with the token's f32 activations held in LDS.  Accumulation is f32 FMA; the
// reference sums sequentially, so these outputs match it within f32 rounding
// (the tolerance path), not bit for bit.
//
// gate_up (model/moe.go:64-75): one lane group computes gate row o and up row o
//   of one expert and writes silu(g) * u -- the SwiGLU is fused.
// down + combine (model/moe.go:76-97): one lane group computes output row j of
//   one token over its k routed experts in rank order, scaled by the routing
//   weights, then adds sigmoid(gate . x) * shared_down[j] . act_s.  No atomics:
//   every output element is written once, deterministically.
#include "common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace qmoe {

constexpr int kBlock = 256;

// Largest power of two <= 64 that divides n (lanes per row).
__host__ __device__ inline int lanes_per_row(int n) {
  int l = 64;
  while (l > 1 && (n % l) != 0) l >>= 1;
  return l;
}

// Dot of `nch` 16-byte chunks of a stored row with f32 activations in LDS,
// this lane taking chunks sl, sl+lpr, ...; returns the lane's partial sum.
template <int FMT>
__device__ __forceinline__ float row_dot(const uint8_t *__restrict__ row, const uint16_t *__restrict__ srow,
                                         const float *__restrict__ xs, int nch, int sl, int lpr) {
  constexpr int EPC = Chunk<FMT>::kElems;
  float acc = 0.0f;
  for (int c = sl; c < nch; c += lpr) {
    float w[EPC];
    float sc;
    load_chunk<FMT>(row, srow, c, w, sc);
    const float4 *xv = reinterpret_cast<const float4 *>(xs + c * EPC);
    float part = 0.0f;
#pragma unroll
    for (int q = 0; q < EPC / 4; q++) {
      float4 xx = xv[q];
      part = fmaf(w[4 * q + 0], xx.x, part);
      part = fmaf(w[4 * q + 1], xx.y, part);
      part = fmaf(w[4 * q + 2], xx.z, part);
      part = fmaf(w[4 * q + 3], xx.w, part);
    }
    if constexpr (fmt_quant(FMT)) acc = fmaf(part, sc, acc);
    else acc += part;
  }
  return acc;
}

__device__ __forceinline__ float silu_ref(float g) {
  // silu, model/tensors.go:91-95
  return g / (1.0f + (float)exp(-(double)g));
}

template <int FMT>
__global__ void __launch_bounds__(kBlock) gate_up_gemv_kernel(GateUpArgs a, int rows_per_block) {
  extern __shared__ __align__(16) float xs[];
  const int p = blockIdx.y;
  const int t = p / a.k;
  const int e = a.ids ? a.ids[p] : 0;
  const int H = a.H, I = a.I;
  for (int i = threadIdx.x * 4; i < H; i += kBlock * 4)
    *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(a.x + (size_t)t * H + i);
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (a.shared_gate && blockIdx.x == 0 && wave == 0) {
    // shared-expert gate, model/moe.go:89-93
    float g = 0.0f;
    for (int i = lane; i < H; i += 64) g = fmaf(xs[i], a.shared_gate[i], g);
    g = group_sum(g, 64);
    if (lane == 0) a.sg[t] = 1.0f / (1.0f + (float)exp(-(double)g));
  }

  constexpr int EPC = Chunk<FMT>::kElems;
  const int nch = H / EPC;
  const int lpr = lanes_per_row(nch);
  const int per_wave = 64 / lpr;
  const int sub = lane / lpr, sl = lane % lpr;
  const int64_t row_bytes = fmt_matrix_bytes(FMT, 1, H);
  const int nsc = H / kGroup;
  const uint8_t *gbase = a.gate + (size_t)e * a.expert_bytes;
  const uint8_t *ubase = a.up + (size_t)e * a.expert_bytes;
  const uint16_t *gsb = fmt_quant(FMT) ? a.gate_s + (size_t)e * a.expert_scales : nullptr;
  const uint16_t *usb = fmt_quant(FMT) ? a.up_s + (size_t)e * a.expert_scales : nullptr;
  const int o_begin = blockIdx.x * rows_per_block;
  const int o_end = min(o_begin + rows_per_block, I);
  for (int o = o_begin + wave * per_wave + sub; o < o_end; o += (kBlock / 64) * per_wave) {
    float g = row_dot<FMT>(gbase + (size_t)o * row_bytes, gsb ? gsb + (size_t)o * nsc : nullptr, xs,
                           nch, sl, lpr);
    float u = row_dot<FMT>(ubase + (size_t)o * row_bytes, usb ? usb + (size_t)o * nsc : nullptr, xs,
                           nch, sl, lpr);
    g = group_sum(g, lpr);
    u = group_sum(u, lpr);
    if (sl == 0) a.act[(size_t)p * I + o] = silu_ref(g) * u;
  }
}

template <int FMT>
static hipError_t gate_up_fmt(const GateUpArgs &a, hipStream_t st) {
  constexpr int EPC = Chunk<FMT>::kElems;
  const int lpr = lanes_per_row(a.H / EPC);
  const int rows_per_block = (kBlock / 64) * (64 / lpr);
  dim3 grid((a.I + rows_per_block - 1) / rows_per_block, a.T * a.k);
  hipLaunchKernelGGL(gate_up_gemv_kernel<FMT>, grid, dim3(kBlock), (size_t)a.H * sizeof(float), st, a,
                     rows_per_block);
  return hipGetLastError();
}

hipError_t launch_gate_up_gemv(const GateUpArgs &a, hipStream_t st) {
  switch (a.fmt) {
  case kF32: return gate_up_fmt<kF32>(a, st);
  case kBF16: return gate_up_fmt<kBF16>(a, st);
  case kINT8: return gate_up_fmt<kINT8>(a, st);
  default: return gate_up_fmt<kINT4>(a, st);
  }
}

template <int EFMT, int SFMT>
__global__ void __launch_bounds__(kBlock) down_gemv_kernel(DownArgs a, int rows_per_block) {
  extern __shared__ __align__(16) float as[];
  const int t = blockIdx.y;
  const int H = a.H, I = a.I, k = a.k, Is = a.Is;
  for (int i = threadIdx.x * 4; i < k * I; i += kBlock * 4)
    *reinterpret_cast<float4 *>(as + i) = *reinterpret_cast<const float4 *>(a.act + (size_t)t * k * I + i);
  for (int i = threadIdx.x * 4; i < Is; i += kBlock * 4)
    *reinterpret_cast<float4 *>(as + k * I + i) = *reinterpret_cast<const float4 *>(a.act_s + (size_t)t * Is + i);
  __syncthreads();

  constexpr int EPC = Chunk<EFMT>::kElems;
  constexpr int SEPC = Chunk<SFMT>::kElems;
  const int nch = I / EPC;
  const int snch = Is / SEPC;
  const int lpr = lanes_per_row(nch);
  const int per_wave = 64 / lpr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / lpr, sl = lane % lpr;
  const int64_t row_bytes = fmt_matrix_bytes(EFMT, 1, I);
  const int nsc = I / kGroup;
  const int64_t srow_bytes = fmt_matrix_bytes(SFMT, 1, Is);
  const int snsc = Is / kGroup;
  const int j_begin = blockIdx.x * rows_per_block;
  const int j_end = min(j_begin + rows_per_block, H);
  for (int j = j_begin + wave * per_wave + sub; j < j_end; j += (kBlock / 64) * per_wave) {
    float acc = 0.0f;
    for (int r = 0; r < k; r++) {
      const int e = a.ids[(size_t)t * k + r];
      const float wr = a.weights[(size_t)t * k + r];
      const uint8_t *row = a.down + (size_t)e * a.expert_bytes + (size_t)j * row_bytes;
      const uint16_t *srow =
          fmt_quant(EFMT) ? a.down_s + (size_t)e * a.expert_scales + (size_t)j * nsc : nullptr;
      float d = row_dot<EFMT>(row, srow, as + r * I, nch, sl, lpr);
      d = group_sum(d, lpr);
      acc = fmaf(wr, d, acc);
    }
    if (Is > 0) {
      const uint8_t *row = a.sdown + (size_t)j * srow_bytes;
      const uint16_t *srow = fmt_quant(SFMT) ? a.sdown_s + (size_t)j * snsc : nullptr;
      float d = row_dot<SFMT>(row, srow, as + k * I, snch, sl, lpr);
      d = group_sum(d, lpr);
      acc = fmaf(a.sg[t], d, acc);
    }
    if (sl == 0) a.out[(size_t)t * H + j] = acc;
  }
}

template <int EFMT, int SFMT>
static hipError_t down_fmt2(const DownArgs &a, hipStream_t st) {
  constexpr int EPC = Chunk<EFMT>::kElems;
  const int lpr = lanes_per_row(a.I / EPC);
  const int rows_per_block = (kBlock / 64) * (64 / lpr);
  dim3 grid((a.H + rows_per_block - 1) / rows_per_block, a.T);
  size_t lds = (size_t)(a.k * a.I + a.Is) * sizeof(float);
  hipLaunchKernelGGL((down_gemv_kernel<EFMT, SFMT>), grid, dim3(kBlock), lds, st, a, rows_per_block);
  return hipGetLastError();
}

template <int EFMT>
static hipError_t down_fmt(const DownArgs &a, hipStream_t st) {
  switch (a.Is > 0 ? a.sfmt : EFMT) {
  case kF32: return down_fmt2<EFMT, kF32>(a, st);
  case kBF16: return down_fmt2<EFMT, kBF16>(a, st);
  case kINT8: return down_fmt2<EFMT, kINT8>(a, st);
  default: return down_fmt2<EFMT, kINT4>(a, st);
  }
}

hipError_t launch_down_gemv(const DownArgs &a, hipStream_t st) {
  switch (a.fmt) {
  case kF32: return down_fmt<kF32>(a, st);
  case kBF16: return down_fmt<kBF16>(a, st);
  case kINT8: return down_fmt<kINT8>(a, st);
  default: return down_fmt<kINT4>(a, st);
  }
}

}  // namespace qmoe
