// linear.hip -- qwen-go's dense projection on the device: y = x @ W^T for T
// tokens, W (rows, cols) in f32, bf16 or the group-32 int8/int4 formats, every
// output the reference's sequential f32 sum
//   s = 0; for k in 0..cols-1: s = fl(s + fl(x[k] * w[k]))
// (linear.matvec / matvecRange model/model.go:131-176, matmulVec
// model/tensors.go:77-89, quantLinear.forward model/moe.go:159-162 with
// w = float32(code) * scale), bit for bit.  This is the GEMV the LM head
// (model/model.go:519-525) and the dense MLP projections (model.go:350-358)
// run through.
//
// One lane owns one row, so each output keeps its own accumulator in k order;
// a wave owns a block of 64 rows.  The weights are stored for that: the
// "lane stream" layout.  A row is cut into 16-byte units; unit u of the 64
// rows of block b sits at ((b * units_per_row + u) * 64 + lane) * 16, so one
// wave-wide 16-byte load is 1 KiB of contiguous memory.  For the group-32
// formats every 8 groups of a row (256 elements) form a super-chunk whose
// first unit holds the 8 fp16 scales and whose other units hold the codes
// (16 units int8, 8 units int4), so the scales arrive in the same stream.
// Each lane keeps R super-chunks of loads in flight in registers; x (uniform
// across the wave) is read through scalar loads.  No LDS, no barriers: bound by
// HBM for large row counts, by the load latency of the few waves otherwise.
#include "common.hpp"
#include "kernels.hpp"

namespace qmoe {

constexpr int kLinMaxTok = 8;  // tokens per pass
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Lane-stream geometry of a format (the qmoe_format numbers: f32, bf16,
// int8 / int4 group-32 with fp16 scales, int8 / int4 group-32 with f32
// scales): units per super-chunk (SCU), elements per super-chunk; for the
// group-32 formats the super-chunk's 8 scales come first, in one unit (fp16)
// or two (f32).
template <int LF>
struct LinFmt {
  static constexpr int kBase = LF == kLinI8F32S ? kINT8 : LF == kLinI4F32S ? kINT4 : LF;  // code / element type
  static constexpr int kScaleBytes = (LF == kINT8 || LF == kINT4) ? 2 : (LF == kLinI8F32S || LF == kLinI4F32S) ? 4 : 0;
  static constexpr bool kQuant = kScaleBytes > 0;
  static constexpr int kScaleUnits = kScaleBytes * 8 / 16;
  static constexpr int kCodeUnits = kBase == kINT8 ? 16 : 8;          // 16-byte units of codes / elements
  static constexpr int kUnits = kCodeUnits + kScaleUnits;              // SCU
  static constexpr int kElems = kCodeUnits * Chunk<kBase>::kElems;     // 32 f32, 64 bf16, 256 int8/int4
  static constexpr int kRing = kQuant ? 1 : 2;                         // super-chunks in flight
  // deeper ring for launches of at most one wave per SIMD, where the few waves
  // are bound by the latency of their own loads
  static constexpr int kDeepRing = kBase == kINT8 ? 2 : kBase == kINT4 ? 4 : 6;
};

int linear_step(int fmt) {
  switch (fmt) {
  case kF32: return LinFmt<kF32>::kElems;
  case kBF16: return LinFmt<kBF16>::kElems;
  case kINT8: return LinFmt<kINT8>::kElems;
  case kINT4: return LinFmt<kINT4>::kElems;
  case kLinI8F32S: return LinFmt<kLinI8F32S>::kElems;
  case kLinI4F32S: return LinFmt<kLinI4F32S>::kElems;
  default: return 0;
  }
}

// x of one token sits in LDS: at most kLinMaxLds bytes.
constexpr int kLinMaxLds = 160 * 1024;

bool linear_supported(int fmt, int cols) {
  const int step = linear_step(fmt);
  return step > 0 && cols > 0 && cols % step == 0 && (int64_t)cols * 4 <= kLinMaxLds;
}

int64_t linear_units_per_row(int fmt, int cols) {
  switch (fmt) {
  case kF32: return cols / LinFmt<kF32>::kElems * LinFmt<kF32>::kUnits;
  case kBF16: return cols / LinFmt<kBF16>::kElems * LinFmt<kBF16>::kUnits;
  case kINT8: return cols / LinFmt<kINT8>::kElems * LinFmt<kINT8>::kUnits;
  case kINT4: return cols / LinFmt<kINT4>::kElems * LinFmt<kINT4>::kUnits;
  case kLinI8F32S: return cols / LinFmt<kLinI8F32S>::kElems * LinFmt<kLinI8F32S>::kUnits;
  default: return cols / LinFmt<kLinI4F32S>::kElems * LinFmt<kLinI4F32S>::kUnits;
  }
}

int64_t linear_stream_bytes(int fmt, int rows, int cols) {
  return (int64_t)((rows + 63) / 64) * linear_units_per_row(fmt, cols) * 64 * 16;
}

// The f32 weights of one 16-byte unit of codes / elements (exact: f32, bf16
// widening, or code * scale with the fp16 scale widened exactly).
template <int FMT>
__device__ __forceinline__ void lin_widen(const u32x4 v, float s0, float s1, float (&w)[Chunk<FMT>::kElems]) {
#pragma clang fp contract(off)
  if constexpr (FMT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = __uint_as_float(v[i]);
  } else if constexpr (FMT == kBF16) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w[2 * i] = __uint_as_float(v[i] << 16);
      w[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  } else if constexpr (FMT == kINT8) {
    // 16 elements: half a group, one scale
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int b = 0; b < 4; b++) w[4 * i + b] = (float)(int8_t)((v[i] >> (8 * b)) & 0xffu) * s0;
  } else {
    // 32 elements: one group, hi nibble = the even element
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t byte = (v[i] >> (8 * b)) & 0xffu;
        w[8 * i + 2 * b] = ((float)(byte >> 4) - 8.0f) * s0;
        w[8 * i + 2 * b + 1] = ((float)(byte & 0xfu) - 8.0f) * s0;
      }
  }
  (void)s1;
}

__device__ __forceinline__ float half_of(const u32x4 v, int g) {
  return f16_to_f32((uint16_t)((g & 1) ? (v[g >> 1] >> 16) : (v[g >> 1] & 0xffffu)));
}

// x of one unit for TT tokens: elements [k, k + EPC) of each token row.
template <int FMT, int TT>
struct LinX {
  float v[TT][Chunk<FMT>::kElems];
};

template <int FMT, int TT>
__device__ __forceinline__ void lin_read_x(LinX<FMT, TT> &o, const float *const *xt, int k) {
  constexpr int EPC = Chunk<FMT>::kElems;
#pragma unroll
  for (int t = 0; t < TT; t++)
#pragma unroll
    for (int e = 0; e < EPC; e += 4) {
      const float4 q = *reinterpret_cast<const float4 *>(xt[t] + k + e);
      o.v[t][e] = q.x;
      o.v[t][e + 1] = q.y;
      o.v[t][e + 2] = q.z;
      o.v[t][e + 3] = q.w;
    }
}

// Whether x of the next unit is read one unit ahead (held in registers while
// the current unit computes): for the narrow bf16 / f32 units, whose widening
// is too short to cover the LDS latency.  The int8 / int4 units read their x
// at the start of the unit, behind 16 / 32 widenings.
template <int FMT, int TT>
constexpr bool kLinLookahead = TT * Chunk<FMT>::kElems <= 16;

// One super-chunk c of the ring slot b.  Units are consumed in order; when
// RELOAD each is replaced, as soon as its unit has been summed, by the same
// unit of super-chunk c + R (the scale vector after the last unit).  Reusing
// the register only after the sum keeps each slot in one register across
// iterations: no copies, which would wait for every load in flight.  A
// scheduling barrier closes every unit, so the loads stay in ring order.
template <int LF, int TT, int R, bool RELOAD>
__device__ __forceinline__ void lin_super(u32x4 (&b)[LinFmt<LF>::kUnits], const u32x4 *__restrict__ p, int c,
                                          const float *const *xt, int cols, LinX<LinFmt<LF>::kBase, TT> &xc,
                                          float (&acc)[TT]) {
#pragma clang fp contract(off)
  using F = LinFmt<LF>;
  constexpr int FMT = F::kBase;
  constexpr int SCU = F::kUnits, EPC = Chunk<FMT>::kElems;
  constexpr int U0 = F::kScaleUnits;
  constexpr bool LA = kLinLookahead<FMT, TT>;
  const u32x4 *nx = p + (size_t)((c + R) * SCU) * 64;
#pragma unroll
  for (int u = 0; u < F::kCodeUnits; u++) {
    const int k = c * F::kElems + u * EPC;
    LinX<FMT, TT> xn;
    if constexpr (LA) lin_read_x<FMT, TT>(xn, xt, min(k + EPC, cols - EPC));  // next unit (the last re-reads itself)
    else lin_read_x<FMT, TT>(xc, xt, k);
    float s = 0.0f;
    if constexpr (F::kQuant) {
      const int g = FMT == kINT8 ? u >> 1 : u;  // the unit's group of 32 elements
      if constexpr (F::kScaleBytes == 2) s = half_of(b[0], g);
      else s = __uint_as_float(b[g >> 2][g & 3]);
    }
    u32x4 v = b[U0 + u];
    // int8: opaque here, or the compiler splits the loads into bytes at the
    // load and holds 4x the registers across the ring
    if constexpr (FMT == kINT8) asm volatile("" : "+v"(v));
    float wv[EPC];
    lin_widen<FMT>(v, s, 0.0f, wv);
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
      for (int e = 0; e < EPC; e++) acc[t] = acc[t] + xc.v[t][e] * wv[e];
    if constexpr (RELOAD) b[U0 + u] = __builtin_nontemporal_load(nx + (size_t)(U0 + u) * 64);
    if constexpr (LA) xc = xn;
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (RELOAD) {
#pragma unroll
    for (int q = 0; q < F::kScaleUnits; q++) b[q] = __builtin_nontemporal_load(nx + (size_t)q * 64);
  }
}

template <int LF, int TT, int R>
__global__ void __launch_bounds__(256) linear_stream_kernel(const float *__restrict__ x, int T, int cols,
                                                            const u32x4 *__restrict__ w, int rows,
                                                            float *__restrict__ y) {
#pragma clang fp contract(off)
  using F = LinFmt<LF>;
  constexpr int FMT = F::kBase;
  constexpr int SCU = F::kUnits;
  extern __shared__ __align__(16) float xs[];  // this workgroup's tokens of x, (nt, cols)
  const int t0 = blockIdx.y * TT;
  const int nt = min(TT, T - t0);
  for (int i = threadIdx.x * 4; i < nt * cols; i += blockDim.x * 4)
    *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + (size_t)t0 * cols + i);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int blk = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // 64-row block of this wave
  if (blk * 64 >= rows) return;                                         // whole waves only: no barriers follow
  // rows of x past the last token re-read the last one: their sums are never
  // stored, and the reads stay unconditional
  const float *xt[TT];
#pragma unroll
  for (int t = 0; t < TT; t++) xt[t] = xs + min(t, nt - 1) * cols;
  const int nsc = cols / F::kElems;  // super-chunks per row
  const u32x4 *p = w + (size_t)blk * nsc * SCU * 64 + lane;
  float acc[TT];
#pragma unroll
  for (int t = 0; t < TT; t++) acc[t] = 0.0f;
  // ring of R super-chunks in flight (slot r holds super-chunk c with c % R == r)
  u32x4 buf[R][SCU];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int u = 0; u < SCU; u++) {
      // unconditional, in ring order (a short row re-reads its first super-chunk):
      // the waits in the loop can then count the loads in flight
      buf[r][u] = __builtin_nontemporal_load(p + (size_t)((r < nsc ? r : 0) * SCU + u) * 64);
      __builtin_amdgcn_sched_barrier(0);
    }
  LinX<FMT, TT> xc;
  if constexpr (kLinLookahead<FMT, TT>) lin_read_x<FMT, TT>(xc, xt, 0);
  int c = 0;
  // steady state: every reload is in range, no branches around the loads
#pragma nounroll
  for (; c + 2 * R <= nsc; c += R) {
#pragma unroll
    for (int r = 0; r < R; r++) lin_super<LF, TT, R, true>(buf[r], p, c + r, xt, cols, xc, acc);
  }
  // the last fewer than 2R super-chunks
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (c + r < nsc) {
      if (c + r + R < nsc) lin_super<LF, TT, R, true>(buf[r], p, c + r, xt, cols, xc, acc);
      else lin_super<LF, TT, R, false>(buf[r], p, c + r, xt, cols, xc, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
    if (c + R + r < nsc) lin_super<LF, TT, R, false>(buf[r], p, c + R + r, xt, cols, xc, acc);
  const int row = blk * 64 + lane;
  if (row < rows) {
#pragma unroll
    for (int t = 0; t < TT; t++)
      if (t < nt) y[(size_t)(t0 + t) * rows + row] = acc[t];
  }
}

template <int FMT, int TT, int R = LinFmt<FMT>::kRing>
static hipError_t linear_launch_tt(const float *x, int T, const LinMat &m, float *y, hipStream_t st) {
  const int blocks = (m.rows + 63) / 64;
  // one wave per workgroup when there are few: each gets a CU of its own
  const int wpg = blocks <= m.n_cu ? 1 : 4;
  const dim3 grid((unsigned)((blocks + wpg - 1) / wpg), (unsigned)((T + TT - 1) / TT));
  const size_t lds = (size_t)TT * m.cols * 4;
  if (lds > 64 * 1024) {
    static bool raised = false;  // per instantiation; the limit is the same for every device
    if (!raised) {
      const hipError_t e = hipFuncSetAttribute((const void *)linear_stream_kernel<FMT, TT, R>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLinMaxLds);
      if (e != hipSuccess) return e;
      raised = true;
    }
  }
  QMOE_LAUNCH((linear_stream_kernel<FMT, TT, R>), grid, dim3(64 * wpg), lds, st, x, T, m.cols,
              reinterpret_cast<const u32x4 *>(m.w), m.rows, y);
  return hipGetLastError();
}

// Tokens per pass: up to 8, as many as fit the workgroup's LDS copy of x.
int linear_tokens_per_pass(int T, int cols) {
  int tt = T >= 5 ? 8 : T >= 3 ? 4 : T;
  while (tt > 1 && (size_t)tt * cols * 4 > 64 * 1024) tt /= 2;
  return tt;
}

template <int FMT>
static hipError_t linear_launch_fmt(const float *x, int T, const LinMat &m, float *y, hipStream_t st) {
  const int tt = linear_tokens_per_pass(T, m.cols);
  if (tt == 1 && T == 1 && (m.rows + 63) / 64 <= 4 * m.n_cu)
    return linear_launch_tt<FMT, 1, LinFmt<FMT>::kDeepRing>(x, T, m, y, st);
  switch (tt) {
  case 1: return linear_launch_tt<FMT, 1>(x, T, m, y, st);
  case 2: return linear_launch_tt<FMT, 2>(x, T, m, y, st);
  case 4: return linear_launch_tt<FMT, 4>(x, T, m, y, st);
  default: return linear_launch_tt<FMT, kLinMaxTok>(x, T, m, y, st);
  }
}

hipError_t launch_linear(const float *x, int T, const LinMat &m, float *y, hipStream_t st) {
  if (!linear_supported(m.fmt, m.cols) || T <= 0) return hipErrorInvalidValue;
  const int tt = linear_tokens_per_pass(T, m.cols);
  if ((T + tt - 1) / tt > 65535) return hipErrorInvalidValue;
  switch (m.fmt) {
  case kF32: return linear_launch_fmt<kF32>(x, T, m, y, st);
  case kBF16: return linear_launch_fmt<kBF16>(x, T, m, y, st);
  case kINT8: return linear_launch_fmt<kINT8>(x, T, m, y, st);
  case kINT4: return linear_launch_fmt<kINT4>(x, T, m, y, st);
  case kLinI8F32S: return linear_launch_fmt<kLinI8F32S>(x, T, m, y, st);
  default: return linear_launch_fmt<kLinI4F32S>(x, T, m, y, st);
  }
}

// ---- relayout: row-major (rows, cols) codes / elements (+ their fp16 or f32
// scales, (rows, cols / 32)) into the lane stream.  One thread per (unit,
// lane); rows past the end are zeros.
template <int LF>
__global__ void linear_relayout_kernel(const uint8_t *__restrict__ src, const void *__restrict__ ss, int rows,
                                       int cols, u32x4 *__restrict__ dst, int64_t total) {
  using F = LinFmt<LF>;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i & 63);
  const int64_t unit = i >> 6;  // (blk * nsc + sc) * SCU + u
  const int nsc = cols / F::kElems;
  const int u = (int)(unit % F::kUnits);
  const int64_t bs = unit / F::kUnits;
  const int sc = (int)(bs % nsc);
  const int64_t blk = bs / nsc;
  const int64_t row = blk * 64 + lane;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row < rows) {
    const int64_t row_bytes = fmt_matrix_bytes(F::kBase, 1, cols);
    if (u < F::kScaleUnits) {
      if constexpr (F::kScaleBytes == 2) {
        const uint16_t *sr = static_cast<const uint16_t *>(ss) + row * (cols / kGroup) + sc * 8;
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = (uint32_t)sr[2 * j] | ((uint32_t)sr[2 * j + 1] << 16);
        v = u32x4{h[0], h[1], h[2], h[3]};
      } else if constexpr (F::kScaleBytes == 4) {
        const uint32_t *sr = static_cast<const uint32_t *>(ss) + row * (cols / kGroup) + sc * 8 + u * 4;
        v = u32x4{sr[0], sr[1], sr[2], sr[3]};
      }
    } else {
      const int cu = u - F::kScaleUnits;
      v = *reinterpret_cast<const u32x4 *>(src + row * row_bytes + (int64_t)sc * F::kCodeUnits * 16 + cu * 16);
    }
  }
  dst[i] = v;
}

hipError_t launch_linear_relayout(int fmt, const uint8_t *src, const void *ss, int rows, int cols, void *dst,
                                  hipStream_t st) {
  if (!linear_supported(fmt, cols)) return hipErrorInvalidValue;
  const int64_t total = linear_stream_bytes(fmt, rows, cols) / 16;
  const dim3 grid((unsigned)((total + 255) / 256));
  u32x4 *d = reinterpret_cast<u32x4 *>(dst);
#define RL(LF) hipLaunchKernelGGL(linear_relayout_kernel<LF>, grid, dim3(256), 0, st, src, ss, rows, cols, d, total)
  switch (fmt) {
  case kF32: RL(kF32); break;
  case kBF16: RL(kBF16); break;
  case kINT8: RL(kINT8); break;
  case kINT4: RL(kINT4); break;
  case kLinI8F32S: RL(kLinI8F32S); break;
  default: RL(kLinI4F32S); break;
  }
#undef RL
  return hipGetLastError();
}

// ---- greedy token: argmax over each row of (T, n) logits ----
// model.go:652-660: best = 0; v[i] > v[best] moves it.  So the result is the
// first index of the maximum over the non-NaN entries (ties, including -0 vs
// +0, keep the lower index), 0 when there are none, and 0 whenever v[0] is NaN
// (no comparison against a NaN best succeeds).  Two stages: workgroups reduce
// chunks to (value, index) pairs, one workgroup per row reduces the pairs.
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxChunk = 1024;  // elements per first-stage workgroup (about 150 for a 152k vocabulary)

struct ArgPair {
  float v;
  int i;  // -1: no non-NaN entry seen
};

__device__ __forceinline__ ArgPair arg_better(ArgPair a, ArgPair b) {
  if (b.i < 0) return a;
  if (a.i < 0) return b;
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

__device__ __forceinline__ ArgPair arg_block(ArgPair p) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    ArgPair o;
    o.v = __shfl_down(p.v, off, 64);
    o.i = __shfl_down(p.i, off, 64);
    p = arg_better(p, o);
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wv] = p.v;
    si[wv] = p.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; w++) p = arg_better(p, ArgPair{sv[w], si[w]});
  }
  return p;
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_partial_kernel(const float *__restrict__ v, int n,
                                                                         float *__restrict__ pv,
                                                                         int *__restrict__ pi) {
  const int row = blockIdx.y, nb = gridDim.x;
  const float *r = v + (size_t)row * n;
  const int lo = blockIdx.x * kArgmaxChunk, hi = min(n, lo + kArgmaxChunk);
  ArgPair p{0.0f, -1};
  // each thread scans its elements in increasing index order
  for (int i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
    const float x = r[i];
    if (x == x) p = arg_better(p, ArgPair{x, i});
  }
  p = arg_block(p);
  if (threadIdx.x == 0) {
    pv[(size_t)row * nb + blockIdx.x] = p.v;
    pi[(size_t)row * nb + blockIdx.x] = p.i;
  }
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_final_kernel(const float *__restrict__ v, int n, int nb,
                                                                       const float *__restrict__ pv,
                                                                       const int *__restrict__ pi,
                                                                       int32_t *__restrict__ out) {
  const int row = blockIdx.x;
  ArgPair p{0.0f, -1};
  for (int b = threadIdx.x; b < nb; b += kArgmaxThreads)
    p = arg_better(p, ArgPair{pv[(size_t)row * nb + b], pi[(size_t)row * nb + b]});
  p = arg_block(p);
  if (threadIdx.x == 0) {
    const float v0 = v[(size_t)row * n];
    out[row] = (v0 != v0 || p.i < 0) ? 0 : p.i;
  }
}

int argmax_partials(int n) { return (n + kArgmaxChunk - 1) / kArgmaxChunk; }

hipError_t launch_argmax(const float *v, int T, int n, float *pv, int *pi, int32_t *out, hipStream_t st) {
  if (T <= 0 || n <= 0) return hipErrorInvalidValue;
  const int nb = argmax_partials(n);
  QMOE_LAUNCH(argmax_partial_kernel, dim3(nb, T), dim3(kArgmaxThreads), 0, st, v, n, pv, pi);
  QMOE_LAUNCH(argmax_final_kernel, dim3(T), dim3(kArgmaxThreads), 0, st, v, n, nb, pv, pi, out);
  return hipGetLastError();
}

}  // namespace qmoe
