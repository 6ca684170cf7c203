// prefill.hip -- the MoE block for many tokens: dispatch, grouped expert
// GEMMs on bf16 MFMA, combine.
//
//   prep      x (T, H) f32 -> bf16 (round to nearest even), and the shared
//             expert's scalar gate sg[t] = sigmoid(x[t] . sharedGate)
//             (model/moe.go:89-93).
//   dispatch  one workgroup: per-expert counts of the (token, rank) pairs in an
//             LDS histogram, exclusive prefix scan -> each expert's slot
//             range, then a scatter of every pair into its expert's range
//             (tok[slot], its routing weight, slot_of[t*k + r]).  The shared
//             expert is group E, owning slots [T*k, T*k + T) in token order.
//             Also the tile table: one entry per 128 slots of a group.
//   gate_up   grouped GEMM: per (tile, 64 intermediate columns) a 128 x 128
//             output block = 128 gathered bf16 rows of x times the expert's
//             gate rows [n0, n0+64) and up rows [I+n0, I+n0+64) over K = H,
//             on v_mfma_f32_32x32x16_bf16 with f32 accumulation; SwiGLU in the
//             epilogue (model/moe.go:64-75): act = silu(g) * u, stored bf16.
//   down      grouped GEMM: act rows of the tile times the expert's down
//             matrix over K = I; the routing weight (or shared gate) scales
//             the f32 result, y[slot] = w * (down . act) (model/moe.go:76-84).
//   combine   out[t] = sum over ranks r in rank order of y[slot_of[t, r]],
//             then + y[shared slot of t] (model/moe.go:82-97).
// The slot order inside an expert comes from LDS atomics and may vary from run
// to run; every output row depends only on its own token, so results do not.
//
// Tiles are staged through LDS with global_load_lds (16 bytes per lane) in
// two stages, an XOR swizzle of the 16-byte chunks of each 128-byte row so
// that the MFMA operand reads (one row per lane) hit distinct banks.  The
// down matrices are stored transposed, (I, H), for the decode kernel; their
// tiles are transposed in registers on the way into LDS.
#include "common.hpp"
#include "kernels.hpp"

namespace qmoe {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kBM = 128;        // slots per tile
constexpr int kBK = 64;         // K per stage (128 bytes of bf16 per row)
constexpr int kGemmThreads = 256;
constexpr int kStageBytes = 2 * kBM * kBK * 2;  // A (128 x 64) + B (128 x 64) bf16

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);  // NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// LDS byte offset of the 16-byte chunk c (of 8 k values) of row r in a
// 128-byte-row tile, XOR-swizzled by the row.
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

__device__ __forceinline__ void dma16(const void *src, unsigned char *lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(0), other counters untouched.
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// ------------------------------------------------------------------ prep

__global__ void __launch_bounds__(256) prep_kernel(const float *__restrict__ x, int H,
                                                  const float *__restrict__ shared_gate,
                                                  uint16_t *__restrict__ xb, float *__restrict__ sg) {
  const int t = blockIdx.x;
  const float *xr = x + (size_t)t * H;
  uint16_t *xo = xb + (size_t)t * H;
  float dot = 0.0f;
  for (int h = threadIdx.x * 4; h < H; h += 1024) {
    const float4 v = *reinterpret_cast<const float4 *>(xr + h);
    uint2 p;
    p.x = (uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16);
    p.y = (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16);
    *reinterpret_cast<uint2 *>(xo + h) = p;
    if (shared_gate) {
      const float4 g = *reinterpret_cast<const float4 *>(shared_gate + h);
      dot += v.x * g.x + v.y * g.y + v.z * g.z + v.w * g.w;
    }
  }
  if (!shared_gate) return;
  __shared__ float part[4];
  dot = group_sum(dot, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = dot;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float s = part[0] + part[1] + part[2] + part[3];
    sg[t] = 1.0f / (1.0f + (float)exp(-(double)s));  // sigmoid1, model/tensors.go:97
  }
}

// -------------------------------------------------------------- dispatch

constexpr int kDispatchThreads = 1024;

__global__ void __launch_bounds__(kDispatchThreads)
    dispatch_kernel(const int32_t *__restrict__ ids, const float *__restrict__ wts, const float *__restrict__ sg,
                    int T, int k, int E, int with_shared, PrefillPlan p) {
  __shared__ int cnt[1024], incl[1024], tincl[1024], cur[1024];
  const int tid = threadIdx.x;
  const int n = T * k;
  cnt[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += kDispatchThreads) atomicAdd(&cnt[ids[i]], 1);
  __syncthreads();
  // inclusive scans of the counts and of the tiles per expert (E <= 1024)
  const int c = tid < E ? cnt[tid] : 0;
  const int ct = (c + kBM - 1) / kBM;
  incl[tid] = c;
  tincl[tid] = ct;
  __syncthreads();
  for (int d = 1; d < kDispatchThreads; d <<= 1) {
    const int a = tid >= d ? incl[tid - d] : 0;
    const int b = tid >= d ? tincl[tid - d] : 0;
    __syncthreads();
    incl[tid] += a;
    tincl[tid] += b;
    __syncthreads();
  }
  const int off = incl[tid] - c, toff = tincl[tid] - ct;
  const int routed_tiles = tincl[kDispatchThreads - 1];
  if (tid < E) {
    p.grp_off[tid] = off;
    p.grp_cnt[tid] = c;
    cur[tid] = off;
    for (int q = 0; q < ct; q++) {
      p.tile_grp[toff + q] = tid;
      p.tile_m0[toff + q] = q * kBM;
    }
  }
  const int shared_tiles = with_shared ? (T + kBM - 1) / kBM : 0;
  for (int q = tid; q < shared_tiles; q += kDispatchThreads) {
    p.tile_grp[routed_tiles + q] = E;
    p.tile_m0[routed_tiles + q] = q * kBM;
  }
  if (tid == 0) {
    p.n_tiles[0] = routed_tiles;
    p.n_tiles[1] = shared_tiles;
    p.grp_off[E] = n;
    p.grp_cnt[E] = with_shared ? T : 0;
  }
  __syncthreads();
  for (int i = tid; i < n; i += kDispatchThreads) {
    const int slot = atomicAdd(&cur[ids[i]], 1);
    p.tok[slot] = i / k;
    p.wslot[slot] = wts[i];
    p.slot_of[i] = slot;
  }
  if (with_shared)
    for (int t = tid; t < T; t += kDispatchThreads) {
      p.tok[n + t] = t;
      p.wslot[n + t] = sg[t];
    }
}

// ------------------------------------------------------------ tile setup

struct TileInfo {
  int g, slot0, rows;
  bool ok;
};

__device__ __forceinline__ TileInfo tile_of(const PrefillPlan &p, int E, bool shared_launch) {
  TileInfo ti{0, 0, 0, false};
  const int nt = shared_launch ? p.n_tiles[1] : p.n_tiles[0];
  if ((int)blockIdx.x >= nt) return ti;
  const int idx = shared_launch ? p.n_tiles[0] + blockIdx.x : blockIdx.x;
  ti.g = p.tile_grp[idx];
  const int m0 = p.tile_m0[idx];
  ti.slot0 = p.grp_off[ti.g] + m0;
  ti.rows = min(kBM, p.grp_cnt[ti.g] - m0);
  ti.ok = ti.g <= E && ti.rows > 0;
  return ti;
}

// --------------------------------------------------------------- gate_up

// Output block 128 slots x (64 gate + 64 up) columns.  Wave w: slots
// [64 (w & 1), +64), gate/up columns [32 (w >> 1), +32) -- the gate and up
// accumulators of a lane hold the same (slot, column), so SwiGLU is local.
__global__ void __launch_bounds__(kGemmThreads) gemm_gate_up_bf16(PrefillArgs a, int shared_launch) {
  const TileInfo ti = tile_of(a.p, a.E, shared_launch);
  if (!ti.ok) return;
  const bool sh = ti.g == a.E;
  const int N = sh ? a.Is : a.I;
  const int n0 = blockIdx.y * 64;
  if (n0 >= N) return;
  const int H = a.H;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;

  // rows this thread stages: A rows / B rows ((i * 4 + w) * 8 + lane / 8)
  const uint16_t *arow[4], *brow[4];
  const uint8_t *gbase = sh ? a.sgate : a.gu + (size_t)ti.g * a.gu_bytes;
  const uint8_t *ubase = sh ? a.sup : gbase + (size_t)a.I * H * 2;
  int chunk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = (i * 4 + w) * 8 + (lane >> 3);
    chunk[i] = (lane & 7) ^ (r & 7);
    const int m = min(r, ti.rows - 1);
    arow[i] = a.xb + (size_t)a.p.tok[ti.slot0 + m] * H;
    brow[i] = reinterpret_cast<const uint16_t *>(r < 64 ? gbase + (size_t)(n0 + r) * H * 2
                                                        : ubase + (size_t)(n0 + r - 64) * H * 2);
  }
  auto issue = [&](int stage, int k0) {
    unsigned char *sa = lds + stage * kStageBytes, *sb = sa + kBM * 128;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      dma16(arow[i] + k0 + chunk[i] * 8, sa + (i * 4 + w) * 1024);
      dma16(brow[i] + k0 + chunk[i] * 8, sb + (i * 4 + w) * 1024);
    }
  };

  const int wm = w & 1, wn = w >> 1;
  f32x16_t acc[2][2];  // [m block][gate, up]
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[b][q][e] = 0.0f;

  const int KT = H / kBK;
  issue(0, 0);
  const int ar0 = wm * 64 + (lane & 31), br0 = wn * 32 + (lane & 31), hi = lane >> 5;
  for (int kt = 0; kt < KT; kt++) {
    wait_vm0();
    __syncthreads();  // stage kt landed everywhere; stage kt + 1 is free
    const unsigned char *sa = lds + (kt & 1) * kStageBytes, *sb = sa + kBM * 128;
    bf16x8_t av[2][4], bv[2][4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const int c = ks * 2 + hi;
#pragma unroll
      for (int b = 0; b < 2; b++) av[b][ks] = *reinterpret_cast<const bf16x8_t *>(sa + swz(ar0 + 32 * b, c));
      bv[0][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(br0, c));
      bv[1][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(64 + br0, c));
    }
    if (kt + 1 < KT) issue((kt + 1) & 1, (kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int q = 0; q < 2; q++)
          acc[b][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b][ks], bv[q][ks], acc[b][q], 0, 0, 0);
  }
  // epilogue: act = silu(g) * u -> bf16, row pitch Imax
  const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = wm * 64 + b * 32 + 8 * j + 4 * hi + i;
        if (m < ti.rows) {
          const float g = acc[b][0][4 * j + i], u = acc[b][1][4 * j + i];
          const float s = g / (1.0f + __expf(-g));
          a.act[(size_t)(ti.slot0 + m) * a.Imax + n] = f32_to_bf16_rne(s * u);
        }
      }
}

// ------------------------------------------------------------------ down

// Output block 128 slots x 128 hidden columns.  Wave w: slots
// [64 (w & 1), +64), columns [64 (w >> 1), +64).  The down matrix is stored
// (I, H), N-contiguous: each thread loads 4 K rows x 8 columns (4 x 16 bytes),
// transposes them in registers and writes 8 column-rows of 4 K values.
__global__ void __launch_bounds__(kGemmThreads) gemm_down_bf16(PrefillArgs a, int shared_launch) {
  const TileInfo ti = tile_of(a.p, a.E, shared_launch);
  if (!ti.ok) return;
  const bool sh = ti.g == a.E;
  const int K = sh ? a.Is : a.I;
  const int H = a.H;
  const int n0 = blockIdx.y * 128;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;

  const uint16_t *arow[4];
  int chunk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = (i * 4 + w) * 8 + (lane >> 3);
    chunk[i] = (lane & 7) ^ (r & 7);
    arow[i] = a.act + (size_t)(ti.slot0 + min(r, ti.rows - 1)) * a.Imax;
  }
  const uint16_t *dbase = reinterpret_cast<const uint16_t *>(sh ? a.sdown : a.dn + (size_t)ti.g * a.dn_bytes);
  const int kq = tid >> 4, nc = tid & 15;  // this thread's 4 K rows and 8 columns of the B tile
  const uint16_t *bsrc = dbase + (size_t)(4 * kq) * H + n0 + 8 * nc;
  uint4 breg[4];
  auto load_b = [&](int k0) {
#pragma unroll
    for (int r = 0; r < 4; r++) breg[r] = *reinterpret_cast<const uint4 *>(bsrc + (size_t)(k0 + r) * H);
  };
  auto store_b = [&](int stage) {
    unsigned char *sb = lds + stage * kStageBytes + kBM * 128;
    const uint32_t in[4][4] = {{breg[0].x, breg[0].y, breg[0].z, breg[0].w},
                               {breg[1].x, breg[1].y, breg[1].z, breg[1].w},
                               {breg[2].x, breg[2].y, breg[2].z, breg[2].w},
                               {breg[3].x, breg[3].y, breg[3].z, breg[3].w}};
#pragma unroll
    for (int d = 0; d < 4; d++) {
      // columns 2d (low halves) and 2d + 1 (high halves) of the 4 K rows
      const uint32_t lo01 = __builtin_amdgcn_perm(in[1][d], in[0][d], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(in[3][d], in[2][d], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(in[1][d], in[0][d], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(in[3][d], in[2][d], 0x07060302u);
      const int r0 = 8 * nc + 2 * d, r1 = r0 + 1;
      *reinterpret_cast<uint2 *>(sb + swz(r0, kq >> 1) + (kq & 1) * 8) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2 *>(sb + swz(r1, kq >> 1) + (kq & 1) * 8) = make_uint2(hi01, hi23);
    }
  };
  auto issue_a = [&](int stage, int k0) {
    unsigned char *sa = lds + stage * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(arow[i] + k0 + chunk[i] * 8, sa + (i * 4 + w) * 1024);
  };

  const int wm = w & 1, wn = w >> 1;
  f32x16_t acc[2][2];  // [m block][n block]
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[b][q][e] = 0.0f;

  const int KT = K / kBK;
  issue_a(0, 0);
  load_b(0);
  wait_vm0();
  store_b(0);
  const int ar0 = wm * 64 + (lane & 31), br0 = wn * 64 + (lane & 31), hi = lane >> 5;
  for (int kt = 0; kt < KT; kt++) {
    __syncthreads();  // stage kt complete (A by DMA, B by stores); stage kt + 1 free
    const unsigned char *sa = lds + (kt & 1) * kStageBytes, *sb = sa + kBM * 128;
    bf16x8_t av[2][4], bv[2][4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const int c = ks * 2 + hi;
#pragma unroll
      for (int b = 0; b < 2; b++) {
        av[b][ks] = *reinterpret_cast<const bf16x8_t *>(sa + swz(ar0 + 32 * b, c));
        bv[b][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(br0 + 32 * b, c));
      }
    }
    if (kt + 1 < KT) {
      issue_a((kt + 1) & 1, (kt + 1) * kBK);
      load_b((kt + 1) * kBK);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int q = 0; q < 2; q++)
          acc[b][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b][ks], bv[q][ks], acc[b][q], 0, 0, 0);
    if (kt + 1 < KT) {
      wait_vm0();
      store_b((kt + 1) & 1);
    }
  }
  // epilogue: y[slot] = w_slot * acc, f32
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = wm * 64 + b * 32 + 8 * j + 4 * hi + i;
        if (m < ti.rows) {
          const int slot = ti.slot0 + m;
          const float ws = a.p.wslot[slot];
#pragma unroll
          for (int q = 0; q < 2; q++) {
            const int n = n0 + wn * 64 + q * 32 + (lane & 31);
            a.y[(size_t)slot * H + n] = ws * acc[b][q][4 * j + i];
          }
        }
      }
}

// --------------------------------------------------------------- combine

__global__ void __launch_bounds__(256) combine_kernel(const float *__restrict__ y, const int32_t *__restrict__ slot_of,
                                                      int T, int k, int H, int with_shared,
                                                      float *__restrict__ out) {
  const int t = blockIdx.x;
  for (int j = threadIdx.x * 4; j < H; j += 1024) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r = 0; r < k; r++) {  // rank order, model/moe.go:82-84
      const float4 v = *reinterpret_cast<const float4 *>(y + (size_t)slot_of[(size_t)t * k + r] * H + j);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    if (with_shared) {  // added after the routed sum, model/moe.go:94-96
      const float4 v = *reinterpret_cast<const float4 *>(y + ((size_t)T * k + t) * H + j);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    *reinterpret_cast<float4 *>(out + (size_t)t * H + j) = acc;
  }
}

// ------------------------------------------------------------- launchers

bool prefill_supported(int expert_fmt, int shared_fmt, int H, int I, int Is) {
  // bf16 experts; the shared expert (if any) in the same format
  if (expert_fmt != kBF16) return false;
  if (Is > 0 && shared_fmt != kBF16) return false;
  return H % 128 == 0 && I % 64 == 0 && (Is == 0 || Is % 64 == 0);
}

int prefill_max_tiles(int T, int k, int E) {
  const int n = T * k;
  return (n + kBM - 1) / kBM + (E < n ? E : n);
}

hipError_t launch_prefill_dispatch(const PrefillArgs &a, const int32_t *ids, const float *wts, const float *x,
                                   const float *shared_gate, float *sg, hipStream_t st) {
  const bool with_shared = a.Is > 0;
  hipLaunchKernelGGL(prep_kernel, dim3(a.T), dim3(256), 0, st, x, a.H, with_shared ? shared_gate : nullptr, a.xb,
                     sg);
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, st, ids, wts, sg, a.T, a.k, a.E,
                     (int)with_shared, a.p);
  return hipGetLastError();
}

hipError_t launch_prefill_gate_up(const PrefillArgs &a, bool shared, hipStream_t st) {
  const int tiles = shared ? (a.T + kBM - 1) / kBM : prefill_max_tiles(a.T, a.k, a.E);
  const int ny = (shared ? a.Is : a.I) / 64;
  hipLaunchKernelGGL(gemm_gate_up_bf16, dim3(tiles, ny), dim3(kGemmThreads), 2 * kStageBytes, st, a, (int)shared);
  return hipGetLastError();
}

hipError_t launch_prefill_down(const PrefillArgs &a, bool shared, hipStream_t st) {
  const int tiles = shared ? (a.T + kBM - 1) / kBM : prefill_max_tiles(a.T, a.k, a.E);
  hipLaunchKernelGGL(gemm_down_bf16, dim3(tiles, a.H / 128), dim3(kGemmThreads), 2 * kStageBytes, st, a,
                     (int)shared);
  return hipGetLastError();
}

hipError_t launch_prefill_combine(const PrefillArgs &a, float *out, hipStream_t st) {
  hipLaunchKernelGGL(combine_kernel, dim3(a.T), dim3(256), 0, st, a.y, a.p.slot_of, a.T, a.k, a.H,
                     (int)(a.Is > 0), out);
  return hipGetLastError();
}

}  // namespace qmoe
