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
//             Also the tile table: one entry per 256 slots of a group.
//   gate_up   grouped GEMM: per (tile, 64 intermediate columns) a 256 x 128
//             output block = 256 gathered bf16 rows of x times the expert's
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
// Expert weights are bf16, or int8 / int4 group-32 codes with fp16 scales
// that the GEMMs dequantise to bf16 in LDS on the way to the MFMAs.  Tiles are
// staged through LDS with global_load_lds (16 bytes per lane) in a ring of
// three stages, an XOR swizzle of the 16-byte chunks of each 128-byte row so
// that the MFMA operand reads (one row per lane) hit distinct banks.  The
// down matrices are stored transposed, (I, H), for the decode kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace qmoe {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kBM = 256;        // slots per tile
constexpr int kBK = 64;         // K per stage (128 bytes of bf16 per row)
constexpr int kGemmThreads = 512;

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);  // NaN
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// LDS byte offset of the 16-byte chunk c (of 8 k values) of row r in a
// 128-byte-row tile, XOR-swizzled by the row.  The LDS has 64 banks (256
// bytes) and serves a 16-byte-per-lane read 16 lanes at a time; those lanes
// read 16 consecutive rows at one logical chunk, and (r >> 1) & 7 spreads each
// pair of rows sharing a 256-byte bank line over distinct chunks.
__device__ __forceinline__ int swz_of(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ swz_of(r)) << 4); }

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

__device__ __forceinline__ TileInfo tile_of(const PrefillPlan &p, int E, bool shared_launch, int tile) {
  TileInfo ti{0, 0, 0, false};
  const int nt = shared_launch ? p.n_tiles[1] : p.n_tiles[0];
  if (tile >= nt) return ti;
  const int idx = shared_launch ? p.n_tiles[0] + tile : tile;
  ti.g = p.tile_grp[idx];
  const int m0 = p.tile_m0[idx];
  ti.slot0 = p.grp_off[ti.g] + m0;
  ti.rows = min(kBM, p.grp_cnt[ti.g] - m0);
  ti.ok = ti.g <= E && ti.rows > 0;
  return ti;
}

// ----------------------------------------------------------- grouped GEMM
//
// One workgroup: 256 slots x 128 output columns, 8 waves; wave w owns slots
// [64 (w & 3), +64) and half of the columns (w >> 2).  K advances 64 at a time
// through a ring of 3 LDS stages filled by global_load_lds two steps ahead.
//   A stage: 256 rows x 128 bytes (bf16 rows of x, or of act), chunk-swizzled.
//   B stage (gate_up): 128 weight rows x 128 bytes -- gate rows [n0, n0+64)
//            then up rows [I+n0, I+n0+64) -- chunk-swizzled like A.
//   B stage (down):    64 K rows x 256 bytes of the (I, H) down matrix
//            (128 columns); a lane gathers its 8 K values of one column with
//            8 two-byte LDS reads.  Chunks are XOR-ed with 4 in K rows 8..15
//            of every 16 so that the two half-waves hit different banks.
//
// INT8 / INT4 group-32 experts (model/moe.go:124-157): the stage holds the B
// codes (the same 64 K x 128 columns, 1 or 0.5 byte each) and their fp16
// scales, loaded by global_load_lds like the rest.  Each wave then dequantises
// the code pieces it loaded itself, w = code * scale (the f32 product of
// quantLinear.dequantize) rounded to bf16, into a bf16 B tile laid out as
// above (two such tiles alternate).  Since a wave converts only its own
// loads, its own wait for them suffices and a K step keeps one barrier.

enum GemmKind { kGateUp = 0, kDown = 1 };

constexpr int kWaves = kGemmThreads / 64;
constexpr int kAStage = kBM * kBK * 2;          // 32 KB
constexpr int kBStage = 128 * kBK * 2;          // 16 KB (bf16 B tile)
constexpr int kADma = kAStage / 16 / kGemmThreads;  // 16-byte pieces per thread per stage
constexpr int kBDma = kBStage / 16 / kGemmThreads;

// LDS plan of a B format.
template <int BF>
struct BGeom {
  static constexpr bool kQuant = BF == kINT8 || BF == kINT4;
  static constexpr int kPieceElems = BF == kINT8 ? 16 : 32;         // elements per 16-byte code piece
  static constexpr int kRaw = 128 * kBK * fmt_bytes_x2(BF) / 2;     // code bytes per stage
  static constexpr int kBWaves = kQuant ? kRaw / 16 / 64 : kWaves;  // waves that load (and convert) B
  static constexpr int kScale = kBWaves * 256;                      // fp16 scales per stage, 256 B per wave
  static constexpr int kStage = kAStage + (kQuant ? kRaw + kScale : kBStage);
  static constexpr int kTile = kQuant ? kBStage : 16;               // one dequantised B tile
  static constexpr int kBLoads = kQuant ? 2 : kBDma;                // B loads per B-wave thread per step
};

// s_waitcnt vmcnt(N) with the other counters untouched (gfx9 encoding).  The
// builtin is not a memory operation for the compiler, so the empty asm keeps
// LDS reads of the landed data from being hoisted above it.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
  asm volatile("" ::: "memory");
}

// Wait until this wave's LDS writes have completed.  s_barrier does not wait
// for them on gfx950 (and the compiler inserts no wait before it), so data a
// wave writes to LDS for the others needs this before the barrier.
__device__ __forceinline__ void wait_lds_writes() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier for the GEMM pipeline.  __syncthreads() also waits for
// every outstanding global load (vmcnt(0)), which would drain the prefetched
// stages.  Here each wave has already waited for its own LDS-direct loads of
// the stage (wait_vm), for its LDS reads of the previous stage (consumed by its
// MFMAs) and, where it wrote LDS, for those writes (wait_lds_writes), so the
// bare s_barrier suffices; the empty asm statements keep the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  const bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
  uint32_t r;
  __builtin_memcpy(&r, &h, 4);
  return r;
}

// Dequantised values of one 16-byte code piece, as packed bf16 pairs:
// out[i] holds elements 2i and 2i+1.  scale(e) gives element e's scale.
// INT8: 16 codes, value = code.  INT4: 32 elements, byte b holds element 2b in
// its high nibble and 2b+1 in its low nibble, value = nibble - 8; the product
// (nibble - 8) * s is formed as fma(nibble, s, -8 s), which rounds the same
// exact value once.
template <int BF, typename ScaleFn>
__device__ __forceinline__ void dequant_piece(const uint4 v, ScaleFn scale,
                                              uint32_t (&out)[BGeom<BF>::kPieceElems / 2]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if constexpr (BF == kINT8) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b += 2) {
        const int e = 4 * q + b;
        const float f0 = (float)(int8_t)((u[q] >> (8 * b)) & 0xffu) * scale(e);
        const float f1 = (float)(int8_t)((u[q] >> (8 * b + 8)) & 0xffu) * scale(e + 1);
        out[e / 2] = pack_bf16(f0, f1);
      }
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t hi = (u[q] >> 4) & 0x0f0f0f0fu, lo = u[q] & 0x0f0f0f0fu;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const int e = 8 * q + 2 * b;
        const float s0 = scale(e), s1 = scale(e + 1);
        const float f0 = fmaf((float)((hi >> (8 * b)) & 0xffu), s0, -8.0f * s0);
        const float f1 = fmaf((float)((lo >> (8 * b)) & 0xffu), s1, -8.0f * s1);
        out[e / 2] = pack_bf16(f0, f1);
      }
    }
  }
}

// 4 bytes per lane from global memory into LDS at lds_wave_base + 4 * lane.
__device__ __forceinline__ void dma4(const void *src, const unsigned char *lds_wave_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds_wave_base));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0)
               : "memory", "m0");
}

// Work order, XCD-aware: workgroups are dealt to the 8 XCDs round-robin by
// linear id, so id -> (tile, column chunk) gives every XCD whole tiles and runs
// the ny column chunks of a tile back to back on one XCD, whose L2 then holds
// the tile's A rows (gathered x, or act) for all of them.
constexpr int kXcds = 8;

template <int KIND, int BF>
__global__ void __launch_bounds__(kGemmThreads) grouped_gemm(PrefillArgs a, int shared_launch, int ny) {
  using G = BGeom<BF>;
  __shared__ __align__(16) unsigned char lds0[G::kStage], lds1[G::kStage], lds2[G::kStage];
  __shared__ __align__(16) unsigned char btile[2][G::kTile];
  const int xcd = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int tile = (j / ny) * kXcds + xcd, chunk = j % ny;
  const TileInfo ti = tile_of(a.p, a.E, shared_launch, tile);
  if (!ti.ok) return;
  const bool sh = ti.g == a.E;
  const int H = a.H;
  const int N = KIND == kGateUp ? (sh ? a.Is : a.I) : H;       // output columns of the group
  const int K = KIND == kGateUp ? H : (sh ? a.Is : a.I);
  const int n0 = chunk * (KIND == kGateUp ? 64 : 128);
  if (n0 >= N) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so branches on it are scalar
  const int64_t rb = fmt_matrix_bytes(BF, 1, H);  // bytes of a gate/up row or of a transposed down row

  // A rows staged by this thread: row r = (i * kWaves + w) * 8 + lane / 8
  const uint16_t *arow[kADma];
  int achunk[kADma];
#pragma unroll
  for (int i = 0; i < kADma; i++) {
    const int r = (i * kWaves + w) * 8 + (lane >> 3);
    achunk[i] = (lane & 7) ^ swz_of(r);
    const int m = min(r, ti.rows - 1);
    if constexpr (KIND == kGateUp) arow[i] = a.xb + (size_t)a.p.tok[ti.slot0 + m] * H;
    else arow[i] = a.act + (size_t)(ti.slot0 + m) * a.Imax;
  }
  // B pieces staged by this thread (bf16), or its code piece and scale
  // source (INT formats, waves below kBWaves)
  const uint16_t *bsrc[kBDma];
  const uint8_t *qsrc = nullptr;   // code piece at K step 0
  const uint16_t *ssrc = nullptr;  // scales at K step 0
  const bool bwave = G::kBWaves == kWaves || w < G::kBWaves;
  if constexpr (!G::kQuant) {
#pragma unroll
    for (int i = 0; i < kBDma; i++) {
      const int sidx = (i * kWaves + w) * 64 + lane;  // 16-byte slot of the stage
      if constexpr (KIND == kGateUp) {
        const int r = sidx >> 3, c = (sidx & 7) ^ swz_of(r);
        const uint8_t *gb = sh ? a.sgate : a.gu + (size_t)ti.g * a.gu_bytes;
        const uint8_t *ub = sh ? a.sup : gb + (size_t)a.I * rb;
        const uint8_t *row = r < 64 ? gb + (size_t)(n0 + r) * rb : ub + (size_t)(n0 + r - 64) * rb;
        bsrc[i] = reinterpret_cast<const uint16_t *>(row) + c * 8;
      } else {
        const int kr = sidx >> 4, c = (sidx & 15) ^ (((kr >> 3) & 1) << 2);
        const uint8_t *db = sh ? a.sdown : a.dn + (size_t)ti.g * a.dn_bytes;
        bsrc[i] = reinterpret_cast<const uint16_t *>(db) + (size_t)kr * H + n0 + c * 8;
      }
    }
  } else if (bwave) {
    const int gsc = H / kGroup;  // scales per gate/up row
    if constexpr (KIND == kGateUp) {
      // piece tid: row r, K elements [p * PE, +PE) of the stage
      constexpr int PPR = kBK / G::kPieceElems;
      const int r = tid / PPR, p = tid % PPR;
      const uint8_t *gb = sh ? a.sgate : a.gu + (size_t)ti.g * a.gu_bytes;
      const uint8_t *ub = sh ? a.sup : gb + (size_t)a.I * rb;
      const uint16_t *gs = sh ? a.sgate_s : a.gu_s + (size_t)ti.g * a.gu_scales;
      const uint16_t *us = sh ? a.sup_s : gs + (size_t)a.I * gsc;
      const int row = r < 64 ? n0 + r : n0 + r - 64;
      qsrc = (r < 64 ? gb : ub) + (size_t)row * rb + p * 16;
      ssrc = (r < 64 ? gs : us) + (size_t)row * gsc;  // + 2 kt: the row's two groups of the step
    } else {
      // piece tid: K row kr, columns [n0 + p * PE, +PE); lanes 0..15 load the
      // wave's 128 column scales of its group
      constexpr int PPR = 128 / G::kPieceElems;
      const int kr = tid / PPR, p = tid % PPR;
      const uint8_t *db = sh ? a.sdown : a.dn + (size_t)ti.g * a.dn_bytes;
      const uint16_t *ds = sh ? a.sdown_s : a.dn_s + (size_t)ti.g * a.dn_scales;
      qsrc = db + (size_t)kr * rb + (size_t)n0 * fmt_bytes_x2(BF) / 2 + p * 16;
      ssrc = ds + n0 + (lane & 15) * 8;  // + ((k0 + first K row of the wave) / 32) * H
    }
  }
  auto issue = [&](unsigned char *sa, int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < kADma; i++) dma16(arow[i] + k0 + achunk[i] * 8, sa + (i * kWaves + w) * 1024);
    if constexpr (!G::kQuant) {
      unsigned char *sb = sa + kAStage;
#pragma unroll
      for (int i = 0; i < kBDma; i++) {
        const uint16_t *src = KIND == kGateUp ? bsrc[i] + k0 : bsrc[i] + (size_t)k0 * H;
        dma16(src, sb + (i * kWaves + w) * 1024);
      }
    } else if (bwave) {
      unsigned char *raw = sa + kAStage, *sc = raw + G::kRaw;
      if constexpr (KIND == kGateUp) {
        dma16(qsrc + (size_t)k0 * fmt_bytes_x2(BF) / 2, raw + w * 1024);
        dma4(ssrc + 2 * kt, sc + w * 256);
      } else {
        dma16(qsrc + (size_t)k0 * rb, raw + w * 1024);
        constexpr int RPW = 64 / G::kBWaves;  // K rows per wave
        if (lane < 16) dma16(ssrc + (size_t)((k0 + w * RPW) / kGroup) * H, sc + w * 256);
      }
    }
  };
  // INT formats: dequantise this wave's code pieces of stage `cur` into `bt`
  auto convert = [&](const unsigned char *cur, unsigned char *bt) {
    if constexpr (G::kQuant) {
      if (!bwave) return;
      constexpr int PE = G::kPieceElems;
      const unsigned char *raw = cur + kAStage, *sc = raw + G::kRaw + w * 256;
      const uint4 v = *reinterpret_cast<const uint4 *>(raw + tid * 16);
      uint32_t o[PE / 2];
      if constexpr (KIND == kGateUp) {
        constexpr int PPR = kBK / PE;
        const int r = tid / PPR, p = tid % PPR;
        const uint32_t sw = *reinterpret_cast<const uint32_t *>(sc + lane * 4);
        const float s = f16_to_f32((uint16_t)(((p * PE) / kGroup) ? (sw >> 16) : (sw & 0xffffu)));
        dequant_piece<BF>(v, [&](int) { return s; }, o);
#pragma unroll
        for (int c = 0; c < PE / 8; c++)
          *reinterpret_cast<uint4 *>(bt + swz(r, p * (PE / 8) + c)) =
              make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
      } else {
        constexpr int PPR = 128 / PE;
        const int kr = tid / PPR, p = tid % PPR;
        uint4 sv[PE / 8];
#pragma unroll
        for (int c = 0; c < PE / 8; c++) sv[c] = *reinterpret_cast<const uint4 *>(sc + (p * PE + 8 * c) * 2);
        dequant_piece<BF>(v, [&](int e) {
          const uint32_t word = (&sv[e / 8].x)[(e % 8) / 2];
          return f16_to_f32((uint16_t)((e & 1) ? (word >> 16) : (word & 0xffffu)));
        }, o);
        const int x = ((kr >> 3) & 1) << 2;
#pragma unroll
        for (int c = 0; c < PE / 8; c++)
          *reinterpret_cast<uint4 *>(bt + kr * 256 + (((p * (PE / 8) + c) ^ x) << 4)) =
              make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
      }
      wait_lds_writes();  // the tile is read by every wave after the barrier
    }
  };

  // wave w: slot rows [64 (w >> 1), +64), column half w & 1.  The SIMD of
  // wave w also runs wave w + 4, whose rows lie 128 further: a tile with few
  // rows still keeps every SIMD's MFMA busy, and 32-row blocks past the tile's
  // rows skip their LDS reads and MFMAs.
  const int wm = w >> 1, wn = w & 1, hi = lane >> 5, l32 = lane & 31;
  const int nb = min(2, max(0, (ti.rows - wm * 64 + 31) >> 5));  // live 32-row blocks of this wave
  f32x16_t acc[2][2];  // [slot block][gate/up, or column block]
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[b][q][e] = 0.0f;

  const int KT = K / kBK;
  const int ar0 = wm * 64 + l32;
  // one K step on stage `cur`; refills stage `nxt2` with step kt + 2
  // Every step issues one batch of loads, so that the count of loads in flight
  // is the same at every step: past the end of K the batch re-reads the last K
  // slice into a stage that is never read again.
  auto step = [&](const unsigned char *cur, unsigned char *nxt2, int kt) {
    // stage kt landed; the batch of step kt + 1 may still fly
    if (!G::kQuant || bwave) wait_vm<kADma + G::kBLoads>();
    else wait_vm<kADma>();
    unsigned char *bt = btile[kt & 1];
    convert(cur, bt);
    lds_barrier();  // stage kt visible to all; stage kt + 2 (read at kt - 1) is free
    const unsigned char *sa = cur, *sb = G::kQuant ? bt : cur + kAStage;
    bf16x8_t av[2][4], bv[2][4];
    if (nb == 0) {  // nothing to multiply: keep the pipeline's loads in step
      issue(nxt2, min(kt + 2, KT - 1));
      return;
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const int c = ks * 2 + hi;
#pragma unroll
      for (int b = 0; b < 2; b++)
        if (b < nb) av[b][ks] = *reinterpret_cast<const bf16x8_t *>(sa + swz(ar0 + 32 * b, c));
      if constexpr (KIND == kGateUp) {
        bv[0][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(wn * 32 + l32, c));
        bv[1][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(64 + wn * 32 + l32, c));
      } else {
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const int nl = wn * 64 + q * 32 + l32;
          const unsigned char *col = sb + (((nl >> 3) ^ (hi << 2)) << 4) + (nl & 7) * 2 + (ks * 16 + hi * 8) * 256;
          union {
            uint16_t h[8];
            bf16x8_t v;
          } u;
#pragma unroll
          for (int i = 0; i < 8; i++) u.h[i] = *reinterpret_cast<const uint16_t *>(col + i * 256);
          bv[q][ks] = u.v;
        }
      }
    }
    issue(nxt2, min(kt + 2, KT - 1));
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
      for (int b = 0; b < 2; b++)
        if (b < nb)
#pragma unroll
          for (int q = 0; q < 2; q++)
            acc[b][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b][ks], bv[q][ks], acc[b][q], 0, 0, 0);
  };
  issue(lds0, 0);
  issue(lds1, min(1, KT - 1));
  for (int kt = 0; kt < KT; kt += 3) {
    step(lds0, lds2, kt);
    if (kt + 1 < KT) step(lds1, lds0, kt + 1);
    if (kt + 2 < KT) step(lds2, lds1, kt + 2);
  }
  wait_vm<0>();  // no LDS-direct load may land after the workgroup ends

  if constexpr (KIND == kGateUp) {
    // act = silu(g) * u -> bf16 (model/moe.go:64-75), row pitch Imax
    const int n = n0 + wn * 32 + l32;
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = wm * 64 + b * 32 + 8 * j + 4 * hi + i;
          if (m < ti.rows) {
            const float g = acc[b][0][4 * j + i], u = acc[b][1][4 * j + i];
            const float sgl = g / (1.0f + __expf(-g));
            a.act[(size_t)(ti.slot0 + m) * a.Imax + n] = f32_to_bf16_rne(sgl * u);
          }
        }
  } else {
    // y[slot] = routing weight (or shared gate) * (down . act), f32
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
            for (int q = 0; q < 2; q++)
              a.y[(size_t)slot * H + n0 + wn * 64 + q * 32 + l32] = ws * acc[b][q][4 * j + i];
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
  // bf16, int8 or int4 experts; the shared expert (if any) in the same format
  if (expert_fmt != kBF16 && expert_fmt != kINT8 && expert_fmt != kINT4) return false;
  if (Is > 0 && shared_fmt != expert_fmt) return false;
  return H % 128 == 0 && I % 64 == 0 && (Is == 0 || Is % 64 == 0);
}

int prefill_max_tiles(int T, int k, int E) {
  const int n = T * k;
  return (n + kBM - 1) / kBM + (E < n ? E : n);
}

hipError_t launch_prefill_dispatch(const PrefillArgs &a, const int32_t *ids, const float *wts, const float *x,
                                   const float *shared_gate, float *sg, hipStream_t st) {
  const bool with_shared = a.Is > 0;
  QMOE_LAUNCH(prep_kernel, dim3(a.T), dim3(256), 0, st, x, a.H, with_shared ? shared_gate : nullptr, a.xb,
                     sg);
  QMOE_LAUNCH(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, st, ids, wts, sg, a.T, a.k, a.E,
                     (int)with_shared, a.p);
  return hipGetLastError();
}

template <int KIND>
static hipError_t gemm_launch(const PrefillArgs &a, bool shared, int ny, hipStream_t st) {
  const int tiles = shared ? (a.T + kBM - 1) / kBM : prefill_max_tiles(a.T, a.k, a.E);
  const int blocks = (tiles + kXcds - 1) / kXcds * kXcds * ny;
#define L(BF) QMOE_LAUNCH((grouped_gemm<KIND, BF>), dim3(blocks), dim3(kGemmThreads), 0, st, a, (int)shared, ny)
  switch (a.fmt) {
  case kBF16: L(kBF16); break;
  case kINT8: L(kINT8); break;
  case kINT4: L(kINT4); break;
  default: return hipErrorInvalidValue;
  }
#undef L
  return hipGetLastError();
}

hipError_t launch_prefill_gate_up(const PrefillArgs &a, bool shared, hipStream_t st) {
  return gemm_launch<kGateUp>(a, shared, (shared ? a.Is : a.I) / 64, st);
}

hipError_t launch_prefill_down(const PrefillArgs &a, bool shared, hipStream_t st) {
  return gemm_launch<kDown>(a, shared, a.H / 128, st);
}

hipError_t launch_prefill_combine(const PrefillArgs &a, float *out, hipStream_t st) {
  QMOE_LAUNCH(combine_kernel, dim3(a.T), dim3(256), 0, st, a.y, a.p.slot_of, a.T, a.k, a.H,
                     (int)(a.Is > 0), out);
  return hipGetLastError();
}

}  // namespace qmoe
