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
//             Also the tile table: one entry per BM slots of a group.
//   gate_up   grouped GEMM: per (tile, 128 intermediate columns) a BM x 256
//             output block = BM gathered bf16 rows of x times the expert's
//             gate rows [n0, n0+128) and up rows [I+n0, I+n0+128) over K = H,
//             on v_mfma_f32_32x32x16_bf16 with f32 accumulation; SwiGLU in the
//             epilogue (model/moe.go:64-75): act = silu(g) * u, stored bf16.
//   down      grouped GEMM: act rows of the tile times 256 rows of the
//             expert's down matrix, (H, I) reference layout, over K = I; the
//             routing weight (or shared gate) scales the f32 result,
//             y[slot] = w * (down . act) (model/moe.go:76-84), stored bf16.
//   combine   out[t] = sum over ranks r in rank order of y[slot_of[t, r]],
//             then + y[shared slot of t] (model/moe.go:82-97), in f32.
// The slot order inside an expert comes from LDS atomics and may vary from run
// to run; every output row depends only on its own token, so results do not.
//
// Expert weights are bf16, or int8 / int4 group-32 codes with fp16 scales
// that the GEMMs dequantise to bf16 in LDS on the way to the MFMAs.  Tiles are
// staged through LDS with global_load_lds (16 bytes per lane), an XOR swizzle
// of the 16-byte chunks of each 128-byte row so that the MFMA operand reads
// (one row per lane) hit distinct banks.
#include "common.hpp"
#include "kernels.hpp"

namespace qmoe {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kBK = 64;         // K per stage (128 bytes of bf16 per row)
constexpr int kGemmThreads = 512;

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

// Counts and slot ranges, one workgroup: J pairs per thread, all loaded up
// front so that the global loads overlap (0 = a plain loop for any count).
// Writes each expert's first slot and count, the tile table, and the expert
// cursors that scatter_kernel advances.
template <int J>
__global__ void __launch_bounds__(kDispatchThreads)
    dispatch_kernel(const int32_t *__restrict__ ids, int T, int k, int E, int with_shared, int bm, int bms,
                    PrefillPlan p) {
  __shared__ int cnt[1024], incl[1024], tincl[1024];
  const int tid = threadIdx.x;
  const int n = T * k;
  constexpr int JJ = J > 0 ? J : 1;
  int id[JJ];
  if constexpr (J > 0) {
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int i = tid + j * kDispatchThreads;
      id[j] = i < n ? ids[i] : -1;
    }
  }
  cnt[tid] = 0;
  __syncthreads();
  if constexpr (J > 0) {
#pragma unroll
    for (int j = 0; j < J; j++)
      if (id[j] >= 0) atomicAdd(&cnt[id[j]], 1);
  } else {
    for (int i = tid; i < n; i += kDispatchThreads) atomicAdd(&cnt[ids[i]], 1);
  }
  __syncthreads();
  // inclusive scans of the counts and of the tiles per expert (E <= 1024)
  const int c = tid < E ? cnt[tid] : 0;
  const int ct = (c + bm - 1) / bm;
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
    p.cursor[tid] = off;
    for (int q = 0; q < ct; q++) {
      p.tile_grp[toff + q] = tid;
      p.tile_m0[toff + q] = q * bm;
    }
  }
  // the shared expert's tiles hold bms slots (its GEMMs may run another format)
  const int shared_tiles = with_shared ? (T + bms - 1) / bms : 0;
  for (int q = tid; q < shared_tiles; q += kDispatchThreads) {
    p.tile_grp[routed_tiles + q] = E;
    p.tile_m0[routed_tiles + q] = q * bms;
  }
  if (tid == 0) {
    p.n_tiles[0] = routed_tiles;
    p.n_tiles[1] = shared_tiles;
    p.grp_off[E] = n;
    p.grp_cnt[E] = with_shared ? T : 0;
  }
}

// Every (token, rank) pair into its expert's slot range, kScatterPairs pairs
// per workgroup: each pair takes a rank among the workgroup's pairs of its
// expert (LDS atomics), the workgroup reserves each expert's run with one
// global atomic on its cursor, and the pairs land at run start + rank.  A hot
// expert's cursor then sees one atomic per workgroup instead of one per pair.
// The order of slots within an expert is free: each row of the GEMMs depends
// on its own slot only.  Workgroups past the pairs write the shared expert's
// slots in token order.
constexpr int kScatterPairs = 1024;

__global__ void __launch_bounds__(256) scatter_kernel(const int32_t *__restrict__ ids, const float *__restrict__ wts,
                                                      const float *__restrict__ sg, int T, int k, int E,
                                                      int with_shared, PrefillPlan p) {
  __shared__ int lcnt[1024], lbase[1024];  // E <= 1024
  const int n = T * k, tid = threadIdx.x;
  const int nbr = (n + kScatterPairs - 1) / kScatterPairs;
  if ((int)blockIdx.x >= nbr) {
    const int t = ((int)blockIdx.x - nbr) * 256 + tid;
    if (with_shared && t < T) {
      p.tok[n + t] = t;
      p.wslot[n + t] = sg[t];
    }
    return;
  }
  for (int e = tid; e < E; e += 256) lcnt[e] = 0;
  __syncthreads();
  constexpr int PPT = kScatterPairs / 256;
  int id[PPT], rank[PPT];
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    const int i = blockIdx.x * kScatterPairs + j * 256 + tid;
    id[j] = i < n ? ids[i] : -1;
    rank[j] = id[j] >= 0 ? atomicAdd(&lcnt[id[j]], 1) : 0;
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    const int c = lcnt[e];
    lbase[e] = c ? atomicAdd(&p.cursor[e], c) : 0;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    if (id[j] < 0) continue;
    const int i = blockIdx.x * kScatterPairs + j * 256 + tid;
    const int slot = lbase[id[j]] + rank[j];
    p.tok[slot] = i / k;
    p.wslot[slot] = wts[i];
    p.slot_of[i] = slot;
  }
}

// ------------------------------------------------------------ tile setup

struct TileInfo {
  int g, slot0, rows;
  bool ok;
};

__device__ __forceinline__ TileInfo tile_of(const PrefillPlan &p, int E, bool shared_launch, int tile, int bm) {
  TileInfo ti{0, 0, 0, false};
  const int nt = shared_launch ? p.n_tiles[1] : p.n_tiles[0];
  if (tile >= nt) return ti;
  const int idx = shared_launch ? p.n_tiles[0] + tile : tile;
  ti.g = p.tile_grp[idx];
  const int m0 = p.tile_m0[idx];
  ti.slot0 = p.grp_off[ti.g] + m0;
  ti.rows = min(bm, p.grp_cnt[ti.g] - m0);
  ti.ok = ti.g <= E && ti.rows > 0;
  return ti;
}

// ----------------------------------------------------------- grouped GEMM
//
// One workgroup: a tile of BM slots (256 for bf16 weights, 128 for the
// group-32 formats) x 256 B rows over K, 8 waves in 4 x 2: wave w owns the
// slots [BM/4 (w >> 1), +BM/4) and half of the B rows (w & 1) -- for gate_up
// the gate rows [n0 + 64 (w & 1), +64) and the up rows with the same
// indices, so that a SwiGLU pair stays in one wave; for down 128 output
// columns.  B is always a matrix with its rows along K: gate and up rows of
// the (2I, H) stack, or rows of the down matrix in the reference (H, I)
// layout, which the device keeps next to the decode kernel's transposed copy.
//
// Large tiles keep the bytes that cross the L2 per MFMA low: every K step
// brings BM + 256 rows of 128 bytes into LDS for BM x 256 x 64 multiply-adds.
// K advances 64 at a time.  A (BM x 64 bf16: gathered rows of x, or act) and
// B (256 x 64: bf16, or int8 / int4 codes plus their scales) come into LDS
// by global_load_lds on rings of their own.  Rows are 128 bytes with an XOR
// swizzle of their 16-byte chunks so that the MFMA operand reads (one row per
// lane) hit distinct banks.
//
// INT8 / INT4 group-32 experts (model/moe.go:124-157): each thread
// dequantises the code pieces it loaded itself, w = code * scale (the f32
// product of quantLinear.dequantize) rounded to bf16, into a bf16 B tile (two
// alternate) before the step's barrier; since a wave converts only its own
// loads, its own wait for them suffices and a K step keeps one barrier.

enum GemmKind { kGateUp = 0, kDown = 1 };

constexpr int kWaves = kGemmThreads / 64;
constexpr int kBN = 256;                        // B rows per tile
constexpr int kBStage = kBN * kBK * 2;          // 32 KB (bf16 B tile)

// Tile and LDS plan of a weight format.
template <int BF>
struct GemmCfg {
  static constexpr bool kQuant = BF == kINT8 || BF == kINT4;
  static constexpr int kBM = kQuant ? 128 : 256;                    // slots per tile
  static constexpr int kAStage = kBM * kBK * 2;
  static constexpr int kADma = kAStage / 16 / kGemmThreads;         // A pieces per thread per step
  static constexpr int kAStages = kQuant ? (BF == kINT8 ? 2 : 3) : 2;  // A ring: kAStages - 1 steps ahead
  static constexpr int kPieceElems = BF == kINT8 ? 16 : 32;         // elements per 16-byte code piece
  static constexpr int kRaw = kBN * kBK * fmt_bytes_x2(BF) / 2;     // B bytes per stage (codes, or bf16)
  static constexpr int kBPieces = kRaw / 16 / kGemmThreads;         // B pieces per thread per step
  static constexpr int kScale = kQuant ? kBPieces * kGemmThreads * 4 : 0;  // a scale dword per code piece
  static constexpr int kBSize = kRaw + kScale;                      // one B ring stage
  static constexpr int kBStages = 3;                                 // B ring: kBStages - 1 steps ahead
  static constexpr int kTile = kQuant ? kBStage : 16;               // one dequantised B tile
  static constexpr int kBLoads = kQuant ? 2 * kBPieces : kBPieces;  // B loads per thread per step
  static constexpr int kRB = kBM / 4;                               // slots per wave
  static constexpr int kNRB = kRB / 32;                             // 32-slot blocks per wave
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

// Dequantised values of one 16-byte code piece with one scale s, as packed
// bf16 pairs: out[i] holds elements 2i and 2i+1.  INT8: 16 codes, value =
// code.  INT4: 32 elements, byte b holds element 2b in its high nibble and
// 2b+1 in its low nibble, value = nibble - 8; the product (nibble - 8) * s is
// formed as fma(nibble, s, -8 s), which rounds the same exact value once.
template <int BF>
__device__ __forceinline__ void dequant_piece(const uint4 v, float s, uint32_t (&out)[GemmCfg<BF>::kPieceElems / 2]) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if constexpr (BF == kINT8) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int b = 0; b < 4; b += 2) {
        const float f0 = (float)(int8_t)((u[q] >> (8 * b)) & 0xffu) * s;
        const float f1 = (float)(int8_t)((u[q] >> (8 * b + 8)) & 0xffu) * s;
        out[(4 * q + b) / 2] = pack_bf16(f0, f1);
      }
  } else {
    const float m8 = -8.0f * s;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t hi = (u[q] >> 4) & 0x0f0f0f0fu, lo = u[q] & 0x0f0f0f0fu;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const float f0 = fmaf((float)((hi >> (8 * b)) & 0xffu), s, m8);
        const float f1 = fmaf((float)((lo >> (8 * b)) & 0xffu), s, m8);
        out[4 * q + b] = pack_bf16(f0, f1);
      }
    }
  }
}

// 4 bytes per lane from global memory into LDS at lds_wave_base + 4 * lane.
__device__ __forceinline__ void dma4(const void *src, const unsigned char *lds_wave_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds_wave_base));
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Work order, XCD-aware: workgroups are dealt to the 8 XCDs round-robin by
// linear id.  XCD x runs the x-th contiguous range of tiles -- tiles of one
// expert are adjacent, so an expert's B rows come from HBM about once into that
// XCD's L2 -- and the ny column chunks of a tile back to back, which share the
// tile's A rows in the same L2.
//
// A workgroup holds a CU (its LDS), so an XCD runs its n items in rounds of
// cus = n_cu / 8.  For a gate_up, a last round of at most cus / 2 items runs
// as twice as many half items: the two halves of the tile's slots in two
// workgroups, each with only the waves of its half issuing MFMAs, which takes
// about 0.9 of a full item's time (bf16, C = k, T = 2048 at Qwen3-30B: 48
// items per XCD as 32 full + 32 halves instead of two full rounds).  The
// group-32 formats split only a launch that is one part-filled round.
constexpr int kXcds = 8;

template <int KIND, int BF>
__global__ void __launch_bounds__(kGemmThreads) grouped_gemm(PrefillArgs a, int shared_launch, int ny) {
  using G = GemmCfg<BF>;
  constexpr int NAS = G::kAStages, DA = NAS - 1;  // A ring stages, A prefetch distance
  constexpr int NBS = G::kBStages, DB = NBS - 1;  // B ring stages, B prefetch distance
  __shared__ __align__(16) unsigned char aring[NAS][G::kAStage];
  __shared__ __align__(16) unsigned char bring[NBS][G::kBSize];
  __shared__ __align__(16) unsigned char btile[2][G::kTile];
  const int xcd = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int nt = shared_launch ? a.p.n_tiles[1] : a.p.n_tiles[0];
  const int per_xcd = (nt + kXcds - 1) / kXcds;
  const int n = per_xcd * ny;  // items of this XCD
  int split_from = n;          // items from here on run as two half items
  if constexpr (KIND == kGateUp) {
    // the group-32 formats (lockstep, every wave dequantising the B tile)
    // gain only when the whole launch is one part-filled round (C5's shared
    // expert: 16 items per XCD, 52 -> 43 us); a last round of more items got
    // slower
    const int cus = a.n_cu / kXcds, rem = cus > 0 ? n % cus : 0;
    if (rem > 0 && 2 * rem <= cus && (BF == kBF16 || rem == n)) split_from = n - rem;
  }
  int item = j, half = -1;
  if (j >= split_from) {
    item = split_from + (j - split_from) / 2;
    half = (j - split_from) % 2;
  }
  if (item >= n) return;
  const int chunk = item % ny;
  TileInfo ti = tile_of(a.p, a.E, shared_launch, xcd * per_xcd + item / ny, G::kBM);
  if (half >= 0) {
    ti.slot0 += half * (G::kBM / 2);
    ti.rows = min(G::kBM / 2, ti.rows - half * (G::kBM / 2));
    ti.ok = ti.ok && ti.rows > 0;
  }
  if (!ti.ok) return;
  const bool sh = ti.g == a.E;
  const int H = a.H;
  const int Ig = sh ? a.Is : a.I;                  // intermediate size of the group
  const int N = KIND == kGateUp ? Ig : H;          // output columns of the group
  const int K = KIND == kGateUp ? H : Ig;
  const int n0 = chunk * (KIND == kGateUp ? kBN / 2 : kBN);
  if (n0 >= N) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so branches on it are scalar
  const int64_t rbB = fmt_matrix_bytes(BF, 1, K);         // bytes of one B row
  const int gsc = K / kGroup;                             // scales per B row

  // B row r of the tile and its scale row: gate_up rows n0 + r (gate,
  // r < 128) or up rows n0 + r - 128; down rows n0 + r of the (H, K) matrix
  auto brow = [&](int r, const uint16_t *&srow) -> const uint8_t * {
    srow = nullptr;
    if constexpr (KIND == kGateUp) {
      const uint8_t *gb = sh ? a.sgate : a.gu + (size_t)ti.g * a.gu_bytes;
      const uint8_t *ub = sh ? a.sup : gb + (size_t)a.I * rbB;
      const int row = r < kBN / 2 ? n0 + r : n0 + r - kBN / 2;
      if constexpr (G::kQuant) {
        const uint16_t *gs = sh ? a.sgate_s : a.gu_s + (size_t)ti.g * a.gu_scales;
        const uint16_t *us = sh ? a.sup_s : gs + (size_t)a.I * gsc;
        srow = (r < kBN / 2 ? gs : us) + (size_t)row * gsc;
      }
      return (r < kBN / 2 ? gb : ub) + (size_t)row * rbB;
    } else {
      const uint8_t *db = sh ? a.sdown : a.dn + (size_t)ti.g * a.dn_bytes;
      if constexpr (G::kQuant) srow = (sh ? a.sdown_s : a.dn_s + (size_t)ti.g * a.dn_scales) + (size_t)(n0 + r) * gsc;
      return db + (size_t)(n0 + r) * rbB;
    }
  };

  // A rows staged by this thread: piece i covers rows [a_row0(i), +8), one
  // per 8 lanes.  bf16 (ping-pong below): each half of the waves stages the
  // half of the slots it reads; group-32: the pieces interleave all waves.
  auto a_row0 = [&](int i) {
    if constexpr (G::kQuant) return (i * kWaves + w) * 8;
    else return (w / (kWaves / 2)) * (G::kBM / 2) + (i * (kWaves / 2) + w % (kWaves / 2)) * 8;
  };
  const uint16_t *arow[G::kADma];
  int achunk[G::kADma];
#pragma unroll
  for (int i = 0; i < G::kADma; i++) {
    const int r = a_row0(i) + (lane >> 3);
    achunk[i] = (lane & 7) ^ swz_of(r);
    const int m = min(r, ti.rows - 1);
    if constexpr (KIND == kGateUp) arow[i] = a.xb + (size_t)a.p.tok[ti.slot0 + m] * H;
    else arow[i] = a.act + (size_t)(ti.slot0 + m) * a.Imax;
  }
  // B pieces staged by this thread: piece i is 16-byte slot (i * kWaves + w)
  // * 64 + lane of the stage.  bf16: row r = slot / 8, its chunk swizzled;
  // INT formats: row r = slot / PPR, K elements [p * PE, +PE) of the step,
  // plus the dword of the row's two scales of the step.
  const uint8_t *bsrc[G::kBPieces];
  const uint16_t *ssrc[G::kBPieces];
#pragma unroll
  for (int i = 0; i < G::kBPieces; i++) {
    const int sidx = (i * kWaves + w) * 64 + lane;
    if constexpr (!G::kQuant) {
      const int r = sidx >> 3, c = (sidx & 7) ^ swz_of(r);
      bsrc[i] = brow(r, ssrc[i]) + c * 16;
    } else {
      constexpr int PPR = kBK / G::kPieceElems;
      bsrc[i] = brow(sidx / PPR, ssrc[i]) + (sidx % PPR) * 16;
    }
  }
  // loads of step s (slot by s, source clamped to the last step: past the end
  // of K a step re-reads the last K slice into a slot never read again, so
  // every step issues the same number of loads)
  const int KT = K / kBK;
  auto issue_a = [&](int s) {
    unsigned char *dst = aring[s % NAS];
    const int k0 = min(s, KT - 1) * kBK;
#pragma unroll
    for (int i = 0; i < G::kADma; i++) dma16(arow[i] + k0 + achunk[i] * 8, dst + a_row0(i) * 128);
  };
  auto issue_b = [&](int s) {
    unsigned char *dst = bring[s % NBS];
    const int kt = min(s, KT - 1);
#pragma unroll
    for (int i = 0; i < G::kBPieces; i++) {
      dma16(bsrc[i] + (size_t)kt * kBK * fmt_bytes_x2(BF) / 2, dst + (i * kWaves + w) * 1024);
      if constexpr (G::kQuant) dma4(ssrc[i] + 2 * kt, dst + G::kRaw + (i * kWaves + w) * 256);
    }
  };
  // INT formats: dequantise this thread's code pieces of a stage into `bt`
  auto convert = [&](const unsigned char *stage, unsigned char *bt) {
    if constexpr (G::kQuant) {
      constexpr int PE = G::kPieceElems, PPR = kBK / PE;
#pragma unroll
      for (int i = 0; i < G::kBPieces; i++) {
        const int sidx = (i * kWaves + w) * 64 + lane;
        const int r = sidx / PPR, p = sidx % PPR;
        const uint4 v = *reinterpret_cast<const uint4 *>(stage + sidx * 16);
        const uint32_t sw = *reinterpret_cast<const uint32_t *>(stage + G::kRaw + sidx * 4);
        const float s = f16_to_f32((uint16_t)(((p * PE) / kGroup) ? (sw >> 16) : (sw & 0xffffu)));
        uint32_t o[PE / 2];
        dequant_piece<BF>(v, s, o);
#pragma unroll
        for (int c = 0; c < PE / 8; c++)
          *reinterpret_cast<uint4 *>(bt + swz(r, p * (PE / 8) + c)) =
              make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
      }
      wait_lds_writes();  // the tile is read by every wave after the barrier
    }
  };

  const int wm = w >> 1, wn = w & 1, hi = lane >> 5, l32 = lane & 31;
  // live 32-slot blocks of this wave
  const int nrb = min(G::kNRB, max(0, (ti.rows - wm * G::kRB + 31) >> 5));
  // [slot block][gate 0, gate 1, up 0, up 1 -- or 4 column blocks].  The
  // weight fragment is the MFMA's first operand, so each accumulator holds the
  // transposed 32 x 32 block: lane l has slot l % 32 of the block and element
  // 4 j + i column 8 j + 4 (l / 32) + i -- four consecutive columns per quad,
  // stored as one 8-byte piece in the epilogue.
  f32x16_t acc[G::kNRB][4];
#pragma unroll
  for (int b = 0; b < G::kNRB; b++)
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[b][q][e] = 0.0f;
  int brl[4];  // this lane's B rows (MFMA columns)
#pragma unroll
  for (int q = 0; q < 4; q++)
    brl[q] = KIND == kGateUp ? (q >> 1) * (kBN / 2) + wn * 64 + (q & 1) * 32 + l32 : wn * 128 + q * 32 + l32;
  const int ar0 = wm * G::kRB + l32;

  // prologue: the loads of the steps before 0, in the steady-state order
  // (step s issues A of s + DA, then B of s + DB)
  constexpr int D = DA > DB ? DA : DB;
#pragma unroll
  for (int s = -D; s < 0; s++) {
    if (s + DA >= 0) issue_a(s + DA);
    if (s + DB >= 0) issue_b(s + DB);
  }
  // At step kt the loads issued after A (or B) of kt, whichever came later,
  // may still fly: those of the steps after it, and B (A) of its own step.
  constexpr int kAfterA = (DA - 1) * G::kADma + DA * G::kBLoads;  // A of kt was issued at step kt - DA
  constexpr int kAfterB = (DB - 1) * (G::kADma + G::kBLoads);     // B of kt at step kt - DB, after its A
  constexpr int kWait = kAfterA < kAfterB ? kAfterA : kAfterB;
  // fragment reads of stage kt (live 32-slot blocks only)
  auto read_frags = [&](int kt, const unsigned char *sb, bf16x8_t (&av)[G::kNRB][4], bf16x8_t (&bv)[4][4]) {
    const unsigned char *sa = aring[kt % NAS];
    if (nrb > 0) {
#pragma unroll
      for (int ks = 0; ks < 4; ks++) {
        const int c = ks * 2 + hi;
#pragma unroll
        for (int b = 0; b < G::kNRB; b++)
          if (b < nrb) av[b][ks] = *reinterpret_cast<const bf16x8_t *>(sa + swz(ar0 + 32 * b, c));
#pragma unroll
        for (int q = 0; q < 4; q++) bv[q][ks] = *reinterpret_cast<const bf16x8_t *>(sb + swz(brl[q], c));
      }
    }
  };
  auto mfmas = [&](const bf16x8_t (&av)[G::kNRB][4], const bf16x8_t (&bv)[4][4]) {
    if (nrb > 0) {
#pragma unroll
      for (int ks = 0; ks < 4; ks++)
#pragma unroll
        for (int b = 0; b < G::kNRB; b++)
          if (b < nrb)
#pragma unroll
            for (int q = 0; q < 4; q++)
              acc[b][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bv[q][ks], av[b][ks], acc[b][q], 0, 0, 0);
    }
  };
  if constexpr (G::kQuant) {
    for (int kt = 0; kt < KT; kt++) {
      wait_vm<kWait>();
      const unsigned char *sbs = bring[kt % NBS];
      unsigned char *bt = btile[kt & 1];
      convert(sbs, bt);
      lds_barrier();  // stage kt visible to all; the slots refilled below were read at kt - 1
      bf16x8_t av[G::kNRB][4], bv[4][4];
      read_frags(kt, bt, av, bv);
      issue_a(kt + DA);
      issue_b(kt + DB);
      mfmas(av, bv);
    }
  } else {
    // bf16: ping-pong.  Waves 0-3 (slots [0, BM/2)) and 4-7 (the other half)
    // share the SIMDs pairwise and run half a phase apart: while one group
    // issues its MFMAs for step kt, the other reads its fragments of a stage
    // and issues its loads, and at each barrier they swap.  Group 0 runs
    // M_kt | C_kt, group 1 the same one barrier later.  Hazards:
    //   a group stages only its own half of the A rows, so A of stage kt
    //   must have landed (each wave waiting for its own pieces) before the
    //   barrier that starts the group's M_kt: at the end of its C_{kt-1};
    //   B of stage kt is first read in group 0's M_kt, so group 1 waits for
    //   its B pieces of stage kt at the end of its M_{kt-1} (group 0 at the
    //   end of C_{kt-1}, together with A);
    //   the loads issued in M_kt go to the slot of stage kt - 1, whose last
    //   reader finished -- lgkmcnt(0) -- before the barrier that starts the
    //   issuing group's M_kt (A: the group itself; B: group 1's M_{kt-1}).
    // sched_barrier(0) keeps the compiler from moving MFMAs across phases.
    const bool g1 = w >= kWaves / 2;
    auto phase_barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    wait_vm<kWait>();  // own pieces of stage 0
    phase_barrier();
    if (g1) phase_barrier();
    for (int kt = 0; kt < KT; kt++) {
      bf16x8_t av[G::kNRB][4], bv[4][4];
      read_frags(kt, bring[kt % NBS], av, bv);  // M_kt
      issue_a(kt + DA);
      issue_b(kt + DB);
      wait_lds_writes();  // this wave's reads of stage kt are done before the barrier
      if (g1) wait_vm<kAfterB>();  // own B pieces of stage kt + 1, which group 0 reads next
      phase_barrier();
      mfmas(av, bv);  // C_kt
      if (g1) wait_vm<kAfterA>();  // own A pieces of stage kt + 1 (B: end of M_kt)
      else wait_vm<kWait>();       // own A and B pieces of stage kt + 1
      phase_barrier();
    }
    if (!g1) phase_barrier();
  }
  wait_vm<0>();  // no LDS-direct load may land after the workgroup ends

  // Epilogue through LDS.  A lane's accumulators hold one slot and runs of
  // four columns; stored straight to global memory they were 8-byte pieces
  // of 32 rows a row pitch apart (4.5-9 us per work item).  Each wave writes
  // its bf16 block (its kRB slots x its columns) into a region of its own in
  // the rings, rows padded by 16 bytes so that the 8-byte writes to 32 rows
  // fill the 64 banks twice, and stores it back out in 16-byte chunks along
  // rows (LDS accesses of one wave complete in order).
  constexpr int kWCols = KIND == kGateUp ? kBN / 4 : kBN / 2;  // bf16 columns of a wave
  constexpr int kWPitch = kWCols * 2 + 16;                     // LDS bytes per row of a wave's block
  constexpr int kWBytes = G::kRB * kWPitch;
  constexpr int kInA = (int)(sizeof(aring) / kWBytes);         // waves whose blocks fit in the A ring
  static_assert(kInA + (int)(sizeof(bring) / kWBytes) >= kWaves, "the waves' blocks fit the rings");
  unsigned char *const wt = w < kInA ? &aring[0][0] + w * kWBytes : &bring[0][0] + (w - kInA) * kWBytes;
  __syncthreads();  // every wave's fragment reads of the last stages are done
  auto put4 = [&](int r, int col, const float (&v)[4]) {
    *reinterpret_cast<uint2 *>(wt + r * kWPitch + col * 2) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
  };
  if constexpr (KIND == kGateUp) {
    // act = silu(g) * u -> bf16 (model/moe.go:64-75); the quotient by its
    // reciprocal (about an f32 ulp) ahead of the bf16 rounding
#pragma unroll
    for (int b = 0; b < G::kNRB; b++)
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float g = acc[b][q][4 * j4 + i], u = acc[b][q + 2][4 * j4 + i];
            v[i] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
          }
          put4(b * 32 + l32, q * 32 + 8 * j4 + 4 * hi, v);
        }
  } else {
    // y[slot] = routing weight (or shared gate) * (down . act)
#pragma unroll
    for (int b = 0; b < G::kNRB; b++) {
      const float ws = a.p.wslot[ti.slot0 + min(wm * G::kRB + b * 32 + l32, ti.rows - 1)];
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; i++) v[i] = ws * acc[b][q][4 * j4 + i];
          put4(b * 32 + l32, q * 32 + 8 * j4 + 4 * hi, v);
        }
    }
  }
  wait_lds_writes();  // the block is in LDS before the wave reads it back
  constexpr int kCpr = kWCols * 2 / 16;  // 16-byte chunks per row of a wave's block
  const int nr = min(G::kRB, ti.rows - wm * G::kRB);  // live rows of this wave
  const size_t pitch = KIND == kGateUp ? (size_t)a.Imax : (size_t)H;
  uint16_t *const out0 = (KIND == kGateUp ? a.act : a.y) + (size_t)(ti.slot0 + wm * G::kRB) * pitch + n0 + wn * kWCols;
#pragma unroll
  for (int i = 0; i < G::kRB * kCpr / 64; i++) {
    const int c = i * 64 + lane, r = c / kCpr, ch = c % kCpr;
    if (r < nr)
      *reinterpret_cast<uint4 *>(out0 + r * pitch + ch * 8) = *reinterpret_cast<const uint4 *>(wt + r * kWPitch + ch * 16);
  }
}

// --------------------------------------------------------------- combine

__global__ void __launch_bounds__(256) combine_kernel(const uint16_t *__restrict__ y, const int32_t *__restrict__ slot_of,
                                                      int T, int k, int H, int with_shared,
                                                      const float *resid, float *out) {
  const int t = blockIdx.x;
  auto add4 = [](float4 &acc, uint2 v) {  // four bf16 -> f32, in column order
    acc.x += bf16_to_f32(v.x & 0xffffu);
    acc.y += bf16_to_f32(v.x >> 16);
    acc.z += bf16_to_f32(v.y & 0xffffu);
    acc.w += bf16_to_f32(v.y >> 16);
  };
  for (int j = threadIdx.x * 4; j < H; j += 1024) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r = 0; r < k; r++)  // rank order, model/moe.go:82-84
      add4(acc, *reinterpret_cast<const uint2 *>(y + (size_t)slot_of[(size_t)t * k + r] * H + j));
    if (with_shared)  // added after the routed sum, model/moe.go:94-96
      add4(acc, *reinterpret_cast<const uint2 *>(y + ((size_t)T * k + t) * H + j));
    if (resid) {  // the residual add around the block, x += y (model/model.go:515-517)
      const float4 r = *reinterpret_cast<const float4 *>(resid + (size_t)t * H + j);
      acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    *reinterpret_cast<float4 *>(out + (size_t)t * H + j) = acc;
  }
}

// ------------------------------------------------------------- launchers

bool prefill_supported(int expert_fmt, int H, int I, int Is) {
  // bf16, int8 or int4 experts (the shared expert in any format: see
  // prefill_shared_fmt); whole column chunks (gate_up: 128 intermediate
  // columns, down: 256 outputs)
  if (expert_fmt != kBF16 && expert_fmt != kINT8 && expert_fmt != kINT4) return false;
  return H % kBN == 0 && I % (kBN / 2) == 0 && (Is == 0 || Is % (kBN / 2) == 0);
}

int prefill_shared_fmt(int shared_fmt) {
  return shared_fmt == kBF16 || shared_fmt == kINT8 || shared_fmt == kINT4 ? shared_fmt : kBF16;
}

int prefill_tile_slots(int expert_fmt) {
  switch (expert_fmt) {
  case kINT8: return GemmCfg<kINT8>::kBM;
  case kINT4: return GemmCfg<kINT4>::kBM;
  default: return GemmCfg<kBF16>::kBM;
  }
}

int prefill_max_tiles(int T, int k, int E, int bm) {
  const int n = T * k;
  return (n + bm - 1) / bm + (E < n ? E : n);
}

hipError_t launch_prefill_dispatch(const PrefillArgs &a, const int32_t *ids, const float *wts, const float *x,
                                   const float *shared_gate, float *sg, bool x_ready, hipStream_t st) {
  const bool with_shared = a.Is > 0;
  if (!x_ready || with_shared)
    QMOE_LAUNCH(prep_kernel, dim3(a.T), dim3(256), 0, st, x, a.H, with_shared ? shared_gate : nullptr, a.xb, sg);
  const int n = a.T * a.k;
#define L(J) QMOE_LAUNCH(dispatch_kernel<J>, dim3(1), dim3(kDispatchThreads), 0, st, ids, a.T, a.k, a.E, \
                         (int)with_shared, a.bm, a.bms, a.p)
  if (n <= 4 * kDispatchThreads) L(4);
  else if (n <= 16 * kDispatchThreads) L(16);
  else if (n <= 48 * kDispatchThreads) L(48);
  else L(0);
#undef L
  const int blocks = (n + kScatterPairs - 1) / kScatterPairs + (with_shared ? (a.T + 255) / 256 : 0);
  QMOE_LAUNCH(scatter_kernel, dim3(blocks), dim3(256), 0, st, ids, wts, sg, a.T, a.k, a.E, (int)with_shared, a.p);
  return hipGetLastError();
}

template <int KIND>
static hipError_t gemm_launch(const PrefillArgs &a, bool shared, int ny, hipStream_t st) {
  // the shared expert's GEMMs run in its own format, on tiles of its own size
  const int fmt = shared ? a.sfmt : a.fmt, bm = shared ? a.bms : a.bm;
  const int tiles = shared ? (a.T + bm - 1) / bm : prefill_max_tiles(a.T, a.k, a.E, bm);
  // a bf16 gate_up may split its last round: up to n_cu / 8 more workgroups per XCD
  const int halves = KIND == kGateUp ? a.n_cu / kXcds : 0;
  const int blocks = ((tiles + kXcds - 1) / kXcds * ny + halves) * kXcds;
  if (bm != prefill_tile_slots(fmt)) return hipErrorInvalidValue;
#define L(BF) QMOE_LAUNCH((grouped_gemm<KIND, BF>), dim3(blocks), dim3(kGemmThreads), 0, st, a, (int)shared, ny)
  switch (fmt) {
  case kBF16: L(kBF16); break;
  case kINT8: L(kINT8); break;
  case kINT4: L(kINT4); break;
  default: return hipErrorInvalidValue;
  }
#undef L
  return hipGetLastError();
}

hipError_t launch_prefill_gate_up(const PrefillArgs &a, bool shared, hipStream_t st) {
  return gemm_launch<kGateUp>(a, shared, (shared ? a.Is : a.I) / (kBN / 2), st);
}

hipError_t launch_prefill_down(const PrefillArgs &a, bool shared, hipStream_t st) {
  return gemm_launch<kDown>(a, shared, a.H / kBN, st);
}

hipError_t launch_prefill_combine(const PrefillArgs &a, float *out, hipStream_t st) {
  QMOE_LAUNCH(combine_kernel, dim3(a.T), dim3(256), 0, st, a.y, a.p.slot_of, a.T, a.k, a.H,
                     (int)(a.Is > 0), a.resid, out);
  return hipGetLastError();
}

}  // namespace qmoe
