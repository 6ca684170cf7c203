// kernels.hpp -- host-side launchers of the gfx950 MoE kernels (internal API
// between the kernel translation units and the C ABI in layer.hip).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmoe {

// Kernel timing for qmoe_profile_*: while a stage is profiled, the layer sets
// these to an event pair; the stage's launches then go through
// hipExtLaunchKernelGGL, which records `start` when its first kernel starts and
// `stop` when its last kernel ends -- the kernels' own execution time, without
// the dispatch gap that events recorded around the launch would add.
struct ProfEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local ProfEvents g_prof;

#define QMOE_LAUNCH(kernel, grid, block, lds, st, ...)                                              \
  do {                                                                                             \
    if (::qmoe::g_prof.stop) {                                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, st, ::qmoe::g_prof.start, ::qmoe::g_prof.stop, \
                            0, __VA_ARGS__);                                                       \
      ::qmoe::g_prof.start = nullptr;                                                              \
    } else {                                                                                       \
      hipLaunchKernelGGL(kernel, grid, block, lds, st, __VA_ARGS__);                               \
    }                                                                                              \
  } while (0)

// One stored weight matrix (or a stack of them) on the device.
struct DevMat {
  const uint8_t *w = nullptr;       // codes / elements
  const uint16_t *s = nullptr;      // fp16 scales (INT formats)
  int fmt = 0;
  int rows = 0, cols = 0;           // one matrix
  int64_t mat_bytes = 0;            // bytes per matrix in the stack
  int64_t mat_scales = 0;           // scales per matrix in the stack
  bool transposed = false;          // stored as the (cols, rows) transpose
};

// ---- router (router.hip) ----
// logits (T, E) = x (T, H) @ router^T, each logit one sequential f32 sum in
// h order with separate multiply and add roundings (model/tensors.go:77-89,
// model/model.go:167-176).  xb (T > 32 only; may be null): also store x
// rounded to bf16, (T, H), for the batched GEMMs.
hipError_t launch_router_logits(const float *x, int T, const DevMat &router, float *logits, uint16_t *xb,
                                hipStream_t st);
// Certified router partials for decode-sized T: sb (T, E, 2) f64 = {S, B}
// per (token, expert), S ~ exact sum of the reference's f32 products, B a
// bound on the reference's sequential rounding error.  zero_out (T, H), when
// given, is zeroed for the fused expert kernel.
bool router_certified_supported(const DevMat &router);
// The post-attention norm folded into launch_router_sb (w null: none): x is
// then the residual stream, the partials use its norm, and the normed tokens
// are stored into xn (T, H) for the expert kernel.
struct RouterNorm {
  const float *w = nullptr;
  float eps = 0.0f;
  int force_seq = 0;
  unsigned int *redo = nullptr;
  float *xn = nullptr;
};
hipError_t launch_router_sb(const float *x, int T, const DevMat &router, double *sb, float *zero_out,
                            const float *resid, const RouterNorm &norm,
                            hipStream_t st);
// Certified router partials for T > 32 on the matrix cores (bf16 router, H a
// multiple of 64, at most 8192): the same sb as launch_router_sb, from x split
// into exact bf16 parts inside the kernel.
bool router_cert_mfma_supported(const DevMat &router);
// fbl / qcnt (may be null): the exact queue of launch_select_candidates,
// cleared by this launch for the selection after it.
hipError_t launch_router_cert_mfma(const float *x, int T, const DevMat &router, double *sb, int *fbl,
                                   uint32_t *qcnt, hipStream_t st);
// Selection for T > 32 from the matrix-core partials (bf16 router): exact
// logits of the candidates the bounds leave, ranked; the exact path for the
// tokens whose ranks they cannot separate, queued in fbl (1 + T ints).
// Tokens the candidates cannot settle are queued in fbl and routed on the
// exact path, each split over several workgroups: qlt holds the logits of the
// first kExactQueueMax queued tokens, qcnt their workgroup counts.  fbl[0]
// and qcnt must be zero on entry (launch_router_cert_mfma clears them).
constexpr int kExactQueueMax = 64;
hipError_t launch_select_candidates(const float *x, int T, const DevMat &router, int k, int scope, const double *sb,
                                    int32_t *ids, float *weights, int *fbl, float *qlt, uint32_t *qcnt,
                                    unsigned int *fallbacks, hipStream_t st);
// Certified selection per token from sb, exact fallback on failure.
hipError_t launch_select_cert(const float *x, int T, const DevMat &router, int k, int scope, const double *sb,
                              int32_t *ids, float *weights, unsigned int *fallbacks, hipStream_t st);
// softmax (tensors.go:106-121) + selection over the first `scope` candidates
// + renormalisation (moe.go:44-57,63).  ids/weights (T, k).
hipError_t launch_softmax_select(const float *logits, int T, int E, int k, int scope,
                                 int32_t *ids, float *weights, hipStream_t st);

// ---- expert products (fused.hip) ----
// One kernel per forward; each block takes an equal share of a token's
// flattened intermediate rows (k*I routed + Is shared): its experts (from
// the router partials sb with certification, or from precomputed ids/weights
// when sb is null), gate_up + SwiGLU, and the matching rows of the transposed
// down matrix, accumulated into out with f32 atomics.  out must be zero on
// entry.  A launch covers the k_routed routed ranks and/or the shared expert.
struct FusedArgs {
  const float *x;
  int T, H, E, k, scope, I, Is;
  const uint8_t *rw;                  // router, for the exact fallback
  const uint16_t *rs;
  int rfmt;
  const double *sb;                   // router partials (T, E, 2), or null
  int fmt;                            // weight format of this launch
  const uint8_t *gu, *dn;             // gate_up (E, 2I, H); down transposed (E, I, H)
  const uint16_t *gu_s, *dn_s;        // scales (E, 2I, H/32) and (E, I/32, H)
  int64_t gu_bytes, gu_scales, dn_bytes, dn_scales;
  const uint8_t *sgate, *sup, *sdown; // shared: (Is, H), (Is, H), transposed down (Is, H)
  const uint16_t *sgate_s, *sup_s, *sdown_s;
  const float *shared_gate;
  int32_t *ids;                       // (T, k): written when sb is given, read otherwise
  float *weights;                     // (T, k)
  unsigned int *fallbacks;
  float *out;                         // (T, H), accumulated
  const float *resid;                 // (T, H) residual stream out starts from (null: 0); may be out
  int k_routed, with_shared;          // ranks of this launch
  int n_cu;                           // compute units of the device
  int nb, rb;                         // filled by the launcher: blocks per token, rows per block
  int burst;                          // filled by the launcher: LDS holds the burst-mode down rows
  uint64_t rank_gap;                  // filled by the launcher: s_memrealtime ticks between ranks' bursts
  // T = 1, bf16 router: the kernel computes the router partials itself
  // (fused_router = router chunks per lane, 1, 2 or 4; sb null), exchanges
  // them between its workgroups through rtag (one word per expert) tagged with
  // epoch (1..255, a new value every call) and zeroes out itself, each
  // workgroup a slice, announced in ztag (one word per workgroup, at most
  // kMaxExchangeBlocks).  Every wait for those words gives up after
  // xchg_ticks s_memrealtime ticks (100 MHz; 0: at once), sets xchg_err
  // (host-visible) and finishes the workgroup on the exact routing path.
  int fused_router;
  uint64_t *rtag;
  uint32_t *ztag;
  uint32_t epoch;
  int *xchg_err;
  uint64_t xchg_ticks;
  int *occ_out;                       // internal: occupancy query instead of a launch
  // T = 1 with fused_router: x is the residual stream, normalised in the
  // kernel's prologue with norm_w (H) and norm_eps (null: x is the input)
  const float *norm_w;
  float norm_eps;
  int norm_force_seq;
  unsigned int *norm_redo;
};
constexpr int kMaxExchangeBlocks = 4096;
// Default wait for the exchanged words: 2 ms.  They normally arrive within a
// few microseconds; a device that does not run every workgroup of the launch
// at once would otherwise leave the waiting workgroups spinning.
constexpr uint64_t kExchangeTicks = 200000;
hipError_t launch_expert_fused(const FusedArgs &a, hipStream_t st);
// Workgroups of the expert kernel's launch for these arguments, and in
// *resident how many of its workgroups the device holds at once: the
// in-kernel router exchange needs every workgroup resident.
int fused_exchange_blocks(const FusedArgs &a, int *resident);
bool fused_supported(int fmt, int H, int E);  // the LDS plan fits
hipError_t launch_zero(float *p, int64_t n, hipStream_t st);

// ---- post-attention norm (norm.hip) ----
// xn (T, n) = gemmaRMSNormApply(x, w, eps) per token (model/tensors.go:147-157),
// bit for bit; redo (may be null) counts tokens whose certified sum of squares
// had to be recomputed in index order (every token when force_seq).
hipError_t launch_gemma_norm(const float *x, int T, int n, const float *w, float eps, float *xn, unsigned int *redo,
                             bool force_seq, hipStream_t st);
// dst (n floats) = src; nothing when they are the same.
hipError_t launch_copy(const float *src, float *dst, int64_t n, hipStream_t st);

// ---- prefill: dispatch, grouped MFMA GEMMs, combine (prefill.hip) ----
// Slots: the T*k (token, rank) pairs grouped by expert, then the shared
// expert's T slots (group E) in token order.
struct PrefillPlan {
  int32_t *tok;                 // (slots) token of each slot
  float *wslot;                 // (slots) routing weight, or the shared gate
  int32_t *slot_of;             // (T, k) slot of each (token, rank)
  int32_t *grp_off, *grp_cnt;   // (E + 1) first slot and slot count per group
  int32_t *cursor;              // (E) next free slot per expert while scattering
  int32_t *tile_grp, *tile_m0;  // tile table: group and first row of each tile
  int32_t *n_tiles;             // [0] routed tiles, [1] shared tiles (after the routed ones)
};
struct PrefillArgs {
  int T, H, E, k, I, Is, Imax;  // Imax = max(I, Is), the row pitch of act
  int fmt;                      // routed experts' weight format: BF16, INT8 or INT4
  int bm;                       // slots per routed tile, prefill_tile_slots(fmt)
  int sfmt;                     // the shared expert's batched format, prefill_shared_fmt
  int bms;                      // slots per shared tile, prefill_tile_slots(sfmt)
  int n_cu;                     // compute units of the device (8 XCDs)
  uint16_t *xb;                 // (T, H) x in bf16
  PrefillPlan p;
  const uint8_t *gu, *dn;       // gate_up (E, 2I, H); down in the reference layout (E, H, I)
  const uint16_t *gu_s, *dn_s;  // scales (E, 2I, H/32) and (E, H, I/32)
  int64_t gu_bytes, gu_scales, dn_bytes, dn_scales;
  const uint8_t *sgate, *sup, *sdown;  // shared: (Is, H), (Is, H), down (H, Is)
  const uint16_t *sgate_s, *sup_s, *sdown_s;
  uint16_t *act;                // (slots, Imax) SwiGLU output, bf16
  uint16_t *y;                  // (slots, H) weighted expert outputs, bf16
  const float *resid;           // (T, H) added to the combined output (null: none); may be out
};
bool prefill_supported(int expert_fmt, int H, int I, int Is);
// The format the batched path keeps the shared expert in: its own when the
// GEMMs take it (bf16, int8, int4), else bf16 (an f32 shared expert is
// rounded to bf16, as the GEMMs round every dequantised weight).
int prefill_shared_fmt(int shared_fmt);
int prefill_tile_slots(int expert_fmt);              // slots per GEMM tile for the format
int prefill_max_tiles(int T, int k, int E, int bm);  // routed tiles, upper bound
// x_ready: a.xb already holds x in bf16 (the exact router stored it); the
// prep launch then runs only for the shared gate.
hipError_t launch_prefill_dispatch(const PrefillArgs &a, const int32_t *ids, const float *wts, const float *x,
                                   const float *shared_gate, float *sg, bool x_ready, hipStream_t st);
hipError_t launch_prefill_gate_up(const PrefillArgs &a, bool shared, hipStream_t st);
hipError_t launch_prefill_down(const PrefillArgs &a, bool shared, hipStream_t st);
hipError_t launch_prefill_combine(const PrefillArgs &a, float *out, hipStream_t st);

// ---- quantiser / dequantiser (quant.hip) ----
hipError_t launch_quantize(int bits, const float *w, int64_t n_rows, int cols, uint8_t *codes,
                           uint16_t *scales, hipStream_t st);
hipError_t launch_dequantize(const DevMat &m, int64_t index, float *out, hipStream_t st);
// quantLinear.dequantize with f32 scales (rows of cols elements, codes int8 or
// packed int4) into f32: the storage of the group-32 formats with f32 scales.
hipError_t launch_dequant_f32s(int bits, const uint8_t *codes, const float *scales, int64_t n_rows, int cols,
                               float *out, hipStream_t st);
// f32 -> bf16 (round to nearest even): the batched path's copy of an f32
// shared expert.
hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t st);
// (rows, cols) reference-layout stack -> (cols, rows) transposes, codes and
// scales moved unchanged (INT4 re-paired along the new rows).
hipError_t launch_relayout_transpose(int fmt, const uint8_t *src, const uint16_t *ss, int64_t n_mat, int rows,
                                     int cols, uint8_t *dst, uint16_t *ds, hipStream_t st);

// ---- dense projection and greedy token (linear.hip) ----
// y (T, rows) = x (T, cols) @ W^T with W (rows, cols) in f32, bf16, int8 or
// int4 group-32 (fp16 scales), each output the sequential f32 sum of
// linear.matvec / matmulVec / quantLinear.forward (model/model.go:131-176,
// model/tensors.go:77-89, model/moe.go:159-162).  W is held in the lane-stream
// layout that launch_linear_relayout writes (linear_stream_bytes bytes).
// The GEMV's formats: the Fmt values plus the group-32 formats with f32
// scales (the qmoe_format numbers QMOE_INT8G32_F32S / QMOE_INT4G32_F32S),
// kept as codes + f32 scales.
constexpr int kLinI8F32S = 4, kLinI4F32S = 5;
struct LinMat {
  const uint8_t *w = nullptr;
  int fmt = 0, rows = 0, cols = 0;
  int n_cu = 256;  // compute units of the device (launch shape)
};
int linear_step(int fmt);  // cols must be a multiple of it (32 f32, 64 bf16, 256 for the group-32 formats)
bool linear_supported(int fmt, int cols);  // also cols <= 40960 (x of a token in LDS)
int linear_tokens_per_pass(int T, int cols);  // a launch covers T in passes of this many tokens
int64_t linear_stream_bytes(int fmt, int rows, int cols);
// ss: fp16 scale bits (int8/int4) or f32 scales (the f32-scale formats), (rows, cols / 32)
hipError_t launch_linear_relayout(int fmt, const uint8_t *src, const void *ss, int rows, int cols, void *dst,
                                  hipStream_t st);
hipError_t launch_linear(const float *x, int T, const LinMat &m, float *y, hipStream_t st);
// argmax of each row of v (T, n) with model.go:652-660's semantics; pv/pi
// hold T * argmax_partials(n) pairs.
int argmax_partials(int n);
hipError_t launch_argmax(const float *v, int T, int n, float *pv, int *pi, int32_t *out, hipStream_t st);

}  // namespace qmoe
