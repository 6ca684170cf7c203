// kernels.hpp -- host-side launchers of the gfx950 MoE kernels (internal API
// between the kernel translation units and the C ABI in layer.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmoe {

// One stored weight matrix (or a stack of them) on the device.
struct DevMat {
  const uint8_t *w = nullptr;       // codes / elements
  const uint16_t *s = nullptr;      // fp16 scales (INT formats)
  int fmt = 0;
  int rows = 0, cols = 0;           // one matrix
  int64_t mat_bytes = 0;            // bytes per matrix in the stack
  int64_t mat_scales = 0;           // scales per matrix in the stack
};

// ---- router (router.hip) ----
// logits (T, E) = x (T, H) @ router^T, each logit one sequential f32 sum in
// h order with separate multiply and add roundings (model/tensors.go:77-89,
// model/model.go:167-176).
hipError_t launch_router_logits(const float *x, int T, const DevMat &router, float *logits,
                                hipStream_t st);
// Certified router partials for decode-sized T: sb (T, E, 2) f64 = {S, B}
// per (token, expert), S ~ exact sum of the reference's f32 products, B a
// bound on the reference's sequential rounding error.  zero_out (T, H), when
// given, is zeroed for the fused expert kernel.
bool router_certified_supported(const DevMat &router);
hipError_t launch_router_sb(const float *x, int T, const DevMat &router, double *sb, float *zero_out,
                            hipStream_t st);
// Certified selection per token from sb, exact fallback on failure.
hipError_t launch_select_cert(const float *x, int T, const DevMat &router, int k, int scope, const double *sb,
                              int32_t *ids, float *weights, unsigned int *fallbacks, hipStream_t st);
// softmax (tensors.go:106-121) + selection over the first `scope` candidates
// + renormalisation (moe.go:44-57,63).  ids/weights (T, k).
hipError_t launch_softmax_select(const float *logits, int T, int E, int k, int scope,
                                 int32_t *ids, float *weights, hipStream_t st);

// ---- bandwidth-bound expert GEMVs (gemv.hip) ----
// act[t*k + r, o] = silu(gate_e[o] . x_t) * (up_e[o] . x_t), e = ids[t*k + r]
// (moe.go:64-75); gate rows are rows [0,I) of the stacked (E, 2I, H) gate_up
// and up rows are rows [I,2I).  With Is > 0 the shared expert is computed in
// the same launch: act_s[t, o] and sg[t] = sigmoid(x_t . shared_gate).
struct GateUpArgs {
  const float *x;
  const int32_t *ids;
  int T, k, H, I;
  const uint8_t *gate;                // row 0 of expert 0 of the stack
  const uint16_t *gate_s;
  int64_t expert_bytes, expert_scales;  // stride between experts
  int fmt;
  float *act;                         // (T*k, I)
  // shared expert (Is == 0: none)
  int Is;
  const uint8_t *sgate, *sup;
  const uint16_t *sgate_s, *sup_s;
  int sfmt;
  float *act_s;                       // (T, Is)
  const float *shared_gate;           // (H)
  float *sg;                          // (T)
};
hipError_t launch_gate_up_gemv(const GateUpArgs &a, hipStream_t st);

// out[t, j] = sum_r w[t,r] * (down_{e_r}[j] . act[t*k+r])  (rank order)
//             + sg[t] * (shared_down[j] . act_s[t])        (moe.go:76-97)
struct DownArgs {
  const float *act;                   // (T*k, I)
  const int32_t *ids;
  const float *weights;               // (T*k)
  int T, k, H, I;
  const uint8_t *down;
  const uint16_t *down_s;
  int64_t expert_bytes, expert_scales;
  int fmt;
  // shared expert (Is == 0: none)
  const float *act_s;                 // (T, Is)
  const float *sg;                    // (T)
  int Is;
  const uint8_t *sdown;
  const uint16_t *sdown_s;
  int sfmt;
  float *out;                         // (T, H)
};
hipError_t launch_down_gemv(const DownArgs &a, hipStream_t st);

// ---- fused decode path (fused.hip) ----
// Per (token, rank, 32 intermediate rows): routing from the router partials,
// gate_up + SwiGLU, and the matching down columns accumulated into out with
// f32 atomics.  out must be zero on entry (launch_router_sb zeroes it).  The
// shared expert must use the routed experts' format.
struct FusedArgs {
  const float *x;
  int T, H, E, k, scope, I, Is;
  const uint8_t *rw;                  // router, for the exact fallback
  const uint16_t *rs;
  int rfmt;
  const double *sb;                   // router partials (T, E, 2)
  int fmt;
  const uint8_t *gu, *dn;
  const uint16_t *gu_s, *dn_s;
  int64_t gu_bytes, gu_scales, dn_bytes, dn_scales;
  const uint8_t *sgate, *sup, *sdown;
  const uint16_t *sgate_s, *sup_s, *sdown_s;
  const float *shared_gate;
  int32_t *ids;                       // (T, k) out
  float *weights;                     // (T, k) out
  unsigned int *fallbacks;
  float *out;                         // (T, H), accumulated
  int ng, ranks;                      // filled by the launcher
};
hipError_t launch_expert_fused(const FusedArgs &a, hipStream_t st);
constexpr int kFusedMaxT = 8;

// ---- quantiser / dequantiser (quant.hip) ----
hipError_t launch_quantize(int bits, const float *w, int64_t n_rows, int cols, uint8_t *codes,
                           uint16_t *scales, hipStream_t st);
hipError_t launch_dequantize(const DevMat &m, int64_t index, float *out, hipStream_t st);

}  // namespace qmoe
