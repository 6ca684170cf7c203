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
// softmax (tensors.go:106-121) + selection over the first `scope` candidates
// + renormalisation (moe.go:44-57,63).  ids/weights (T, k).
hipError_t launch_softmax_select(const float *logits, int T, int E, int k, int scope,
                                 int32_t *ids, float *weights, hipStream_t st);

// ---- bandwidth-bound expert GEMVs (gemv.hip) ----
// act[p, o] = silu(gate_e[o] . x_t) * (up_e[o] . x_t) for p = t*k + r, e = ids[p]
// (moe.go:64-75).  With ids == nullptr the matrix is a single (shared) expert
// and k must be 1.  gate / up are the gate rows and the up rows of the stack:
// for stacked experts up = gate + I rows.
struct GateUpArgs {
  const float *x;
  const int32_t *ids;
  int T, k, H, I;
  const uint8_t *gate, *up;           // row 0 of expert 0
  const uint16_t *gate_s, *up_s;
  int64_t expert_bytes, expert_scales;  // stride between experts
  int fmt;
  float *act;                         // (T*k, I)
  const float *shared_gate;           // optional (H): writes sg[t] = sigmoid(x_t . shared_gate)
  float *sg;
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

// ---- quantiser / dequantiser (quant.hip) ----
hipError_t launch_quantize(int bits, const float *w, int64_t n_rows, int cols, uint8_t *codes,
                           uint16_t *scales, hipStream_t st);
hipError_t launch_dequantize(const DevMat &m, int64_t index, float *out, hipStream_t st);

}  // namespace qmoe
