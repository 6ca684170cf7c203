/*
 * qmoe.h -- C ABI of the MI355X (gfx950) MoE block that replaces the body of
 * qwen-go's moeMLP.forward.
 *
 * The ABI is plain C: handles, host or device pointers, sizes and a status
 * code.  It carries no HIP or torch types, so a cgo shim can bind it directly.
 * Citations are to the qwen-go source tree (file:line).
 *
 * Layouts (row-major, identical to the reference's safetensors layout):
 *   router      (E, H)                        model/load.go:419 (mlp.gate.weight)
 *   gate_up     (E, 2I, H), rows [0,I) gate    model/moe.go:12,59,70-71
 *               and rows [I,2I) up
 *   down        (E, H, I)                      model/moe.go:13,60
 *   shared gate/up (Is, H), down (H, Is)       model/model.go:339-358
 *   shared_gate (H) f32                        model/moe.go:18,89-93
 * Formats (qmoe_format):
 *   QMOE_F32      float32 elements
 *   QMOE_BF16     uint16 bf16 bit patterns (model/model.go:113-115)
 *   QMOE_INT8G32  int8 codes (rows, K) + fp16 scales (rows, K/32)
 *   QMOE_INT4G32  packed bytes (rows, K/2), high nibble = even element,
 *                 value = nibble - 8, + fp16 scales (rows, K/32)
 *                 (model/moe.go:134-157; scales are the fp16 form that
 *                 safetensors F16 files hold, widened exactly)
 *   QMOE_INT8G32_F32S, QMOE_INT4G32_F32S
 *                 the same codes with f32 scales (rows, K/32): the
 *                 quantLinear the loader builds from qwen-quant output, which
 *                 writes its scales as F32 (cmd/qwen-quant/main.go:198-210,
 *                 model/load.go:527-582).  Stored on the device as their exact
 *                 f32 dequantisation float32(code) * scale (moe.go:134-157),
 *                 which is what quantLinear.forward multiplies with
 *                 (moe.go:159-162); 4 bytes per weight on the device.
 * For stacked experts the scale arrays are (E, rows, K/32).
 *
 * Threading: every call on one handle is serialised by a per-handle mutex, so
 * concurrent Generate goroutines may share a handle.  qmoe_forward_device is
 * asynchronous on the caller's stream and uses the handle's workspace: calls on
 * one handle must be ordered on one stream (or synchronised by the caller).
 */
#ifndef QMOE_H
#define QMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QMOE_OK = 0,
    QMOE_ERR_INVALID = 1,     /* bad argument: null pointer, dims, T < 0, format */
    QMOE_ERR_STATE = 2,       /* weights not uploaded, or handle destroyed */
    QMOE_ERR_NOMEM = 3,       /* device allocation failed */
    QMOE_ERR_HIP = 4,         /* HIP runtime error (message in qmoe_last_error) */
    QMOE_ERR_UNSUPPORTED = 5  /* valid but not supported (e.g. E > 1024) */
} qmoe_status;

typedef enum {
    QMOE_F32 = 0,
    QMOE_BF16 = 1,
    QMOE_INT8G32 = 2,
    QMOE_INT4G32 = 3,
    QMOE_INT8G32_F32S = 4,
    QMOE_INT4G32_F32S = 5
} qmoe_format;

/* Layer description.  Field meanings follow model/config.go:24-27 and
 * moeMLP (model/moe.go:10-25). */
typedef struct {
    int32_t hidden;        /* H, nEmbed */
    int32_t n_experts;     /* E, NExperts */
    int32_t top_k;         /* k, NExpertsPerToken */
    int32_t moe_inter;     /* I, NMoeMlp */
    int32_t shared_inter;  /* Is, NSharedExpertMlp; 0 = no shared expert */
    int32_t select_scope;  /* C in [k, E]: stable-sort the first C probabilities and
                              take the first k.  0 or k = model/moe.go:45-53 as
                              written (always experts {0..k-1}, ordered by p);
                              E = true top-k, ties to the lowest index */
    int32_t router_fmt;    /* qmoe_format of the router (E, H) */
    int32_t expert_fmt;    /* qmoe_format of the stacked experts */
    int32_t shared_fmt;    /* qmoe_format of the shared expert projections */
    int32_t device;        /* HIP device ordinal */
} qmoe_desc;

typedef struct qmoe_layer qmoe_layer;

/* newMoeMLP (model/moe.go:27-39): validates the description and allocates the
 * device weight arrays.  Quantised formats need H and I (and Is) % 32 == 0. */
qmoe_status qmoe_create(const qmoe_desc *desc, qmoe_layer **out);

/* Releases device memory.  Safe on NULL; a handle must not be used after it. */
void qmoe_destroy(qmoe_layer *layer);

/* Message of the last failing call on this handle (or of the last failing
 * qmoe_create on this thread when layer is NULL).  Never NULL. */
const char *qmoe_last_error(const qmoe_layer *layer);
const char *qmoe_status_string(qmoe_status s);

/* Weight upload from host memory (copied, not retained), as the loader's
 * loadMLP / installQuant fill moeMLP (model/load.go:415-459, 646-664):
 * router = mlp.gate (or routerQuant), experts = the stacked gate_up/down,
 * shared = shared.{gate,up,down} (or their gateQuant/upQuant/downQuant) and
 * sharedGate.  scales: fp16 bit patterns (uint16) for QMOE_INT8G32 and
 * QMOE_INT4G32, float32 for the *_F32S formats, ignored otherwise. */
qmoe_status qmoe_set_router(qmoe_layer *layer, const void *w, const void *scales);
qmoe_status qmoe_set_experts(qmoe_layer *layer, const void *gate_up, const void *gate_up_scales,
                             const void *down, const void *down_scales);
qmoe_status qmoe_set_shared(qmoe_layer *layer, const void *gate, const void *gate_scales,
                            const void *up, const void *up_scales, const void *down,
                            const void *down_scales, const float *shared_gate);

/* Quantises f32 expert weights on the device into the layer's INT8G32 or
 * INT4G32 expert format: quantizeInt8 / quantizeInt4 (model/moe.go:165-217)
 * per (rows, K) matrix, then the f32 scale rounded to fp16 (nearest-even).
 * Codes are computed from the unrounded f32 scale, as the reference does.
 * gate_up (E, 2I, H) and down (E, H, I) f32 host arrays. */
qmoe_status qmoe_quantize_experts(qmoe_layer *layer, const float *gate_up, const float *down);

/* Device-pointer quantiser used by qmoe_quantize_experts: n_mat stacked
 * (rows, cols) f32 matrices -> codes (int8 (rows,cols) or packed int4
 * (rows,cols/2)) and fp16 scales (rows, cols/32).  bits = 8 or 4.
 * Asynchronous on stream (hipStream_t; NULL = default stream). */
qmoe_status qmoe_quantize_device(int32_t bits, const float *d_w, int64_t n_mat, int32_t rows,
                                 int32_t cols, void *d_codes, uint16_t *d_scales, void *stream);

/* moeMLP.forward (model/moe.go:41-99) for T tokens, host pointers, synchronous.
 * x (T, H) f32 in; out (T, H) f32 out.  ids (T, k) int32 and weights (T, k) f32
 * receive the selected experts and renormalised routing weights in rank
 * order; either may be NULL.  T == 0 is a no-op.  The Go seam calls it with
 * T = 1 (model/model.go:508-514).
 * Precision: ids are the reference's exactly; the routing weights are within
 * 1e-4 relative of the reference's f32 softmax on the decode path (T <= 32:
 * computed from the certified f64 partial sums) and within 1e-6 on the
 * batched path (the reference's f32 softmax of the exact logits); out is
 * within 1e-3 (decode) / 2e-2 (batched, bf16 matrix cores) normwise per token.
 * At T = 1 the expert kernel's workgroups exchange the router partials among
 * themselves; if that exchange times out (the device did not run them all at
 * once) this call returns QMOE_ERR_HIP and its outputs are not valid. */
qmoe_status qmoe_forward(qmoe_layer *layer, const float *x, int32_t T, float *out, int32_t *ids,
                         float *weights);

/* Same, on device pointers, asynchronous on stream (hipStream_t; NULL = the
 * default stream).  No host synchronisation, so an exchange timeout of this
 * call is reported by the next call on the handle (which then returns
 * QMOE_ERR_HIP without running); the report clears it. */
qmoe_status qmoe_forward_device(qmoe_layer *layer, const float *d_x, int32_t T, float *d_out,
                                int32_t *d_ids, float *d_weights, void *stream);

/* ---- the block with its neighbours (model/model.go:506-517) ----
 * decodeLayers normalises a copy of each token of the residual stream with the
 * layer's post-attention GemmaRMSNorm (gemmaRMSNormApply, model/tensors.go:
 * 147-157), runs the MoE block on it and adds the result back:
 *   x[t] += moeMLP.forward(gemmaRMSNorm(x[t], w, eps)).
 * qmoe_set_post_norm uploads w (H) f32 (postAttentionLayernorm) and eps
 * (float32(RmsNormEps)); the norm is computed bit for bit as the reference
 * does (its f64 sum of squares certified, or redone in index order).  The
 * residual add is folded into the block's output (out starts from x), so the
 * normed copy and the block's own output never make a round trip. */
qmoe_status qmoe_set_post_norm(qmoe_layer *layer, const float *w, float eps);
/* x (T, H) f32 host pointer, updated in place; ids / weights as qmoe_forward.
 * Synchronous. */
qmoe_status qmoe_forward_residual(qmoe_layer *layer, float *x, int32_t T, int32_t *ids, float *weights);
/* Device pointers, asynchronous on stream: d_out = d_x + block(norm(d_x));
 * d_out may be d_x (in place). */
qmoe_status qmoe_forward_residual_device(qmoe_layer *layer, const float *d_x, int32_t T, float *d_out,
                                         int32_t *d_ids, float *d_weights, void *stream);
/* Tokens whose norm recomputed its sum of squares in index order (the
 * certification did not settle the f32 rounding), since create. */
qmoe_status qmoe_norm_recomputes(qmoe_layer *layer, int64_t *count);
/* The norm alone on host pointers, x (T, H) -> xn (T, H): for bit-exact tests. */
qmoe_status qmoe_norm_debug(qmoe_layer *layer, const float *x, int32_t T, float *xn);
/* on != 0: every norm takes the index-order path (tests of that path). */
qmoe_status qmoe_debug_norm_sequential(qmoe_layer *layer, int32_t on);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  qmoe_forward_device for decode-sized batches, T <= 32,
 * with no allocation of any kind: the kernels' scratch (router partials and
 * logits, ids and weights, the exact-path queue; at most 1 MiB for E <= 1024,
 * k <= 64) lives in a static device array that each device holds until the
 * process ends.  Larger T returns QMOE_ERR_UNSUPPORTED.  Every call on one
 * device shares that array, so calls that overlap on a device (different
 * handles on streams that are not ordered) race; order them on one stream.
 * No profiling events are recorded by this entry. */
qmoe_status qmoe_forward_device_noalloc(qmoe_layer *layer, const float *d_x, int32_t T, float *d_out,
                                        int32_t *d_ids, float *d_weights, void *stream);

/* Exact f32 copy of a stored weight matrix, dequantised on the device as
 * quantLinear.dequantize does (model/moe.go:134-157); bf16 widened as bf16f32.
 * which: 0 expert gate_up (2I, H), 1 expert down (H, I), 2 router (E, H),
 *        3 shared gate (Is, H), 4 shared up (Is, H), 5 shared down (H, Is).
 * expert is ignored for which >= 2.  out is a host array of rows*cols f32. */
qmoe_status qmoe_dequant_debug(qmoe_layer *layer, int32_t which, int32_t expert, float *out);

/* Kernel stages of one forward, for qmoe_profile_*. */
enum {
    QMOE_STAGE_ROUTER = 0,         /* router logits */
    QMOE_STAGE_SELECT = 1,         /* softmax + selection + renormalisation */
    QMOE_STAGE_GATE_UP = 2,        /* batched: routed experts gate_up + SwiGLU (MFMA) */
    QMOE_STAGE_SHARED_GATE_UP = 3, /* batched: shared expert gate_up + SwiGLU (MFMA) */
    QMOE_STAGE_DOWN = 4,           /* batched: down of routed and shared experts (MFMA) */
    QMOE_STAGE_FUSED = 5,          /* decode: routing + gate_up + down in one kernel */
    QMOE_STAGE_DISPATCH = 6,       /* batched: x to bf16, shared gate, per-expert token lists */
    QMOE_STAGE_COMBINE = 7,        /* batched: rank-order sum of the expert outputs + shared */
    QMOE_STAGE_COUNT = 8
};

/* Which kernels a forward of T tokens runs, with no reference counterpart
 * (the reference has one CPU path):
 *   QMOE_PATH_GEMV  decode kernels, f32 activations and accumulation (parity
 *                   bar 1e-3 normwise against model/moe.go);
 *   QMOE_PATH_MFMA  dispatch + grouped GEMMs on bf16 MFMA with f32
 *                   accumulation, x and the SwiGLU output rounded to bf16
 *                   (parity bar 2e-2 normwise).
 * The router and the selection are exact on both paths, so expert ids always
 * match the reference bit for bit.  Returns -1 for a null handle. */
enum { QMOE_PATH_GEMV = 0, QMOE_PATH_MFMA = 1 };
int32_t qmoe_forward_path(const qmoe_layer *layer, int32_t T);

/* Instrumentation with no reference counterpart (the reference has no
 * timers): when bit s of stage_mask is set, every later forward records a HIP
 * event pair on its stream around stage s's kernel launch.  qmoe_profile_read
 * waits for the recorded events and returns the summed milliseconds and the
 * launch count per stage (arrays of QMOE_STAGE_COUNT); reset != 0 zeroes the
 * totals.  Events are released back to the handle's pool on each read, so read
 * at least every few thousand forwards. */
qmoe_status qmoe_profile_enable(qmoe_layer *layer, uint32_t stage_mask);
qmoe_status qmoe_profile_read(qmoe_layer *layer, double *stage_ms, int64_t *stage_launches,
                              int32_t reset);

/* Diagnostics with no reference counterpart: the number of tokens, since
 * qmoe_create, whose routing the certified decode router could not certify
 * (a near or exact tie within its rounding bound) and therefore recomputed
 * with the exact sequential path.  Synchronises the device. */
qmoe_status qmoe_router_fallbacks(qmoe_layer *layer, int64_t *count);

/* Diagnostics with no reference counterpart: the certified router's partials
 * for tokens x (host, T x hidden f32) -- sb_out (host, T x n_experts x 2
 * doubles) receives {S, B} per (token, expert), where the reference's f32
 * logit is guaranteed to lie in [S - B, S + B].  T <= 32: the decode router
 * (S: the f64 sum of the f32 products; B: the bound on the sequential f32
 * sum).  T > 32: the matrix-core router (bf16 router, hidden a multiple of 64
 * and at most 8192; S: f32 block sums of exact bf16 pieces of x; B also
 * bounds their roundings), which forward uses when T x n_experts >= 2^20.
 * QMOE_ERR_UNSUPPORTED for a router format or size neither takes.
 * Synchronises the device. */
qmoe_status qmoe_router_bounds_debug(qmoe_layer *layer, const float *x, int32_t T, double *sb_out);

/* Diagnostics with no reference counterpart: the number of tokens, since
 * qmoe_create, whose certification failed at first and succeeded once the
 * few candidates in doubt had their exact sequential logits computed (no
 * full exact routing needed).  Synchronises the device. */
qmoe_status qmoe_router_rescues(qmoe_layer *layer, int64_t *count);

/* Diagnostics with no reference counterpart: the longest wait of the T = 1
 * expert kernel's workgroups for each other's router partials, in ticks of
 * the device's 100 MHz real-time counter (ticks < 0: the default, 2 ms;
 * 0: give up at once).  A wait that gives up makes the call fail with
 * QMOE_ERR_HIP, and every workgroup still finishes (on exact routing).  For
 * tests of that error path. */
qmoe_status qmoe_debug_exchange_budget(qmoe_layer *layer, int64_t ticks);

/* No counterpart in the reference: sizes the handle's workspace for calls of
 * up to max_T tokens now (longer prompts run in chunks of at most
 * 65535 / top_k tokens, so larger values are capped there), so that no later
 * call allocates device memory -- e.g. at load, with the longest prompt a
 * server accepts.  Calls with more tokens still grow it. */
qmoe_status qmoe_reserve(qmoe_layer *layer, int32_t max_T);

/* Bytes of device memory held by the handle (weights + workspace). */
int64_t qmoe_device_bytes(const qmoe_layer *layer);

/* ---- dense projection: linear / quantLinear on the device ----
 * One (out_dim, in_dim) weight matrix W, y = x @ W^T for T tokens, each output
 * the reference's sequential f32 sum fl(s + fl(x[k] * w[k])) in k order --
 * bit for bit.  It replaces linear.matvec / mat2D / proj
 * (model/model.go:131-205) and quantLinear.forward (model/moe.go:159-162)
 * for the dense MLP projections (model.go:350-358) and the LM head
 * (model.go:519-525, tied: the embedding matrix).  Formats as above; every
 * group-32 format keeps its codes and its own scales (fp16, or the f32 scales
 * of qwen-quant's projections), each weight dequantised in the kernel as
 * float32(code) * scale exactly as quantLinear.dequantize does.  in_dim must
 * be a multiple of 32 (f32), 64 (bf16) or 256 (the group-32 formats) and at
 * most 40960; other shapes return QMOE_ERR_UNSUPPORTED.  The device copy is
 * rearranged at upload for the GEMV (64-row blocks; the same bytes plus
 * padding to a multiple of 64 rows).  Same threading rules as qmoe_layer. */
typedef struct qmoe_linear qmoe_linear;

qmoe_status qmoe_linear_create(int32_t out_dim, int32_t in_dim, int32_t fmt, int32_t device, qmoe_linear **out);
void qmoe_linear_destroy(qmoe_linear *lin);
/* Message of the last failing call on lin (NULL: the last failing
 * qmoe_linear_create on this thread).  Never NULL. */
const char *qmoe_linear_last_error(const qmoe_linear *lin);
/* W (out_dim, in_dim) in the handle's format from host memory (copied). */
qmoe_status qmoe_linear_set(qmoe_linear *lin, const void *w, const void *scales);
/* y (T, out_dim) = x (T, in_dim) @ W^T, host pointers, synchronous. */
qmoe_status qmoe_linear_forward(qmoe_linear *lin, const float *x, int32_t T, float *y);
/* The same on device pointers, asynchronous on stream (NULL: the default
 * stream); no workspace. */
qmoe_status qmoe_linear_forward_device(qmoe_linear *lin, const float *d_x, int32_t T, float *d_y, void *stream);
/* Greedy decode's next token (model.go:519-525 then argmax model.go:652-660)
 * for T rows: token[t] = argmax_j (x[t] @ W^T)[j], host pointers, synchronous;
 * logits (T, out_dim) is also written when non-NULL. */
qmoe_status qmoe_linear_greedy(qmoe_linear *lin, const float *x, int32_t T, int32_t *token, float *logits);
/* argmax of each row of d_v (T, n), model.go:652-660: the first index of the
 * maximum over the non-NaN entries, 0 when v[0] is NaN or there is none.
 * Device pointers, asynchronous on stream; uses lin's workspace. */
qmoe_status qmoe_linear_argmax_device(qmoe_linear *lin, const float *d_v, int32_t T, int32_t n, int32_t *d_token,
                                      void *stream);
int64_t qmoe_linear_device_bytes(const qmoe_linear *lin);

#ifdef __cplusplus
}
#endif
#endif
