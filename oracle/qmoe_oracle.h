/*
 * qmoe_oracle.h -- CPU restatement of qwen-go's MoE block (model/moe.go).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in qwen-go_amd/ and the CPU baseline timed beside it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product (libqmoe.so) never links, loads or calls it.
 *
 * Every function follows the reference's loop order and f32 rounding: plain
 * f32 multiplies and adds, no FMA contraction (built with -ffp-contract=off,
 * matching Go on amd64 at GOAMD64=v1), exp evaluated in double and rounded to
 * f32 exactly as the Go code writes float32(math.Exp(float64(v))).
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   orc_f16_to_f32        all 65536 bit patterns vs numpy float16->float32
 *   orc_f32_to_f16_rne    random + edge values vs numpy astype(float16)
 *   orc_bf16_to_f32 / orc_f32_to_bf16_rne   vs torch bfloat16 conversions
 *   orc_quantize_int8/4   hand-computed known answers (incl. a half-way
 *                         rounding case), round-trip bound |w-dq| <= s/2,
 *                         code ranges, amax element -> +-127 / +-7
 *   orc_dequantize        known bytes (0x81 -> -127*s, 0x9F -> (+1,+7)*s)
 *   orc_matvec            numpy float32 scalar loop (pins no-FMA order) and
 *                         numpy float64 within the f32 error bound
 *   orc_softmax           known answer of TestMoERouting (logits [3,0,0,0]),
 *                         numpy float64 within tolerance, sum ~ 1
 *   orc_select            brute-force stable sort of (-p, index) over the
 *                         first C candidates; C=k reproduces the reference's
 *                         first-k quirk (set {0..k-1})
 *   orc_moe_forward       numpy float64 layer on small shapes, linearity /
 *                         zero-weight closed forms, TestMoERouting
 * Parity unpinned: the last bit of exp-dependent values (softmax, silu,
 * sigmoid) where the double result lies within ~1 ulp of an f32 rounding
 * boundary -- Go's math.Exp cannot be run here.
 */
#ifndef QMOE_ORACLE_H
#define QMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight formats, same numbering as the product's qmoe_format. */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_INT8G32 = 2, ORC_INT4G32 = 3 };

/* One (out, in) projection, reference `linear` / `quantLinear`
 * (model/model.go:106-111, model/moe.go:126-132).
 *   ORC_F32:     w = float[out*in]
 *   ORC_BF16:    w = uint16 bf16 bits [out*in]
 *   ORC_INT8G32: w = int8 codes [out*in],        scale = float[out*in/32]
 *   ORC_INT4G32: w = packed bytes [out*in/2],    scale = float[out*in/32]
 *                (hi nibble = even element, stored +8) */
typedef struct {
    int fmt;
    int out_dim;
    int in_dim;
    const void *w;
    const float *scale;
} orc_linear;

/* The MoE layer, reference moeMLP (model/moe.go:10-25).
 * Stacked experts: gate_up (E, 2I, H) rows [0,I) gate and [I,2I) up,
 * down (E, H, I); quantised formats hold codes with the same row layout and
 * per-row group-32 scales (E, rows, K/32).
 * scope: selection candidate scope C (k <= C <= E).  C = k reproduces
 * model/moe.go:45-53 exactly (the insertion sort only visits idx[0..k-1]);
 * C = E is true top-k with lowest-index tie-break. */
typedef struct {
    int hidden, n_experts, top_k, inter, shared_inter, scope;
    orc_linear router;            /* (E, H) */
    int expert_fmt;
    const void *gate_up;
    const float *gate_up_scale;
    const void *down;
    const float *down_scale;
    orc_linear sh_gate, sh_up, sh_down; /* only when shared_inter > 0 */
    const float *shared_gate;            /* (H) f32, only when shared_inter > 0 */
    int threads;  /* workers for bf16 linears with rows*in >= 65536, as Go's
                     linear.matvec (model/model.go:131-164); 1 = serial */
} orc_moe;

/* Scalar conversions. */
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16_rne(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16_rne(float f);
void orc_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n);
void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);
void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);

/* model/moe.go:165-188 / :190-217.  scales are the unrounded f32 values. */
void orc_quantize_int8(const float *w, int out_dim, int in_dim, int8_t *codes, float *scales);
void orc_quantize_int4(const float *w, int out_dim, int in_dim, uint8_t *codes, float *scales);
/* Stacked variant: n_mat independent (out,in) matrices back to back. */
void orc_quantize_stack(int bits, const float *w, int n_mat, int out_dim, int in_dim,
                        void *codes, float *scales);
/* model/moe.go:134-157 */
void orc_dequantize(int bits, const void *codes, const float *scales, int out_dim, int in_dim,
                    float *w);

/* y = x @ W^T for one vector: matmulVec / bf16matvec / quantLinear.forward
 * (tensors.go:77-89, moe.go:102-113, moe.go:159-162). */
void orc_matvec(const orc_linear *l, const float *x, float *y, int threads);

void orc_softmax(float *v, int n);                        /* tensors.go:106-121 */
void orc_silu(float *v, int n);                           /* tensors.go:91-95 */
float orc_sigmoid1(float x);                              /* tensors.go:97 */
/* Selection + renormalisation, moe.go:44-57,63: probs (E) -> idx (k) and
 * weights w_r = p / (wSum + 1e-9f). */
void orc_select(const float *probs, int n_experts, int top_k, int scope, int32_t *idx,
                float *weights);

/* argmax, model.go:652-660: best = 0, moved by v[i] > v[best]. */
int orc_argmax(const float *v, int n);

/* gemmaRMSNormApply, tensors.go:147-157, in place on x (n): the sum of
 * squares in f64, inv = float32(1 / sqrt(s/n + eps)), x = x * inv * (1 + w). */
void orc_gemma_rmsnorm(float *x, const float *w, int n, float eps);

/* moeMLP.forward (moe.go:41-99) applied to each of T tokens in turn, as
 * decodeLayers does (model.go:508-514).  x (T,H), out (T,H); ids/weights
 * (T,k) in rank order, may be NULL.  Returns 0, or -1 on bad arguments. */
int orc_moe_forward(const orc_moe *m, const float *x, int T, float *out, int32_t *ids,
                    float *weights);

/* Router stage alone (moe.go:42-57): logits -> probs (T,E) after softmax. */
int orc_moe_router(const orc_moe *m, const float *x, int T, float *probs, int32_t *ids,
                   float *weights);

#ifdef __cplusplus
}
#endif
#endif
