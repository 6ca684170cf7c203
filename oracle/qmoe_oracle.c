/*
 * qmoe_oracle.c -- CPU restatement of qwen-go's MoE block.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline for the HIP
 * product in qwen-go_amd/.  Never linked into libqmoe.so.
 *
 * Build: oracle/Makefile, gcc -O2 -ffp-contract=off (no FMA contraction and
 * no fast-math, as Go amd64 at GOAMD64=v1 evaluates x*y+z with two roundings).
 * Each function cites the reference lines it restates, relative to the
 * qwen-go source tree.
 */
#include "qmoe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QGROUP 32 /* quantGroup, model/moe.go:124 */

/* ---------------------------------------------------------------- scalars */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16f32, model/model.go:113-115: the 16 bits become the high half. */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* f32 -> bf16 round-to-nearest-even (the synthetic-weight format step; not
 * in the reference, which only reads bf16 files). */
uint16_t orc_f32_to_bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) /* NaN: keep quiet */
        return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* f16to32, safetensors/safetensors.go:182-207: exact widening, including
 * subnormals (normalised by shifting the fraction until the implicit bit). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t ex = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t fr = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (fr == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 127 - 15 + 1;
            while ((fr & 0x400u) == 0) { fr <<= 1; e--; }
            fr &= 0x3ffu;
            bits = (sign << 31) | (e << 23) | (fr << 13);
        }
    } else if (ex == 0x1f) {
        bits = (sign << 31) | (0xffu << 23) | (fr << 13);
    } else {
        bits = (sign << 31) | ((ex - 15 + 127) << 23) | (fr << 13);
    }
    return u2f(bits);
}

/* f32 -> f16 round-to-nearest-even.  The reference's quantiser keeps f32
 * scales; the device format stores them as fp16, so this is the one rounding
 * step the build adds (the oracle then widens the same fp16 value). */
uint16_t orc_f32_to_f16_rne(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ax = u & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / NaN */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    int e = (int)(ax >> 23) - 127;       /* unbiased exponent */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u; /* 24-bit significand */
    if (e >= -14) {                      /* normal f16 */
        uint32_t he = (uint32_t)(e + 15);
        uint32_t rem = m & 0x1fffu;      /* 13 dropped bits */
        uint32_t q = (he << 10) | ((m >> 13) & 0x3ffu);
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    if (e < -25) return (uint16_t)sign;  /* below half the smallest subnormal */
    /* subnormal: value = m * 2^(e-23); unit = 2^-24 -> shift = -e - 1 */
    int shift = -e - 1;                  /* in [14, 24] */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void orc_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_bf16_rne(src[i]);
}
void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}
void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16_rne(src[i]);
}

/* abs32 / clamp / roundF32, model/moe.go:241-258.  roundF32 is
 * float32(math.Round(float64(x))): half away from zero, which is C round(). */
static inline float abs32(float x) { return x < 0 ? -x : x; }
static inline float clampf(float x, float lo, float hi) {
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}
static inline float round_f32(float x) { return (float)round((double)x); }

/* ------------------------------------------------------------- quantiser */

/* quantizeInt8, model/moe.go:165-188. */
void orc_quantize_int8(const float *w, int out_dim, int in_dim, int8_t *codes, float *scales) {
    int ng = in_dim / QGROUP;
    for (int o = 0; o < out_dim; o++) {
        for (int b = 0; b < ng; b++) {
            const float *g = w + (size_t)o * in_dim + (size_t)b * QGROUP;
            float amax = 0.0f;
            for (int j = 0; j < QGROUP; j++) {
                float a = abs32(g[j]);
                if (a > amax) amax = a;
            }
            float s = amax / 127.0f;
            if (s < 1e-8f) s = 1e-8f;
            scales[(size_t)o * ng + b] = s;
            for (int j = 0; j < QGROUP; j++) {
                float v = round_f32(g[j] / s);
                codes[(size_t)o * in_dim + (size_t)b * QGROUP + j] = (int8_t)clampf(v, -127.0f, 127.0f);
            }
        }
    }
}

/* quantizeInt4, model/moe.go:190-217.  Even element -> high nibble. */
void orc_quantize_int4(const float *w, int out_dim, int in_dim, uint8_t *codes, float *scales) {
    int ng = in_dim / QGROUP;
    memset(codes, 0, (size_t)out_dim * (size_t)(in_dim / 2));
    for (int o = 0; o < out_dim; o++) {
        for (int b = 0; b < ng; b++) {
            const float *g = w + (size_t)o * in_dim + (size_t)b * QGROUP;
            float amax = 0.0f;
            for (int j = 0; j < QGROUP; j++) {
                float a = abs32(g[j]);
                if (a > amax) amax = a;
            }
            float s = amax / 7.0f;
            if (s < 1e-8f) s = 1e-8f;
            scales[(size_t)o * ng + b] = s;
            for (int j = 0; j < QGROUP; j++) {
                float v = clampf(round_f32(g[j] / s), -7.0f, 7.0f) + 8.0f;
                uint8_t nib = (uint8_t)((int)v & 0xf);
                uint8_t *dst = codes + (size_t)o * (in_dim / 2) + (size_t)b * (QGROUP / 2) + j / 2;
                if (j % 2 == 0) *dst |= (uint8_t)(nib << 4);
                else *dst |= nib;
            }
        }
    }
}

void orc_quantize_stack(int bits, const float *w, int n_mat, int out_dim, int in_dim,
                        void *codes, float *scales) {
    size_t welems = (size_t)out_dim * in_dim;
    size_t nsc = (size_t)out_dim * (in_dim / QGROUP);
    for (int e = 0; e < n_mat; e++) {
        if (bits == 8)
            orc_quantize_int8(w + e * welems, out_dim, in_dim, (int8_t *)codes + e * welems,
                              scales + e * nsc);
        else
            orc_quantize_int4(w + e * welems, out_dim, in_dim, (uint8_t *)codes + e * (welems / 2),
                              scales + e * nsc);
    }
}

/* quantLinear.dequantize, model/moe.go:134-157. */
void orc_dequantize(int bits, const void *codes, const float *scales, int out_dim, int in_dim,
                    float *w) {
    int ng = in_dim / QGROUP;
    if (bits == 8) {
        const int8_t *q = (const int8_t *)codes;
        for (int o = 0; o < out_dim; o++)
            for (int c = 0; c < in_dim; c++)
                w[(size_t)o * in_dim + c] =
                    (float)q[(size_t)o * in_dim + c] * scales[(size_t)o * ng + c / QGROUP];
        return;
    }
    const uint8_t *q = (const uint8_t *)codes;
    for (int o = 0; o < out_dim; o++) {
        for (int c = 0; c < in_dim / 2; c++) {
            uint8_t b = q[(size_t)o * (in_dim / 2) + c];
            float hi = (float)((int)(b >> 4) & 0xf) - 8.0f;
            float lo = (float)((int)b & 0xf) - 8.0f;
            w[(size_t)o * in_dim + 2 * c] = hi * scales[(size_t)o * ng + (2 * c) / QGROUP];
            w[(size_t)o * in_dim + 2 * c + 1] = lo * scales[(size_t)o * ng + (2 * c + 1) / QGROUP];
        }
    }
}

/* ---------------------------------------------------------------- GEMVs */

/* Rows [lo,hi) of y = x @ W^T.  The inner loops are matmulVec
 * (tensors.go:77-89), matvecRange / bf16matvec (model.go:167-176,
 * moe.go:102-113), and for the quantised formats quantLinear.forward
 * (moe.go:159-162): dequantise then matmulVec.  Dequantising one row at a time
 * gives the same f32 weights as the whole-matrix dequantize. */
static void matvec_rows(const orc_linear *l, const float *x, float *y, int lo, int hi) {
    int in = l->in_dim;
    int ng = in / QGROUP;
    switch (l->fmt) {
    case ORC_F32: {
        const float *w = (const float *)l->w;
        for (int o = lo; o < hi; o++) {
            const float *wr = w + (size_t)o * in;
            float s = 0.0f;
            for (int k = 0; k < in; k++) s += x[k] * wr[k];
            y[o] = s;
        }
        break;
    }
    case ORC_BF16: {
        const uint16_t *w = (const uint16_t *)l->w;
        for (int o = lo; o < hi; o++) {
            const uint16_t *wr = w + (size_t)o * in;
            float s = 0.0f;
            for (int k = 0; k < in; k++) s += x[k] * orc_bf16_to_f32(wr[k]);
            y[o] = s;
        }
        break;
    }
    case ORC_INT8G32: {
        const int8_t *q = (const int8_t *)l->w;
        for (int o = lo; o < hi; o++) {
            const int8_t *qr = q + (size_t)o * in;
            const float *sr = l->scale + (size_t)o * ng;
            float s = 0.0f;
            for (int k = 0; k < in; k++) {
                float wv = (float)qr[k] * sr[k / QGROUP];
                s += x[k] * wv;
            }
            y[o] = s;
        }
        break;
    }
    case ORC_INT4G32: {
        const uint8_t *q = (const uint8_t *)l->w;
        for (int o = lo; o < hi; o++) {
            const uint8_t *qr = q + (size_t)o * (in / 2);
            const float *sr = l->scale + (size_t)o * ng;
            float s = 0.0f;
            for (int c = 0; c < in / 2; c++) {
                uint8_t b = qr[c];
                float whi = ((float)((int)(b >> 4) & 0xf) - 8.0f) * sr[(2 * c) / QGROUP];
                float wlo = ((float)((int)b & 0xf) - 8.0f) * sr[(2 * c + 1) / QGROUP];
                s += x[2 * c] * whi;
                s += x[2 * c + 1] * wlo;
            }
            y[o] = s;
        }
        break;
    }
    default:
        break;
    }
}

typedef struct {
    const orc_linear *l;
    const float *x;
    float *y;
    int lo, hi;
} mv_job;

static void *mv_worker(void *arg) {
    mv_job *j = (mv_job *)arg;
    matvec_rows(j->l, j->x, j->y, j->lo, j->hi);
    return NULL;
}

/* linear.matvec fan-out, model/model.go:131-164: bf16 linears with
 * out*in >= 65536 split rows into ceil(out/workers) chunks, one goroutine
 * each; everything else runs on the caller.  Each row is one sequential sum,
 * so the split never changes the result. */
void orc_matvec(const orc_linear *l, const float *x, float *y, int threads) {
    const long min_work = 1L << 16;
    if (l->fmt != ORC_BF16 || threads <= 1 || (long)l->out_dim * l->in_dim < min_work) {
        matvec_rows(l, x, y, 0, l->out_dim);
        return;
    }
    if (threads > 8) threads = 8; /* runtimeNumWorkers cap, tensors.go:50-59 */
    int chunk = (l->out_dim + threads - 1) / threads;
    pthread_t tid[8];
    mv_job jobs[8];
    int spawned = 0;
    for (int i = 0; i < threads; i++) {
        int lo = i * chunk, hi = lo + chunk;
        if (hi > l->out_dim) hi = l->out_dim;
        if (lo >= hi) break;
        jobs[spawned] = (mv_job){l, x, y, lo, hi};
        if (pthread_create(&tid[spawned], NULL, mv_worker, &jobs[spawned]) != 0) {
            matvec_rows(l, x, y, lo, hi);
            continue;
        }
        spawned++;
    }
    for (int i = 0; i < spawned; i++) pthread_join(tid[i], NULL);
}

/* ------------------------------------------------------------ activations */

/* softmax, model/tensors.go:106-121. */
void orc_softmax(float *v, int n) {
    float mx = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        v[i] = (float)exp((double)(v[i] - mx));
        sum += v[i];
    }
    for (int i = 0; i < n; i++) v[i] /= sum;
}

/* silu, model/tensors.go:91-95. */
void orc_silu(float *v, int n) {
    for (int i = 0; i < n; i++) v[i] = v[i] / (1.0f + (float)exp(-(double)v[i]));
}

/* sigmoid1, model/tensors.go:97. */
float orc_sigmoid1(float x) { return 1.0f / (1.0f + (float)exp(-(double)x)); }

/* argmax, model/model.go:652-660. */
int orc_argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* gemmaRMSNormApply, model/tensors.go:147-157.  float64(v) * float64(v) is
 * exact; the sum rounds in f64 in index order; 1 / sqrt(s/n + eps) runs in
 * f64 (eps widened from f32) and rounds once to f32; then
 * x = fl(fl(x * inv) * fl(1 + w)), left to right. */
void orc_gemma_rmsnorm(float *x, const float *w, int n, float eps) {
    double s = 0.0;
    for (int i = 0; i < n; i++) s += (double)x[i] * (double)x[i];
    const float inv = (float)(1.0 / sqrt(s / (double)n + (double)eps));
    for (int i = 0; i < n; i++) {
        const float a = x[i] * inv;
        const float b = 1.0f + w[i];
        x[i] = a * b;
    }
}

/* Selection and renormalisation, model/moe.go:44-57 and :63.  The reference
 * loop runs i < topK; generalised here to i < scope, so scope == top_k is the
 * reference bit for bit and scope == n_experts is a full stable sort. */
void orc_select(const float *probs, int n_experts, int top_k, int scope, int32_t *idx_out,
                float *weights) {
    int *idx = (int *)malloc(sizeof(int) * (size_t)n_experts);
    for (int i = 0; i < n_experts; i++) idx[i] = i;
    for (int i = 1; i < scope && i < n_experts; i++) {
        for (int j = i; j > 0 && probs[idx[j]] > probs[idx[j - 1]]; j--) {
            int t = idx[j];
            idx[j] = idx[j - 1];
            idx[j - 1] = t;
        }
    }
    float wsum = 0.0f;
    for (int i = 0; i < top_k; i++) wsum += probs[idx[i]];
    for (int i = 0; i < top_k; i++) {
        idx_out[i] = idx[i];
        if (weights) weights[i] = probs[idx[i]] / (wsum + 1e-9f);
    }
    free(idx);
}

/* ----------------------------------------------------------------- layer */

static int check_layer(const orc_moe *m, int T) {
    if (!m || T < 0) return -1;
    if (m->hidden <= 0 || m->n_experts <= 0 || m->top_k <= 0 || m->inter <= 0) return -1;
    if (m->top_k > m->n_experts) return -1;
    if (m->scope < m->top_k || m->scope > m->n_experts) return -1;
    return 0;
}

static orc_linear expert_linear(const orc_moe *m, int e, int which) {
    /* which 0: gate_up (2I, H); 1: down (H, I) */
    orc_linear l;
    l.fmt = m->expert_fmt;
    l.out_dim = which == 0 ? 2 * m->inter : m->hidden;
    l.in_dim = which == 0 ? m->hidden : m->inter;
    size_t elems = (size_t)l.out_dim * l.in_dim;
    size_t nsc = (size_t)l.out_dim * (l.in_dim / QGROUP);
    const char *base = (const char *)(which == 0 ? m->gate_up : m->down);
    const float *sc = which == 0 ? m->gate_up_scale : m->down_scale;
    size_t bytes;
    switch (l.fmt) {
    case ORC_F32: bytes = elems * 4; break;
    case ORC_BF16: bytes = elems * 2; break;
    case ORC_INT8G32: bytes = elems; break;
    default: bytes = elems / 2; break;
    }
    l.w = base + (size_t)e * bytes;
    l.scale = sc ? sc + (size_t)e * nsc : NULL;
    return l;
}

int orc_moe_router(const orc_moe *m, const float *x, int T, float *probs, int32_t *ids,
                   float *weights) {
    if (check_layer(m, T)) return -1;
    int H = m->hidden, E = m->n_experts, K = m->top_k;
    int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (size_t)K);
    for (int t = 0; t < T; t++) {
        float *p = probs + (size_t)t * E;
        orc_matvec(&m->router, x + (size_t)t * H, p, m->threads); /* moe.go:42 */
        orc_softmax(p, E);                                         /* moe.go:43 */
        orc_select(p, E, K, m->scope, ids ? ids + (size_t)t * K : tmp,
                   weights ? weights + (size_t)t * K : NULL);
    }
    free(tmp);
    return 0;
}

/* moeMLP.forward, model/moe.go:41-99, once per token (model.go:508-514). */
int orc_moe_forward(const orc_moe *m, const float *x, int T, float *out, int32_t *ids,
                    float *weights) {
    if (check_layer(m, T)) return -1;
    int H = m->hidden, E = m->n_experts, K = m->top_k, I = m->inter, Is = m->shared_inter;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    float *gu = (float *)malloc(sizeof(float) * 2 * (size_t)I);
    float *d = (float *)malloc(sizeof(float) * (size_t)H);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)K);
    float *wts = (float *)malloc(sizeof(float) * (size_t)K);
    int sIs = Is > 0 ? Is : 1;
    float *sg_buf = (float *)malloc(sizeof(float) * (size_t)sIs);
    float *su_buf = (float *)malloc(sizeof(float) * (size_t)sIs);
    float *s_buf = (float *)malloc(sizeof(float) * (size_t)H);
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        float *ot = out + (size_t)t * H;
        orc_matvec(&m->router, xt, logits, m->threads);  /* moe.go:42 */
        orc_softmax(logits, E);                          /* moe.go:43 */
        orc_select(logits, E, K, m->scope, idx, wts);    /* moe.go:44-57, 63 */
        for (int j = 0; j < H; j++) ot[j] = 0.0f;        /* moe.go:58 */
        for (int r = 0; r < K; r++) {                    /* moe.go:61-85 */
            int e = idx[r];
            float w = wts[r];
            orc_linear lgu = expert_linear(m, e, 0);
            matvec_rows(&lgu, xt, gu, 0, 2 * I);         /* moe.go:65-69, single-threaded */
            float *g = gu, *u = gu + I;
            orc_silu(g, I);                              /* moe.go:72 */
            for (int j = 0; j < I; j++) g[j] *= u[j];    /* moe.go:73-75 */
            orc_linear ld = expert_linear(m, e, 1);
            matvec_rows(&ld, g, d, 0, H);                /* moe.go:77-81 */
            for (int j = 0; j < H; j++) ot[j] += w * d[j]; /* moe.go:82-84 */
        }
        if (Is > 0) {                                    /* moe.go:86-97 */
            /* denseMLP.forward, model.go:350-358 */
            orc_matvec(&m->sh_gate, xt, sg_buf, m->threads);
            orc_matvec(&m->sh_up, xt, su_buf, m->threads);
            orc_silu(sg_buf, Is);
            for (int j = 0; j < Is; j++) sg_buf[j] *= su_buf[j];
            orc_matvec(&m->sh_down, sg_buf, s_buf, m->threads);
            float g = 0.0f;
            for (int i = 0; i < H; i++) g += xt[i] * m->shared_gate[i];
            float sg = orc_sigmoid1(g);
            for (int j = 0; j < H; j++) ot[j] += sg * s_buf[j];
        }
        if (ids)
            for (int r = 0; r < K; r++) ids[(size_t)t * K + r] = idx[r];
        if (weights)
            for (int r = 0; r < K; r++) weights[(size_t)t * K + r] = wts[r];
    }
    free(logits); free(gu); free(d); free(idx); free(wts);
    free(sg_buf); free(su_buf); free(s_buf);
    return 0;
}
