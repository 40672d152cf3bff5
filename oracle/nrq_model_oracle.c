/*
 * CPU oracle for the Llama-family forward pass -- TEST INFRASTRUCTURE ONLY.
 * Only tests/ and bench.py's cpu_baseline leg use this file, as the checker.
 *
 * Plain-C restatement of crates/nr-model/src/infer.rs (InferCtx::forward,
 * prefill_chunk) over the oracle's scalar-order matvec/matmul, and of the f32
 * vector ops of crates/nr-tensor/src/vec.rs and rope.rs. Every f32 operation
 * is written out in the reference's order; the build uses -ffp-contract=off.
 *
 * libm: the reference calls the `libm` crate 0.2.16 (Cargo.lock:216-219), a
 * port of musl that is not vendored in the reference tree. expf and sincosf
 * below restate musl's published single-precision algorithms (FreeBSD msun
 * e_expf.c; s_sincosf.c with the __sindf/__cosdf kernels and __rem_pio2f),
 * which is what that crate ports; sqrtf is IEEE (correctly rounded). Without
 * the crate present, their bits are "parity unpinned" against the reference;
 * the tests pin them against glibc within 1 ulp instead.
 */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "nrq_oracle.h"

/* ---- libm restatements ----------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* musl scalbnf */
static float scalbnf_(float x, int n) {
    float y = x;
    if (n > 127) {
        y *= u2f(0x7f000000u); /* 2^127 */
        n -= 127;
        if (n > 127) {
            y *= u2f(0x7f000000u);
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        y *= u2f(0x00800000u) * u2f(0x4b800000u); /* 2^-126 * 2^24 */
        n += 126 - 24;
        if (n < -126) {
            y *= u2f(0x00800000u) * u2f(0x4b800000u);
            n += 126 - 24;
            if (n < -126) n = -126;
        }
    }
    return y * u2f((uint32_t)(0x7f + n) << 23);
}

/* musl expf (FreeBSD e_expf.c): reduction x = k*ln2 + r, |r| <= 0.5 ln2,
 * exp(r) by the degree-2 rational form of the Remez polynomial P1, P2. */
float nro_expf(float x) {
    const float half[2] = {0.5f, -0.5f};
    const float ln2hi = 6.9314575195e-01f, ln2lo = 1.4286067653e-06f, invln2 = 1.4426950216e+00f;
    const float P1 = 1.6666625440e-1f, P2 = -2.7667332906e-3f;
    uint32_t hx = f2u(x);
    int sign = (int)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x42aeac50u) {          /* |x| >= -87.33655f or NaN */
        if (hx > 0x7f800000u) return x; /* NaN */
        if (hx >= 0x42b17218u && !sign) return x * u2f(0x7f000000u); /* overflow */
        if (sign && hx >= 0x42cff1b5u) return 0.0f;                   /* underflow */
    }
    int k;
    float hi, lo;
    if (hx > 0x3eb17218u) {       /* |x| > 0.5 ln2 */
        if (hx > 0x3f851592u)     /* |x| > 1.5 ln2 */
            k = (int)(invln2 * x + half[sign]);
        else
            k = 1 - sign - sign;
        float kf = (float)k;
        hi = x - kf * ln2hi;
        lo = kf * ln2lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) { /* |x| > 2^-14 */
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    float xx = x * x;
    float c = x - xx * (P1 + xx * P2);
    float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : scalbnf_(y, k);
}

/* __sindf / __cosdf: polynomials in double on [-pi/4, pi/4] */
static float sindf_(double x) {
    const double S1 = -0x15555554cbac77.0p-55, S2 = 0x111110896efbb2.0p-59;
    const double S3 = -0x1a00f9e2cae774.0p-65, S4 = 0x16cd878c3b46a7.0p-71;
    double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}
static float cosdf_(double x) {
    const double C0 = -0x1ffffffd0c5e81.0p-54, C1 = 0x155553e1053a42.0p-57;
    const double C2 = -0x16c087e80f1e27.0p-62, C3 = 0x199342e0ee5069.0p-68;
    double z = x * x, w = z * z, r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

/* __rem_pio2f, medium-size path (|x| < 2^28 * pi/2); the large path is not
 * reachable by the rope angles here and returns 0 with y = NaN. */
static int rem_pio2f_(float x, double *y) {
    const double toint = 1.5 / 2.220446049250313e-16, pio4 = 0x1.921fb6p-1;
    const double invpio2 = 6.36619772367581382433e-01, pio2_1 = 1.57079631090164184570e+00;
    const double pio2_1t = 1.58932547735281966916e-08;
    uint32_t ix = f2u(x) & 0x7fffffffu;
    if (ix < 0x4dc90fdbu) {
        double fn = (double)x * invpio2 + toint - toint;
        int n = (int)fn;
        *y = x - fn * pio2_1 - fn * pio2_1t;
        if (*y < -pio4) {
            n--;
            fn--;
            *y = x - fn * pio2_1 - fn * pio2_1t;
        } else if (*y > pio4) {
            n++;
            fn++;
            *y = x - fn * pio2_1 - fn * pio2_1t;
        }
        return n;
    }
    *y = NAN;
    return 0;
}

/* musl sincosf */
void nro_sincosf(float x, float *sin, float *cos) {
    const double s1pio2 = 1 * 1.57079632679489661923, s2pio2 = 2 * 1.57079632679489661923;
    const double s3pio2 = 3 * 1.57079632679489661923, s4pio2 = 4 * 1.57079632679489661923;
    uint32_t ix = f2u(x);
    unsigned sign = ix >> 31;
    ix &= 0x7fffffffu;
    if (ix <= 0x3f490fdau) {     /* |x| ~<= pi/4 */
        if (ix < 0x39800000u) {  /* |x| < 2^-12 */
            *sin = x;
            *cos = 1.0f;
            return;
        }
        *sin = sindf_(x);
        *cos = cosdf_(x);
        return;
    }
    if (ix <= 0x407b53d1u) {     /* |x| ~<= 5pi/4 */
        if (ix <= 0x4016cbe3u) { /* |x| ~<= 3pi/4 */
            if (sign) {
                *sin = -cosdf_(x + s1pio2);
                *cos = sindf_(x + s1pio2);
            } else {
                *sin = cosdf_(s1pio2 - x);
                *cos = sindf_(s1pio2 - x);
            }
            return;
        }
        *sin = -sindf_(sign ? x + s2pio2 : x - s2pio2);
        *cos = -cosdf_(sign ? x + s2pio2 : x - s2pio2);
        return;
    }
    if (ix <= 0x40e231d5u) {     /* |x| ~<= 9pi/4 */
        if (ix <= 0x40afeddfu) { /* |x| ~<= 7pi/4 */
            if (sign) {
                *sin = cosdf_(x + s3pio2);
                *cos = -sindf_(x + s3pio2);
            } else {
                *sin = -cosdf_(x - s3pio2);
                *cos = sindf_(x - s3pio2);
            }
            return;
        }
        *sin = sindf_(sign ? x + s4pio2 : x - s4pio2);
        *cos = cosdf_(sign ? x + s4pio2 : x - s4pio2);
        return;
    }
    if (ix >= 0x7f800000u) {
        *sin = *cos = x - x;
        return;
    }
    double y;
    unsigned n = (unsigned)rem_pio2f_(x, &y);
    float s = sindf_(y), c = cosdf_(y);
    switch (n & 3) {
    case 0: *sin = s; *cos = c; break;
    case 1: *sin = c; *cos = -s; break;
    case 2: *sin = -s; *cos = -c; break;
    default: *sin = -c; *cos = s; break;
    }
}

/* ---- vec.rs / rope.rs ---------------------------------------------------------- */

/* vec.rs:4-14: out = x * (1/sqrtf(mean(x^2) + eps)) * weight */
void nro_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* vec.rs:30-42 */
void nro_softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = nro_expf(x[i] - max);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* vec.rs:45-52 */
void nro_swiglu(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float silu = g / (1.0f + nro_expf(-g));
        gate[i] = silu * up[i];
    }
}

/* vec.rs:80-90: first index of the largest value (strict >, NaN never wins) */
uint32_t nro_argmax(const float *x, size_t n) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return (uint32_t)best;
}

/* vec.rs:17-28 (rmsnorm_inplace): ss in element order, then x *= scale * w */
void nro_rmsnorm_inplace(float *x, const float *w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) x[i] *= scale * w[i];
}

/* rope.rs:14-34 without Llama-3 scaling: freqs[i] = theta^(-2i/head_dim) */
void nro_rope_freqs(float *out, size_t head_dim, float theta) {
    for (size_t i = 0; i < head_dim / 2; i++) {
        float exponent = -2.0f * (float)i / (float)head_dim;
        out[i] = powf(theta, exponent);
    }
}

/* rope.rs:49-65: pair i is (2i, 2i+1) (Adjacent, Llama/Granite) or
 * (i, i + head_dim/2) (Neox, Qwen3) */
void nro_rope_apply_style(float *x, size_t n, size_t head_dim, const float *freqs, size_t pos, int neox) {
    size_t half = head_dim / 2;
    for (size_t h = 0; h + head_dim <= n; h += head_dim) {
        float *head = x + h;
        for (size_t i = 0; i < half; i++) {
            float angle = (float)pos * freqs[i];
            float s, c;
            nro_sincosf(angle, &s, &c);
            size_t ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
            float a = head[ia], b = head[ib];
            head[ia] = a * c - b * s;
            head[ib] = a * s + b * c;
        }
    }
}
void nro_rope_apply(float *x, size_t n, size_t head_dim, const float *freqs, size_t pos) {
    nro_rope_apply_style(x, n, head_dim, freqs, pos, 0);
}

/* kernels.rs:146-160 (scalar path) */
static float dot_f16_(const uint16_t *k, const float *q, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += nro_f16_to_f32(k[i]) * q[i];
    return s;
}

/* kernels.rs:163-173 (scalar path) */
static void axpy_f16_(float *out, float a, const uint16_t *v, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] += a * nro_f16_to_f32(v[i]);
}

/* kernels.rs:174-201, dot_f16_f16c: eight lane accumulators, one
 * fmadd(f32(k), q, acc) per 8-element chunk, then the 128-bit halves added,
 * movehl, add_ss with lane 1: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)); the tail
 * past the last whole chunk as the scalar kernel. cvtph_ps is exact, as
 * f16_to_f32 is. */
__attribute__((target("avx2,fma,f16c"))) static float dot_f16_f16c_(const uint16_t *k, const float *q, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++) {
        __m256 kf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + 8 * i)));
        acc = _mm256_fmadd_ps(kf, _mm256_loadu_ps(q + 8 * i), acc);
    }
    __m128 s4 = _mm_add_ps(_mm256_extractf128_ps(acc, 1), _mm256_castps256_ps128(acc));
    s4 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
    s4 = _mm_add_ss(s4, _mm_shuffle_ps(s4, s4, 1));
    float sum = _mm_cvtss_f32(s4);
    for (size_t i = chunks * 8; i < n; i++) sum += nro_f16_to_f32(k[i]) * q[i];
    return sum;
}

/* kernels.rs:203-220, axpy_f16_f16c: out = fmadd(a, f32(v), out) per element of
 * whole 8-element chunks (one rounding), the tail as the scalar kernel. */
__attribute__((target("avx2,fma,f16c"))) static void axpy_f16_f16c_(float *out, float a, const uint16_t *v, size_t n) {
    __m256 av = _mm256_set1_ps(a);
    size_t chunks = n / 8;
    for (size_t i = 0; i < chunks; i++) {
        __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(v + 8 * i)));
        _mm256_storeu_ps(out + 8 * i, _mm256_fmadd_ps(av, vf, _mm256_loadu_ps(out + 8 * i)));
    }
    for (size_t i = chunks * 8; i < n; i++) out[i] += a * nro_f16_to_f32(v[i]);
}

float nro_dot_f16(int order, const uint16_t *k, const float *q, size_t n) {
    return order == NRO_ORDER_AVX2 ? dot_f16_f16c_(k, q, n) : dot_f16_(k, q, n);
}
void nro_axpy_f16(int order, float *out, float a, const uint16_t *v, size_t n) {
    if (order == NRO_ORDER_AVX2) axpy_f16_f16c_(out, a, v, n);
    else axpy_f16_(out, a, v, n);
}

/* ---- InferCtx (infer.rs) ------------------------------------------------------- */

#define NRO_MAX_LAYERS 64
#define NRO_MAX_BATCH 64 /* infer.rs:101 */

struct nro_model {
    int dim, n_layers, n_heads, n_kv_heads, head_dim, kv_dim, ffn_dim, vocab, ctx, threads;
    /* kernel order: scalar (the default, what the device reproduces) or the
     * x86 host's (AVX2 dots, F16C attention: cpu::fast_path / fast_f16) */
    int order;
    float eps;
    /* the recipe (infer.rs:447-461): rope style, muP scalars */
    int neox;
    float embed_scale, att_scale, residual_scale, logit_recip;
    float *freqs;
    const uint8_t *embed, *output;
    int embed_dt, output_dt;
    const float *out_norm;
    struct {
        const uint8_t *w[7]; /* q, k, v, o, gate, up, down */
        int dt[7];
        const float *attn_norm, *ffn_norm;
        const float *q_norm, *k_norm; /* Qwen3 per-head RMSNorm weights, head_dim each */
    } L[NRO_MAX_LAYERS];
    uint16_t *kc, *vc;
    float *x, *xb, *xb2, *q, *k, *v, *att, *attn_out, *gate, *up, *logits;
    float *bx, *bxb, *bq, *bk, *bv, *battn, *bgate, *bup;
    uint8_t *xq;
    int pos;
};

static int qk_of(int dt) { return dt == NRO_Q8_0 ? NRO_QK8_0 : NRO_QK_K; }
static size_t act_bytes(int dt, size_t n) {
    return dt == NRO_Q8_0 ? n / NRO_QK8_0 * NRO_Q8_0_BYTES : n / NRO_QK_K * NRO_Q8K_BYTES;
}

nro_model *nro_model_new(const int dims[8], float eps, float theta, int threads) {
    nro_model *m = (nro_model *)calloc(1, sizeof(nro_model));
    m->dim = dims[0];
    m->n_layers = dims[1];
    m->n_heads = dims[2];
    m->n_kv_heads = dims[3];
    m->head_dim = dims[4];
    m->ffn_dim = dims[5];
    m->vocab = dims[6];
    m->ctx = dims[7];
    m->kv_dim = m->n_kv_heads * m->head_dim;
    m->eps = eps;
    m->threads = threads;
    size_t att_dim = (size_t)m->n_heads * m->head_dim;
    size_t maxd = (size_t)m->dim;
    if (att_dim > maxd) maxd = att_dim;
    if ((size_t)m->ffn_dim > maxd) maxd = (size_t)m->ffn_dim;
    m->freqs = (float *)calloc((size_t)m->head_dim / 2, sizeof(float));
    nro_rope_freqs(m->freqs, (size_t)m->head_dim, theta);
    m->neox = 0;
    m->embed_scale = 1.0f;
    m->att_scale = 1.0f / sqrtf((float)m->head_dim);
    m->residual_scale = 1.0f;
    m->logit_recip = 1.0f;
    size_t kvn = (size_t)m->n_layers * m->ctx * m->kv_dim;
    m->kc = (uint16_t *)calloc(kvn, 2);
    m->vc = (uint16_t *)calloc(kvn, 2);
    m->x = (float *)calloc(m->dim, 4);
    m->xb = (float *)calloc(maxd, 4);
    m->xb2 = (float *)calloc(m->dim, 4);
    m->q = (float *)calloc(att_dim, 4);
    m->k = (float *)calloc(m->kv_dim, 4);
    m->v = (float *)calloc(m->kv_dim, 4);
    m->att = (float *)calloc((size_t)m->n_heads * m->ctx, 4);
    m->attn_out = (float *)calloc(att_dim, 4);
    m->gate = (float *)calloc(m->ffn_dim, 4);
    m->up = (float *)calloc(m->ffn_dim, 4);
    m->logits = (float *)calloc(m->vocab, 4);
    size_t B = NRO_MAX_BATCH;
    m->bx = (float *)calloc(B * m->dim, 4);
    m->bxb = (float *)calloc(B * maxd, 4);
    m->bq = (float *)calloc(B * att_dim, 4);
    m->bk = (float *)calloc(B * m->kv_dim, 4);
    m->bv = (float *)calloc(B * m->kv_dim, 4);
    m->battn = (float *)calloc(B * att_dim, 4);
    m->bgate = (float *)calloc(B * m->ffn_dim, 4);
    m->bup = (float *)calloc(B * m->ffn_dim, 4);
    m->xq = (uint8_t *)calloc(B * (maxd / NRO_QK8_0 * NRO_Q8_0_BYTES + maxd / NRO_QK_K * NRO_Q8K_BYTES) + 64, 1);
    return m;
}

void nro_model_free(nro_model *m) {
    if (!m) return;
    free(m->freqs); free(m->kc); free(m->vc); free(m->x); free(m->xb); free(m->xb2); free(m->q);
    free(m->k); free(m->v); free(m->att); free(m->attn_out); free(m->gate); free(m->up); free(m->logits);
    free(m->bx); free(m->bxb); free(m->bq); free(m->bk); free(m->bv); free(m->battn); free(m->bgate);
    free(m->bup); free(m->xq); free(m);
}

void nro_model_set_globals(nro_model *m, const void *embed, int embed_dt, const void *output, int output_dt,
                           const float *out_norm) {
    m->embed = (const uint8_t *)embed;
    m->embed_dt = embed_dt;
    m->output = (const uint8_t *)output;
    m->output_dt = output_dt;
    m->out_norm = out_norm;
}

void nro_model_set_layer(nro_model *m, int l, const void *const w[7], const int dt[7], const float *attn_norm,
                         const float *ffn_norm) {
    for (int i = 0; i < 7; i++) {
        m->L[l].w[i] = (const uint8_t *)w[i];
        m->L[l].dt[i] = dt[i];
    }
    m->L[l].attn_norm = attn_norm;
    m->L[l].ffn_norm = ffn_norm;
}

/* InferCtx::new's recipe fields (infer.rs:447-461): attn_scale 0 means
 * 1/sqrtf(head_dim); logit_recip = 1/logit_scale */
void nro_model_set_recipe(nro_model *m, int neox, float embed_scale, float attn_scale, float residual_scale,
                          float logit_scale) {
    m->neox = neox;
    m->embed_scale = embed_scale;
    m->att_scale = attn_scale != 0.0f ? attn_scale : 1.0f / sqrtf((float)m->head_dim);
    m->residual_scale = residual_scale;
    m->logit_recip = 1.0f / logit_scale;
}

void nro_model_set_qk_norm(nro_model *m, int l, const float *q_norm, const float *k_norm) {
    m->L[l].q_norm = q_norm;
    m->L[l].k_norm = k_norm;
}

int nro_model_pos(const nro_model *m) { return m->pos; }
void nro_model_reset(nro_model *m) { m->pos = 0; }
void nro_model_set_order(nro_model *m, int order) { m->order = order; }
/* Timing aid for the CPU baseline: moves to position pos (< ctx) without
 * computing the cache rows before it (they keep their contents). */
void nro_model_seek(nro_model *m, int pos) {
    if (pos >= 0 && pos < m->ctx) m->pos = pos;
}
void nro_model_set_freqs(nro_model *m, const float *freqs) {
    memcpy(m->freqs, freqs, (size_t)m->head_dim / 2 * sizeof(float));
}
const float *nro_model_logits(const nro_model *m) { return m->logits; }
const uint16_t *nro_model_kcache(const nro_model *m) { return m->kc; }
const uint16_t *nro_model_vcache(const nro_model *m) { return m->vc; }

/* QMat::dequant_row (infer.rs:37-56) */
static void dequant_row_(const uint8_t *w, int dt, size_t r, size_t cols, float *out) {
    size_t bpr = cols / (size_t)qk_of(dt);
    if (dt == NRO_Q8_0) {
        nro_dequantize_q8_0(w + r * bpr * NRO_Q8_0_BYTES, bpr, out);
    } else {
        for (size_t b = 0; b < bpr; b++) {
            if (dt == NRO_Q4K) nro_dequant_q4k(w + (r * bpr + b) * NRO_Q4K_BYTES, out + b * NRO_QK_K);
            else nro_dequant_q6k(w + (r * bpr + b) * NRO_Q6K_BYTES, out + b * NRO_QK_K);
        }
    }
}

/* Acts::matvec (infer.rs:112-132): quantize x to the weight's activation format, matvec */
static void acts_matvec_(nro_model *m, float *y, const uint8_t *w, int dt, const float *x, size_t rows, size_t cols) {
    if (dt == NRO_Q8_0) nro_quantize_q8_0(x, cols, m->xq);
    else nro_quantize_q8k(x, cols, m->xq);
    nro_matvec(dt, m->order, y, w, m->xq, rows, cols, m->threads);
}

/* Acts::matmul (infer.rs:137-174): per-row quantize, batched matmul */
static void acts_matmul_(nro_model *m, float *y, const uint8_t *w, int dt, const float *xs, size_t rows, size_t cols,
                         size_t batch) {
    size_t xb = act_bytes(dt, cols);
    for (size_t b = 0; b < batch; b++) {
        if (dt == NRO_Q8_0) nro_quantize_q8_0(xs + b * cols, cols, m->xq + b * xb);
        else nro_quantize_q8k(xs + b * cols, cols, m->xq + b * xb);
    }
    nro_matmul(dt, m->order, y, w, m->xq, rows, cols, batch, m->threads);
}

/* causal attention of one token at `pos` over layer l's cache (infer.rs:553-572) */
static void attend_(nro_model *m, int l, size_t pos, const float *q, float *out) {
    size_t hd = (size_t)m->head_dim, gqa = (size_t)(m->n_heads / m->n_kv_heads);
    float scale = m->att_scale;
    for (size_t h = 0; h < (size_t)m->n_heads; h++) {
        const float *qh = q + h * hd;
        size_t kvh = (h / gqa) * hd;
        float *att = m->att + h * (size_t)m->ctx;
        for (size_t t = 0; t <= pos; t++) {
            size_t krow = ((size_t)l * m->ctx + t) * m->kv_dim + kvh;
            att[t] = nro_dot_f16(m->order, m->kc + krow, qh, hd) * scale;
        }
        nro_softmax(att, pos + 1);
        float *o = out + h * hd;
        for (size_t i = 0; i < hd; i++) o[i] = 0.0f;
        for (size_t t = 0; t <= pos; t++) {
            size_t vrow = ((size_t)l * m->ctx + t) * m->kv_dim + kvh;
            nro_axpy_f16(m->order, o, att[t], m->vc + vrow, hd);
        }
    }
}

/* Qwen3's per-head RMSNorm of q and k before rope (infer.rs:533-541) */
static void qk_norm_(nro_model *m, int l, float *q, float *k) {
    size_t hd = (size_t)m->head_dim;
    if (!m->L[l].q_norm || !m->L[l].k_norm) return;
    for (size_t h = 0; h < (size_t)m->n_heads; h++) nro_rmsnorm_inplace(q + h * hd, m->L[l].q_norm, hd, m->eps);
    for (size_t h = 0; h < (size_t)m->n_kv_heads; h++) nro_rmsnorm_inplace(k + h * hd, m->L[l].k_norm, hd, m->eps);
}

/* InferCtx::forward (infer.rs:510-595), with the recipe: muP embedding scale,
 * qk-norm, rope style, attention score scale, residual scale, logit scale. */
const float *nro_model_forward(nro_model *m, uint32_t token) {
    size_t d = (size_t)m->dim, kvd = (size_t)m->kv_dim, ffn = (size_t)m->ffn_dim;
    size_t att_dim = (size_t)m->n_heads * m->head_dim;
    size_t pos = (size_t)m->pos;
    dequant_row_(m->embed, m->embed_dt, token, d, m->x);
    if (m->embed_scale != 1.0f)
        for (size_t i = 0; i < d; i++) m->x[i] *= m->embed_scale; /* vec.rs:61-65 */
    for (int l = 0; l < m->n_layers; l++) {
        nro_rmsnorm(m->xb, m->x, m->L[l].attn_norm, d, m->eps);
        /* matvec_group: all three weights share the activation quantized once */
        acts_matvec_(m, m->q, m->L[l].w[0], m->L[l].dt[0], m->xb, att_dim, d);
        acts_matvec_(m, m->k, m->L[l].w[1], m->L[l].dt[1], m->xb, kvd, d);
        acts_matvec_(m, m->v, m->L[l].w[2], m->L[l].dt[2], m->xb, kvd, d);
        qk_norm_(m, l, m->q, m->k);
        nro_rope_apply_style(m->q, att_dim, (size_t)m->head_dim, m->freqs, pos, m->neox);
        nro_rope_apply_style(m->k, kvd, (size_t)m->head_dim, m->freqs, pos, m->neox);
        size_t row = ((size_t)l * m->ctx + pos) * kvd;
        for (size_t i = 0; i < kvd; i++) {
            m->kc[row + i] = nro_f32_to_f16(m->k[i]);
            m->vc[row + i] = nro_f32_to_f16(m->v[i]);
        }
        attend_(m, l, pos, m->q, m->attn_out);
        acts_matvec_(m, m->xb2, m->L[l].w[3], m->L[l].dt[3], m->attn_out, d, att_dim);
        for (size_t i = 0; i < d; i++) m->x[i] += m->residual_scale * m->xb2[i]; /* saxpy, vec.rs:68-72 */
        nro_rmsnorm(m->xb, m->x, m->L[l].ffn_norm, d, m->eps);
        acts_matvec_(m, m->gate, m->L[l].w[4], m->L[l].dt[4], m->xb, ffn, d);
        acts_matvec_(m, m->up, m->L[l].w[5], m->L[l].dt[5], m->xb, ffn, d);
        nro_swiglu(m->gate, m->up, ffn);
        acts_matvec_(m, m->xb2, m->L[l].w[6], m->L[l].dt[6], m->gate, d, ffn);
        for (size_t i = 0; i < d; i++) m->x[i] += m->residual_scale * m->xb2[i];
    }
    nro_rmsnorm(m->xb, m->x, m->out_norm, d, m->eps);
    acts_matvec_(m, m->logits, m->output, m->output_dt, m->xb, (size_t)m->vocab, d);
    if (m->logit_recip != 1.0f)
        for (size_t i = 0; i < (size_t)m->vocab; i++) m->logits[i] *= m->logit_recip;
    m->pos += 1;
    return m->logits;
}

/* InferCtx::prefill_chunk (infer.rs:601-750): batched matmuls, per-token
 * rope / KV append / causal attention; logits of the last token. */
const float *nro_model_prefill_chunk(nro_model *m, const uint32_t *tokens, int nb) {
    size_t d = (size_t)m->dim, kvd = (size_t)m->kv_dim, ffn = (size_t)m->ffn_dim;
    size_t att_dim = (size_t)m->n_heads * m->head_dim;
    size_t b = (size_t)nb, base = (size_t)m->pos;
    for (size_t i = 0; i < b; i++) {
        dequant_row_(m->embed, m->embed_dt, tokens[i], d, m->bx + i * d);
        if (m->embed_scale != 1.0f)
            for (size_t j = 0; j < d; j++) m->bx[i * d + j] *= m->embed_scale;
    }
    for (int l = 0; l < m->n_layers; l++) {
        for (size_t i = 0; i < b; i++) nro_rmsnorm(m->bxb + i * d, m->bx + i * d, m->L[l].attn_norm, d, m->eps);
        acts_matmul_(m, m->bq, m->L[l].w[0], m->L[l].dt[0], m->bxb, att_dim, d, b);
        acts_matmul_(m, m->bk, m->L[l].w[1], m->L[l].dt[1], m->bxb, kvd, d, b);
        acts_matmul_(m, m->bv, m->L[l].w[2], m->L[l].dt[2], m->bxb, kvd, d, b);
        for (size_t i = 0; i < b; i++) {
            size_t pos = base + i;
            qk_norm_(m, l, m->bq + i * att_dim, m->bk + i * kvd);
            nro_rope_apply_style(m->bq + i * att_dim, att_dim, (size_t)m->head_dim, m->freqs, pos, m->neox);
            nro_rope_apply_style(m->bk + i * kvd, kvd, (size_t)m->head_dim, m->freqs, pos, m->neox);
            size_t row = ((size_t)l * m->ctx + pos) * kvd;
            for (size_t j = 0; j < kvd; j++) {
                m->kc[row + j] = nro_f32_to_f16(m->bk[i * kvd + j]);
                m->vc[row + j] = nro_f32_to_f16(m->bv[i * kvd + j]);
            }
        }
        for (size_t i = 0; i < b; i++) attend_(m, l, base + i, m->bq + i * att_dim, m->battn + i * att_dim);
        acts_matmul_(m, m->bxb, m->L[l].w[3], m->L[l].dt[3], m->battn, d, att_dim, b);
        for (size_t i = 0; i < b * d; i++) m->bx[i] += m->residual_scale * m->bxb[i];
        for (size_t i = 0; i < b; i++) nro_rmsnorm(m->bxb + i * d, m->bx + i * d, m->L[l].ffn_norm, d, m->eps);
        acts_matmul_(m, m->bgate, m->L[l].w[4], m->L[l].dt[4], m->bxb, ffn, d, b);
        acts_matmul_(m, m->bup, m->L[l].w[5], m->L[l].dt[5], m->bxb, ffn, d, b);
        for (size_t i = 0; i < b; i++) nro_swiglu(m->bgate + i * ffn, m->bup + i * ffn, ffn);
        acts_matmul_(m, m->bxb, m->L[l].w[6], m->L[l].dt[6], m->bgate, d, ffn, b);
        for (size_t i = 0; i < b * d; i++) m->bx[i] += m->residual_scale * m->bxb[i];
    }
    nro_rmsnorm(m->xb, m->bx + (b - 1) * d, m->out_norm, d, m->eps);
    acts_matvec_(m, m->logits, m->output, m->output_dt, m->xb, (size_t)m->vocab, d);
    if (m->logit_recip != 1.0f)
        for (size_t i = 0; i < (size_t)m->vocab; i++) m->logits[i] *= m->logit_recip;
    m->pos += nb;
    return m->logits;
}

/* array forms of the libm restatements (test drivers) */
void nro_expf_n(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = nro_expf(x[i]);
}
void nro_sincosf_n(const float *x, float *s, float *c, size_t n) {
    for (size_t i = 0; i < n; i++) nro_sincosf(x[i], s + i, c + i);
}

/* ---- Sampler (crates/nr-model/src/sample.rs) ---------------------------------------- */

#define NRO_TOP_K 64 /* sample.rs:12 */

/* sample.rs:23-30: xorshift64 (13, 7, 17), then the top 24 bits as a fraction */
float nro_sampler_next_f32(uint64_t *rng) {
    uint64_t x = *rng;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *rng = x;
    return (float)(x >> 40) / (float)(1u << 24);
}

/* sample.rs:32-96. Greedy below temperature 0+; else a 64-slot min-heap keyed
 * on the logit (strict > admits, NaN and -inf never do), the candidates in
 * descending logit order, expf((v - max) / T) summed in that order, the
 * shortest prefix whose running sum reaches top_p * sum, and a draw of
 * next_f32() * that prefix sum. Exact ties among the candidates are ordered
 * by token id here (the reference's unstable sort leaves their order open). */
uint32_t nro_sample(float temperature, float top_p, uint64_t *rng, const float *logits, size_t n) {
    if (temperature <= 0.0f) return nro_argmax(logits, n);
    float hv[NRO_TOP_K];
    uint32_t hi[NRO_TOP_K];
    for (int k = 0; k < NRO_TOP_K; k++) {
        hv[k] = -INFINITY;
        hi[k] = 0;
    }
    for (size_t i = 0; i < n; i++) {
        float v = logits[i];
        if (!(v > hv[0])) continue;
        hv[0] = v;
        hi[0] = (uint32_t)i;
        int j = 0; /* sift down */
        for (;;) {
            int l = 2 * j + 1, r = 2 * j + 2, m = j;
            if (l < NRO_TOP_K && hv[l] < hv[m]) m = l;
            if (r < NRO_TOP_K && hv[r] < hv[m]) m = r;
            if (m == j) break;
            float tv = hv[j]; hv[j] = hv[m]; hv[m] = tv;
            uint32_t ti = hi[j]; hi[j] = hi[m]; hi[m] = ti;
            j = m;
        }
    }
    /* descending by logit (insertion sort; ties by token id) */
    float cv[NRO_TOP_K];
    uint32_t ci[NRO_TOP_K];
    for (int k = 0; k < NRO_TOP_K; k++) {
        float v = hv[k];
        uint32_t id = hi[k];
        int p = k;
        while (p > 0 && (cv[p - 1] < v || (cv[p - 1] == v && ci[p - 1] > id))) {
            cv[p] = cv[p - 1];
            ci[p] = ci[p - 1];
            p--;
        }
        cv[p] = v;
        ci[p] = id;
    }
    float mx = cv[0], sum = 0.0f, probs[NRO_TOP_K];
    for (int k = 0; k < NRO_TOP_K; k++) {
        probs[k] = nro_expf((cv[k] - mx) / temperature);
        sum += probs[k];
    }
    float cut = top_p * sum, cum = 0.0f;
    int nn = NRO_TOP_K;
    for (int k = 0; k < NRO_TOP_K; k++) {
        cum += probs[k];
        if (cum >= cut) {
            nn = k + 1;
            break;
        }
    }
    float r = nro_sampler_next_f32(rng) * cum, acc = 0.0f;
    for (int k = 0; k < nn; k++) {
        acc += probs[k];
        if (r <= acc) return ci[k];
    }
    return ci[nn - 1];
}
