/*
 * CPU oracle for the quantized matrix path — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file, as the checker. The product library never links it.
 *
 * Plain-C restatement of crates/nr-tensor (Rust). Build flags matter:
 * -ffp-contract=off keeps every a*b+c as two rounded operations, as Rust
 * (which never contracts) evaluates them; the AVX2 restatements use explicit
 * _mm256_fmadd_ps exactly where the reference does.
 *
 * Pins (each function is checked against something other than itself):
 *   f16 conversions   reference known values, all 65536 patterns against IEEE,
 *                     hand-built subnormal ties (tests/test_oracle.py)
 *   quantize_q8_0     ties away, the f32 `x + 0.5`, the -127 clamp, `v * inv`,
 *   quantize_q8k      `amax / 127`, `iscale * v`, `d = 1 / iscale`: hand-derived
 *                     blocks (tests/test_oracle_scalar_steps.py)
 *   dot_q8_scalar     `(acc * dw) * dx` and the block chain
 *                     (tests/test_oracle_scalar_steps.py, tests/test_oracle.py)
 *   dot_q4k/q6k       the f32 step orders of the scalar and AVX2 kernels
 *                     (tests/test_oracle_kquant_order.py,
 *                     tests/test_oracle_scalar_steps.py)
 *   AVX2 dots, x4     the hsum tree and per-block FMA (tests/test_oracle.py,
 *                     tests/test_oracle_kquant_order.py); x4 == 1-wide
 *   unpack, dequant   packer round trips over every 6-bit value
 *   integer sums      brute force on independently unpacked quants
 */
#include "nrq_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <string.h>
#include <time.h>

/* ---- Rust scalar-cast semantics ---------------------------------------- */

/* `f as i32` in Rust saturates and maps NaN to 0. */
static inline int32_t rust_f32_to_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* f32::max: returns the other operand when one is NaN (same as fmaxf). */
static inline float rust_fmax(float a, float b) { return fmaxf(a, b); }

static inline uint16_t rd16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline int16_t rdi16(const uint8_t *p) { int16_t v; memcpy(&v, p, 2); return v; }
static inline float rdf32(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

/* ---- f16.rs ------------------------------------------------------------- */

/* f16.rs:3-23 */
float nro_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t frac = bits & 0x3ff;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign;
        } else {
            uint32_t msb = 31u - (uint32_t)__builtin_clz(frac); /* 0..=9 */
            uint32_t e = 127u - 24u + msb;
            uint32_t f = (frac << (23u - msb)) & 0x7fffffu;
            out = sign | (e << 23) | f;
        }
    } else if (exp == 0x1f) {
        out = sign | 0x7f800000u | (frac << 13);
    } else {
        out = sign | ((exp + 127u - 15u) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* f16.rs:25-56 — normals round to nearest even, subnormals round half up. */
uint16_t nro_f32_to_f16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    uint16_t sign = (uint16_t)((bits >> 31) << 15);
    int32_t exp = (int32_t)((bits >> 23) & 0xff);
    uint32_t frac = bits & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (frac != 0 ? 0x200 : 0));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t f = frac | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        return (uint16_t)(sign | (uint16_t)((f + half) >> shift));
    }
    uint32_t out = (uint32_t)sign | ((uint32_t)e << 10) | (frac >> 13);
    uint32_t round = frac & 0x1fff;
    if (round > 0x1000 || (round == 0x1000 && (out & 1) != 0)) out += 1;
    return (uint16_t)out;
}

/* ---- q8.rs -------------------------------------------------------------- */

/* q8.rs:27-44 */
void nro_quantize_q8_0(const float *src, size_t n, void *out) {
    uint8_t *o = (uint8_t *)out;
    for (size_t b = 0; b < n / NRO_QK8_0; b++) {
        const float *chunk = src + b * NRO_QK8_0;
        uint8_t *blk = o + b * NRO_Q8_0_BYTES;
        float amax = 0.0f;
        for (int i = 0; i < NRO_QK8_0; i++) amax = rust_fmax(amax, fabsf(chunk[i]));
        uint16_t d_bits = nro_f32_to_f16(amax / 127.0f);
        float d = nro_f16_to_f32(d_bits);
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        memcpy(blk, &d_bits, 2);
        for (int i = 0; i < NRO_QK8_0; i++) {
            float x = chunk[i] * inv;
            float r = x >= 0.0f ? x + 0.5f : x - 0.5f;
            int32_t q = rust_f32_to_i32(r);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            blk[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* q8.rs:47-55 */
void nro_dequantize_q8_0(const void *blocks, size_t nblocks, float *out) {
    const uint8_t *p = (const uint8_t *)blocks;
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = p + b * NRO_Q8_0_BYTES;
        float d = nro_f16_to_f32(rd16(blk));
        for (int i = 0; i < NRO_QK8_0; i++) out[b * NRO_QK8_0 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

/* ---- kquant.rs: quantizers and unpack ------------------------------------ */

/* kquant.rs:145-153 */
static inline int32_t nearest_int(float v) {
    return v >= 0.0f ? rust_f32_to_i32(v + 0.5f) : rust_f32_to_i32(v - 0.5f);
}

/* kquant.rs:157-187 */
void nro_quantize_q8k(const float *src, size_t n, void *out) {
    uint8_t *o = (uint8_t *)out;
    for (size_t b = 0; b < n / NRO_QK_K; b++) {
        const float *chunk = src + b * NRO_QK_K;
        uint8_t *blk = o + b * NRO_Q8K_BYTES;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < NRO_QK_K; i++) {
            float a = fabsf(chunk[i]);
            if (a > amax) { amax = a; max = chunk[i]; }
        }
        if (amax == 0.0f) {
            memset(blk, 0, NRO_Q8K_BYTES);
            continue;
        }
        float iscale = -128.0f / max;
        int8_t qs[NRO_QK_K];
        for (int i = 0; i < NRO_QK_K; i++) {
            int32_t q = nearest_int(iscale * chunk[i]);
            if (q > 127) q = 127;
            qs[i] = (int8_t)q; /* `as i8` keeps the low byte */
        }
        memcpy(blk + 4, qs, NRO_QK_K);
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int k = 0; k < 16; k++) s += qs[j * 16 + k];
            int16_t s16 = (int16_t)s;
            memcpy(blk + 260 + 2 * j, &s16, 2);
        }
        float d = 1.0f / iscale;
        memcpy(blk, &d, 4);
    }
}

/* kquant.rs:83-92 */
void nro_q4k_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* kquant.rs:95-118 */
void nro_dequant_q4k(const void *block, float *out) {
    const uint8_t *b = (const uint8_t *)block;
    float d = nro_f16_to_f32(rd16(b));
    float dmin = nro_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4, *qs = b + 16;
    int is = 0, y = 0;
    for (int chunk = 0; chunk < 4; chunk++) {
        const uint8_t *q = qs + chunk * 32;
        uint8_t sc1, m1, sc2, m2;
        nro_q4k_scale_min(scales, is, &sc1, &m1);
        nro_q4k_scale_min(scales, is + 1, &sc2, &m2);
        float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        for (int k = 0; k < 32; k++) out[y++] = d1 * (float)(q[k] & 0x0F) - min1;
        for (int k = 0; k < 32; k++) out[y++] = d2 * (float)(q[k] >> 4) - min2;
        is += 2;
    }
}

/* kquant.rs:121-142 */
void nro_dequant_q6k(const void *block, float *out) {
    const uint8_t *b = (const uint8_t *)block;
    float d = nro_f16_to_f32(rd16(b + 208));
    const int8_t *scales = (const int8_t *)(b + 192);
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = b + half * 64;
        const uint8_t *qh = b + 128 + half * 32;
        const int8_t *sc = scales + half * 8;
        float *y = out + half * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int32_t q1 = (int32_t)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
            int32_t q2 = (int32_t)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int32_t q3 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int32_t q4 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* kquant.rs:647-712 */
void nro_quantize_q4k_ref(const float *src, void *out_block) {
    float sub_scale[8], sub_min[8];
    for (int j = 0; j < 8; j++) {
        const float *s = src + j * 32;
        float max = -3.40282347e38f, min = 3.40282347e38f;
        for (int k = 0; k < 32; k++) { max = rust_fmax(max, s[k]); min = fminf(min, s[k]); }
        sub_min[j] = rust_fmax(-min, 0.0f);
        sub_scale[j] = rust_fmax((max + sub_min[j]) / 15.0f, 0.0f);
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) { max_scale = rust_fmax(max_scale, sub_scale[j]); max_min = rust_fmax(max_min, sub_min[j]); }
    float d = max_scale / 63.0f, dmin = max_min / 63.0f;
    float df = nro_f16_to_f32(nro_f32_to_f16(d));
    float dminf = nro_f16_to_f32(nro_f32_to_f16(dmin));
    uint8_t scales6[8], mins6[8];
    for (int j = 0; j < 8; j++) {
        scales6[j] = df > 0.0f ? (uint8_t)clampi(nearest_int(sub_scale[j] / df), 0, 63) : 0;
        mins6[j] = dminf > 0.0f ? (uint8_t)clampi(nearest_int(sub_min[j] / dminf), 0, 63) : 0;
    }
    uint8_t *b = (uint8_t *)out_block;
    uint8_t scales[12];
    for (int j = 0; j < 4; j++) {
        scales[j] = (uint8_t)((scales6[j] & 63) | ((scales6[j + 4] >> 4) << 6));
        scales[j + 4] = (uint8_t)((mins6[j] & 63) | ((mins6[j + 4] >> 4) << 6));
        scales[j + 8] = (uint8_t)((scales6[j + 4] & 0x0F) | ((mins6[j + 4] & 0x0F) << 4));
    }
    uint8_t qs[128];
    memset(qs, 0, sizeof qs);
    for (int j = 0; j < 8; j++) {
        float sc = df * (float)scales6[j];
        float m = dminf * (float)mins6[j];
        const float *s = src + j * 32;
        int chunk = j / 2, hi = j % 2 == 1;
        for (int k = 0; k < 32; k++) {
            uint8_t q = sc > 0.0f ? (uint8_t)clampi(nearest_int((s[k] + m) / sc), 0, 15) : 0;
            if (hi) qs[chunk * 32 + k] |= (uint8_t)(q << 4);
            else qs[chunk * 32 + k] |= q;
        }
    }
    uint16_t dh = nro_f32_to_f16(d), dmh = nro_f32_to_f16(dmin);
    memcpy(b, &dh, 2);
    memcpy(b + 2, &dmh, 2);
    memcpy(b + 4, scales, 12);
    memcpy(b + 16, qs, 128);
}

/* kquant.rs:715-771 */
void nro_quantize_q6k_ref(const float *src, void *out_block) {
    float group_amax[16];
    for (int g = 0; g < 16; g++) {
        float m = 0.0f;
        for (int k = 0; k < 16; k++) m = rust_fmax(m, fabsf(src[g * 16 + k]));
        group_amax[g] = m;
    }
    float amax = 0.0f;
    for (int g = 0; g < 16; g++) amax = rust_fmax(amax, group_amax[g]);
    float d = amax / (127.0f * 31.0f);
    float df = nro_f16_to_f32(nro_f32_to_f16(d));
    int8_t scales[16];
    for (int g = 0; g < 16; g++)
        scales[g] = df > 0.0f ? (int8_t)clampi(nearest_int(group_amax[g] / (df * 31.0f)), -128, 127) : 0;
    uint8_t ql[128], qh[64];
    memset(ql, 0, sizeof ql);
    memset(qh, 0, sizeof qh);
    /* (slot, qh_shift, ql_idx, hi) per kquant.rs:759-762 */
    static const int slot_shift[4] = {0, 2, 4, 6};
    static const int slot_off[4] = {0, 32, 0, 32};
    static const int slot_hi[4] = {0, 0, 1, 1};
    for (int half = 0; half < 2; half++) {
        for (int l = 0; l < 32; l++) {
            for (int slot = 0; slot < 4; slot++) {
                int g = (half * 128 + slot * 32 + l) / 16;
                float sc = df * (float)scales[g];
                float v = src[half * 128 + slot * 32 + l];
                uint8_t q = sc != 0.0f ? (uint8_t)clampi(nearest_int(v / sc) + 32, 0, 63) : 32;
                uint8_t lo = q & 0x0F, hib = (q >> 4) & 3;
                int qli = half * 64 + l + slot_off[slot];
                if (slot_hi[slot]) ql[qli] |= (uint8_t)(lo << 4);
                else ql[qli] |= lo;
                qh[half * 32 + l] |= (uint8_t)(hib << slot_shift[slot]);
            }
        }
    }
    uint8_t *b = (uint8_t *)out_block;
    memcpy(b, ql, 128);
    memcpy(b + 128, qh, 64);
    memcpy(b + 192, scales, 16);
    uint16_t dh = nro_f32_to_f16(d);
    memcpy(b + 208, &dh, 2);
}

/* ---- scalar dots ---------------------------------------------------------- */

/* kernels.rs:72-82 */
float nro_dot_q8_scalar(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q8_0_BYTES, *bx = px + b * NRO_Q8_0_BYTES;
        int32_t acc = 0;
        for (int i = 0; i < NRO_QK8_0; i++) acc += (int32_t)(int8_t)bw[2 + i] * (int32_t)(int8_t)bx[2 + i];
        sum += (float)acc * nro_f16_to_f32(rd16(bw)) * nro_f16_to_f32(rd16(bx));
    }
    return sum;
}

/* kquant.rs:192-218 */
float nro_dot_q4k_scalar(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q4K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
        float xd = rdf32(bx);
        float d_all = nro_f16_to_f32(rd16(bw)) * xd;
        float dmin_all = nro_f16_to_f32(rd16(bw + 2)) * xd;
        const uint8_t *scales = bw + 4, *qs = bw + 16;
        const int8_t *q8all = (const int8_t *)(bx + 4);
        float sum_q = 0.0f;
        int32_t sum_m = 0;
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            nro_q4k_scale_min(scales, j, &sc, &m);
            int32_t sub = 0;
            const uint8_t *q = qs + (j / 2) * 32;
            const int8_t *q8 = q8all + j * 32;
            int hi = j % 2 == 1;
            for (int k = 0; k < 32; k++) {
                int32_t qv = hi ? (q[k] >> 4) : (q[k] & 0x0F);
                sub += qv * (int32_t)q8[k];
            }
            sum_q += (float)sc * (float)sub;
            sum_m += (int32_t)m * ((int32_t)rdi16(bx + 260 + 4 * j) + (int32_t)rdi16(bx + 262 + 4 * j));
        }
        sumf += d_all * sum_q - dmin_all * (float)sum_m;
    }
    return sumf;
}

static void q6k_group_sums(const uint8_t *bw, const uint8_t *bx, int half, int32_t gs[8]) {
    const uint8_t *ql = bw + half * 64, *qh = bw + 128 + half * 32;
    const int8_t *q8 = (const int8_t *)(bx + 4) + half * 128;
    for (int g = 0; g < 8; g++) gs[g] = 0;
    for (int l = 0; l < 32; l++) {
        int32_t q1 = (int32_t)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
        int32_t q2 = (int32_t)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int32_t q3 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int32_t q4 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        gs[l / 16] += q1 * q8[l];
        gs[2 + l / 16] += q2 * q8[l + 32];
        gs[4 + l / 16] += q3 * q8[l + 64];
        gs[6 + l / 16] += q4 * q8[l + 96];
    }
}

/* kquant.rs:220-250 */
float nro_dot_q6k_scalar(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q6K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
        float d_all = nro_f16_to_f32(rd16(bw + 208)) * rdf32(bx);
        const int8_t *scales = (const int8_t *)(bw + 192);
        float sum = 0.0f;
        for (int half = 0; half < 2; half++) {
            int32_t gs[8];
            q6k_group_sums(bw, bx, half, gs);
            for (int g = 0; g < 8; g++) sum += (float)scales[half * 8 + g] * (float)gs[g];
        }
        sumf += d_all * sum;
    }
    return sumf;
}

size_t nro_block_sums(int dtype, const void *w, const void *x, size_t nb, int32_t *out) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    size_t n = 0;
    for (size_t b = 0; b < nb; b++) {
        if (dtype == NRO_Q8_0) {
            const uint8_t *bw = pw + b * NRO_Q8_0_BYTES, *bx = px + b * NRO_Q8_0_BYTES;
            int32_t acc = 0;
            for (int i = 0; i < 32; i++) acc += (int32_t)(int8_t)bw[2 + i] * (int32_t)(int8_t)bx[2 + i];
            out[n++] = acc;
        } else if (dtype == NRO_Q4K) {
            const uint8_t *bw = pw + b * NRO_Q4K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
            const int8_t *q8all = (const int8_t *)(bx + 4);
            int32_t sum_m = 0;
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                nro_q4k_scale_min(bw + 4, j, &sc, &m);
                const uint8_t *q = bw + 16 + (j / 2) * 32;
                int32_t sub = 0;
                for (int k = 0; k < 32; k++) {
                    int32_t qv = (j & 1) ? (q[k] >> 4) : (q[k] & 0x0F);
                    sub += qv * (int32_t)q8all[j * 32 + k];
                }
                out[n++] = sub;
                sum_m += (int32_t)m * ((int32_t)rdi16(bx + 260 + 4 * j) + (int32_t)rdi16(bx + 262 + 4 * j));
            }
            out[n++] = sum_m;
        } else {
            const uint8_t *bw = pw + b * NRO_Q6K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
            for (int half = 0; half < 2; half++) {
                int32_t gs[8];
                q6k_group_sums(bw, bx, half, gs);
                for (int g = 0; g < 8; g++) out[n++] = gs[g];
            }
        }
    }
    return n;
}

/* ---- AVX2 dots ------------------------------------------------------------ */

/* kquant.rs:512-522 (and the inline hsum of kernels.rs:279-285) */
__attribute__((target("avx2,fma"))) static inline float hsum256(__m256 v) {
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 s = _mm_add_ps(hi, lo);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* kernels.rs:263-286 */
__attribute__((target("avx2,fma"))) float nro_dot_q8_avx2(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q8_0_BYTES, *bx = px + b * NRO_Q8_0_BYTES;
        __m256 d = _mm256_set1_ps(nro_f16_to_f32(rd16(bw)) * nro_f16_to_f32(rd16(bx)));
        __m256i qw = _mm256_loadu_si256((const __m256i *)(bw + 2));
        __m256i qx = _mm256_loadu_si256((const __m256i *)(bx + 2));
        __m256i abs_w = _mm256_sign_epi8(qw, qw);
        __m256i sgn_x = _mm256_sign_epi8(qx, qw);
        __m256i p16 = _mm256_maddubs_epi16(abs_w, sgn_x);
        __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(p32), acc);
    }
    return hsum256(acc);
}

/* kernels.rs:229-256 */
__attribute__((target("avx2,fma"))) void nro_dot_q8_avx2_x4(const void *w, const void *const xs[4], size_t nb,
                                                            float out[4]) {
    const uint8_t *pw = (const uint8_t *)w;
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q8_0_BYTES;
        __m256i qw = _mm256_loadu_si256((const __m256i *)(bw + 2));
        __m256i abs_w = _mm256_sign_epi8(qw, qw);
        float dw = nro_f16_to_f32(rd16(bw));
        for (int lane = 0; lane < 4; lane++) {
            const uint8_t *bx = (const uint8_t *)xs[lane] + b * NRO_Q8_0_BYTES;
            __m256 d = _mm256_set1_ps(dw * nro_f16_to_f32(rd16(bx)));
            __m256i qx = _mm256_loadu_si256((const __m256i *)(bx + 2));
            __m256i sgn_x = _mm256_sign_epi8(qx, qw);
            __m256i p16 = _mm256_maddubs_epi16(abs_w, sgn_x);
            __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
            acc[lane] = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(p32), acc[lane]);
        }
    }
    for (int lane = 0; lane < 4; lane++) out[lane] = hsum256(acc[lane]);
}

/* kquant.rs:260-305 */
__attribute__((target("avx2,fma"))) float nro_dot_q4k_avx2(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float acc_min = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q4K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
        float xd = rdf32(bx);
        float d = nro_f16_to_f32(rd16(bw)) * xd;
        float dmin = nro_f16_to_f32(rd16(bw + 2)) * xd;
        uint8_t sc[8], mins[8];
        for (int j = 0; j < 8; j++) nro_q4k_scale_min(bw + 4, j, &sc[j], &mins[j]);
        int32_t min_sum = 0;
        for (int j = 0; j < 8; j++)
            min_sum += (int32_t)mins[j] * ((int32_t)rdi16(bx + 260 + 4 * j) + (int32_t)rdi16(bx + 262 + 4 * j));
        acc_min += dmin * (float)min_sum;
        const uint8_t *qs = bw + 16, *q8 = bx + 4;
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i q4bits = _mm256_loadu_si256((const __m256i *)(qs + j * 32));
            __m256i q4l = _mm256_and_si256(q4bits, m4);
            __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            __m256i q8l = _mm256_loadu_si256((const __m256i *)(q8 + j * 64));
            __m256i q8h = _mm256_loadu_si256((const __m256i *)(q8 + j * 64 + 32));
            __m256i p16l = _mm256_maddubs_epi16(q4l, q8l);
            p16l = _mm256_madd_epi16(_mm256_set1_epi16((int16_t)sc[2 * j]), p16l);
            __m256i p16h = _mm256_maddubs_epi16(q4h, q8h);
            p16h = _mm256_madd_epi16(_mm256_set1_epi16((int16_t)sc[2 * j + 1]), p16h);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p16l, p16h));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum256(acc) - acc_min;
}

/* kquant.rs:317-374 */
__attribute__((target("avx2,fma"))) void nro_dot_q4k_avx2_x4(const void *w, const void *const xs[4], size_t nb,
                                                             float out[4]) {
    const uint8_t *pw = (const uint8_t *)w;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    float acc_min[4] = {0, 0, 0, 0};
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q4K_BYTES;
        float d_w = nro_f16_to_f32(rd16(bw));
        float dmin_w = nro_f16_to_f32(rd16(bw + 2));
        uint8_t sc[8], mins[8];
        for (int j = 0; j < 8; j++) nro_q4k_scale_min(bw + 4, j, &sc[j], &mins[j]);
        const uint8_t *bxs[4];
        for (int lane = 0; lane < 4; lane++) {
            bxs[lane] = (const uint8_t *)xs[lane] + b * NRO_Q8K_BYTES;
            int32_t min_sum = 0;
            for (int j = 0; j < 8; j++)
                min_sum += (int32_t)mins[j] *
                           ((int32_t)rdi16(bxs[lane] + 260 + 4 * j) + (int32_t)rdi16(bxs[lane] + 262 + 4 * j));
            acc_min[lane] += dmin_w * rdf32(bxs[lane]) * (float)min_sum;
        }
        const uint8_t *qs = bw + 16;
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(),
                           _mm256_setzero_si256()};
        for (int j = 0; j < 4; j++) {
            __m256i q4bits = _mm256_loadu_si256((const __m256i *)(qs + j * 32));
            __m256i q4l = _mm256_and_si256(q4bits, m4);
            __m256i q4h = _mm256_and_si256(_mm256_srli_epi16(q4bits, 4), m4);
            __m256i scale_l = _mm256_set1_epi16((int16_t)sc[2 * j]);
            __m256i scale_h = _mm256_set1_epi16((int16_t)sc[2 * j + 1]);
            for (int lane = 0; lane < 4; lane++) {
                const uint8_t *q8 = bxs[lane] + 4;
                __m256i q8l = _mm256_loadu_si256((const __m256i *)(q8 + j * 64));
                __m256i q8h = _mm256_loadu_si256((const __m256i *)(q8 + j * 64 + 32));
                __m256i p16l = _mm256_madd_epi16(scale_l, _mm256_maddubs_epi16(q4l, q8l));
                __m256i p16h = _mm256_madd_epi16(scale_h, _mm256_maddubs_epi16(q4h, q8h));
                sumi[lane] = _mm256_add_epi32(sumi[lane], _mm256_add_epi32(p16l, p16h));
            }
        }
        for (int lane = 0; lane < 4; lane++) {
            __m256 d = _mm256_set1_ps(d_w * rdf32(bxs[lane]));
            acc[lane] = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(sumi[lane]), acc[lane]);
        }
    }
    for (int lane = 0; lane < 4; lane++) out[lane] = hsum256(acc[lane]) - acc_min[lane];
}

/* The four 6-bit planes of one Q6_K half (kquant.rs:482-494). */
__attribute__((target("avx2,fma"))) static inline void q6k_planes(const uint8_t *bw, int half, __m256i q6[4]) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(3);
    const uint8_t *ql = bw + half * 64, *qh = bw + 128 + half * 32;
    __m256i q4bits1 = _mm256_loadu_si256((const __m256i *)ql);
    __m256i q4bits2 = _mm256_loadu_si256((const __m256i *)(ql + 32));
    __m256i qhbits = _mm256_loadu_si256((const __m256i *)qh);
    __m256i q4h_0 = _mm256_slli_epi16(_mm256_and_si256(qhbits, m2), 4);
    __m256i q4h_1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhbits, 2), m2), 4);
    __m256i q4h_2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhbits, 4), m2), 4);
    __m256i q4h_3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhbits, 6), m2), 4);
    q6[0] = _mm256_or_si256(_mm256_and_si256(q4bits1, m4), q4h_0);
    q6[1] = _mm256_or_si256(_mm256_and_si256(q4bits2, m4), q4h_1);
    q6[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits1, 4), m4), q4h_2);
    q6[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q4bits2, 4), m4), q4h_3);
}

/* kquant.rs:454-510 */
__attribute__((target("avx2,fma"))) float nro_dot_q6k_avx2(const void *w, const void *x, size_t nb) {
    const uint8_t *pw = (const uint8_t *)w, *px = (const uint8_t *)x;
    const __m256i m32s = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q6K_BYTES, *bx = px + b * NRO_Q8K_BYTES;
        float d = nro_f16_to_f32(rd16(bw + 208)) * rdf32(bx);
        const int8_t *scales = (const int8_t *)(bw + 192);
        __m256i sumi = _mm256_setzero_si256();
        for (int half = 0; half < 2; half++) {
            const uint8_t *q8 = bx + 4 + half * 128;
            const int8_t *sc = scales + half * 8;
            __m256i q6[4];
            q6k_planes(bw, half, q6);
            for (int n = 0; n < 4; n++) {
                __m256i q8v = _mm256_loadu_si256((const __m256i *)(q8 + n * 32));
                __m256i corr = _mm256_maddubs_epi16(m32s, q8v);
                __m256i p16 = _mm256_maddubs_epi16(q6[n], q8v);
                p16 = _mm256_sub_epi16(p16, corr);
                __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc[2 * n + 1]), _mm_set1_epi16(sc[2 * n]));
                p16 = _mm256_madd_epi16(scv, p16);
                sumi = _mm256_add_epi32(sumi, p16);
            }
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum256(acc);
}

/* kquant.rs:383-448 */
__attribute__((target("avx2,fma"))) void nro_dot_q6k_avx2_x4(const void *w, const void *const xs[4], size_t nb,
                                                             float out[4]) {
    const uint8_t *pw = (const uint8_t *)w;
    const __m256i m32s = _mm256_set1_epi8(32);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *bw = pw + b * NRO_Q6K_BYTES;
        float d_w = nro_f16_to_f32(rd16(bw + 208));
        const int8_t *scales = (const int8_t *)(bw + 192);
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(),
                           _mm256_setzero_si256()};
        for (int half = 0; half < 2; half++) {
            const int8_t *sc = scales + half * 8;
            __m256i q6[4];
            q6k_planes(bw, half, q6);
            for (int n = 0; n < 4; n++) {
                __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc[2 * n + 1]), _mm_set1_epi16(sc[2 * n]));
                for (int lane = 0; lane < 4; lane++) {
                    const uint8_t *q8 = (const uint8_t *)xs[lane] + b * NRO_Q8K_BYTES + 4 + half * 128;
                    __m256i q8v = _mm256_loadu_si256((const __m256i *)(q8 + n * 32));
                    __m256i corr = _mm256_maddubs_epi16(m32s, q8v);
                    __m256i p16 = _mm256_sub_epi16(_mm256_maddubs_epi16(q6[n], q8v), corr);
                    sumi[lane] = _mm256_add_epi32(sumi[lane], _mm256_madd_epi16(scv, p16));
                }
            }
        }
        for (int lane = 0; lane < 4; lane++) {
            const uint8_t *bx = (const uint8_t *)xs[lane] + b * NRO_Q8K_BYTES;
            __m256 d = _mm256_set1_ps(d_w * rdf32(bx));
            acc[lane] = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(sumi[lane]), acc[lane]);
        }
    }
    for (int lane = 0; lane < 4; lane++) out[lane] = hsum256(acc[lane]);
}

/* ---- row pool (parallel.rs:14-105) ------------------------------------------ */

typedef void (*range_fn)(void *ctx, size_t r0, size_t r1);

#define NRO_MAX_WORKERS 255
static struct {
    atomic_size_t seq, cursor, total, chunk, done, active, ready;
    _Atomic(range_fn) fn;
    _Atomic(void *) ctx;
    int nworkers;
    pthread_t th[NRO_MAX_WORKERS];
    pthread_mutex_t grow;
} P = {.grow = PTHREAD_MUTEX_INITIALIZER};

/* parallel.rs:74-84 */
static void pool_drain(void) {
    size_t total = atomic_load(&P.total);
    size_t chunk = atomic_load(&P.chunk);
    if (chunk == 0) chunk = 1;
    range_fn fn = atomic_load(&P.fn);
    void *ctx = atomic_load(&P.ctx);
    for (;;) {
        size_t start = atomic_fetch_add(&P.cursor, chunk);
        if (start >= total) break;
        size_t end = start + chunk < total ? start + chunk : total;
        fn(ctx, start, end);
    }
}

/* parallel.rs:57-72; idles with a short sleep after a long spin so that an
 * idle pool does not keep host cores busy between timed runs. */
static void *pool_worker(void *arg) {
    size_t id = (size_t)arg;
    size_t last = atomic_load(&P.seq);
    atomic_fetch_add(&P.ready, 1); /* parallel.rs:58 */
    unsigned long spins = 0;
    for (;;) {
        size_t s = atomic_load(&P.seq);
        if (s != last) {
            last = s;
            spins = 0;
            if (id < atomic_load(&P.active)) {
                pool_drain();
                atomic_fetch_add(&P.done, 1);
            }
            continue;
        }
        if (++spins < (1ul << 22)) {
            _mm_pause();
        } else {
            struct timespec ts = {0, 50000};
            nanosleep(&ts, NULL);
        }
    }
    return NULL;
}

/* parallel.rs:88-105 with n = threads - 1 workers */
static void pool_run(size_t total, range_fn fn, void *ctx, int threads) {
    size_t n = threads > 1 ? (size_t)(threads - 1) : 0;
    if (n > NRO_MAX_WORKERS) n = NRO_MAX_WORKERS;
    if (n == 0 || total < 128) {
        fn(ctx, 0, total);
        return;
    }
    pthread_mutex_lock(&P.grow);
    while ((size_t)P.nworkers < n) {
        pthread_create(&P.th[P.nworkers], NULL, pool_worker, (void *)(size_t)P.nworkers);
        P.nworkers++;
    }
    /* like POOL.activate (parallel.rs:47-50): post only once every worker
     * has read the current seq */
    while (atomic_load(&P.ready) < (size_t)P.nworkers) _mm_pause();
    atomic_store(&P.active, n);
    atomic_store(&P.fn, fn);
    atomic_store(&P.ctx, ctx);
    atomic_store(&P.total, total);
    atomic_store(&P.cursor, 0);
    size_t chunk = total / ((n + 1) * 4);
    atomic_store(&P.chunk, chunk < 16 ? 16 : chunk);
    atomic_store(&P.done, 0);
    atomic_fetch_add(&P.seq, 1);
    pool_drain();
    while (atomic_load(&P.done) < n) _mm_pause();
    pthread_mutex_unlock(&P.grow);
}

/* ---- matvec / matmul --------------------------------------------------------- */

typedef float (*dot1_fn)(const void *, const void *, size_t);
typedef void (*dot4_fn)(const void *, const void *const[4], size_t, float[4]);

typedef struct {
    float *y;
    const uint8_t *w, *x;
    size_t rows, bpr, batch, wbytes, xbytes;
    dot1_fn dot1;
    dot4_fn dot4; /* NULL: scalar order, no 4-wide tiles */
} mv_ctx;

static void select_kernels(int dtype, int order, dot1_fn *d1, dot4_fn *d4, size_t *wb, size_t *xb, size_t *qk) {
    int avx = order == NRO_ORDER_AVX2;
    if (dtype == NRO_Q8_0) {
        *d1 = avx ? nro_dot_q8_avx2 : nro_dot_q8_scalar;
        *d4 = avx ? nro_dot_q8_avx2_x4 : NULL;
        *wb = NRO_Q8_0_BYTES; *xb = NRO_Q8_0_BYTES; *qk = NRO_QK8_0;
    } else if (dtype == NRO_Q4K) {
        *d1 = avx ? nro_dot_q4k_avx2 : nro_dot_q4k_scalar;
        *d4 = avx ? nro_dot_q4k_avx2_x4 : NULL;
        *wb = NRO_Q4K_BYTES; *xb = NRO_Q8K_BYTES; *qk = NRO_QK_K;
    } else {
        *d1 = avx ? nro_dot_q6k_avx2 : nro_dot_q6k_scalar;
        *d4 = avx ? nro_dot_q6k_avx2_x4 : NULL;
        *wb = NRO_Q6K_BYTES; *xb = NRO_Q8K_BYTES; *qk = NRO_QK_K;
    }
}

/* kernels.rs:50-70 / kquant.rs:549-557 */
static void matvec_range(void *vctx, size_t r0, size_t r1) {
    mv_ctx *c = (mv_ctx *)vctx;
    for (size_t r = r0; r < r1; r++) c->y[r] = c->dot1(c->w + r * c->bpr * c->wbytes, c->x, c->bpr);
}

/* kernels.rs:105-142 / kquant.rs:584-621 */
static void matmul_range(void *vctx, size_t r0, size_t r1) {
    mv_ctx *c = (mv_ctx *)vctx;
    size_t xrow = c->bpr * c->xbytes;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t *row = c->w + r * c->bpr * c->wbytes;
        size_t b = 0;
        while (c->dot4 && b + 4 <= c->batch) {
            const void *xs[4] = {c->x + b * xrow, c->x + (b + 1) * xrow, c->x + (b + 2) * xrow, c->x + (b + 3) * xrow};
            float v[4];
            c->dot4(row, xs, c->bpr, v);
            for (int i = 0; i < 4; i++) c->y[(b + i) * c->rows + r] = v[i];
            b += 4;
        }
        for (; b < c->batch; b++) c->y[b * c->rows + r] = c->dot1(row, c->x + b * xrow, c->bpr);
    }
}

void nro_matvec(int dtype, int order, float *y, const void *w, const void *x, size_t rows, size_t cols,
                int threads) {
    mv_ctx c;
    size_t qk;
    dot4_fn d4;
    select_kernels(dtype, order, &c.dot1, &d4, &c.wbytes, &c.xbytes, &qk);
    c.dot4 = NULL;
    c.y = y; c.w = (const uint8_t *)w; c.x = (const uint8_t *)x;
    c.rows = rows; c.bpr = cols / qk; c.batch = 1;
    pool_run(rows, matvec_range, &c, threads);
}

void nro_matmul(int dtype, int order, float *y, const void *w, const void *xs, size_t rows, size_t cols,
                size_t batch, int threads) {
    mv_ctx c;
    size_t qk;
    select_kernels(dtype, order, &c.dot1, &c.dot4, &c.wbytes, &c.xbytes, &qk);
    c.y = y; c.w = (const uint8_t *)w; c.x = (const uint8_t *)xs;
    c.rows = rows; c.bpr = cols / qk; c.batch = batch;
    pool_run(rows, matmul_range, &c, threads);
}

/* ---- xorshift generators (tests/kernels.rs:9-29, tests/kquant.rs:7-39) ---------- */

uint64_t nro_rng_next(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

float nro_rng_f32(uint64_t *s) {
    return (float)(nro_rng_next(s) >> 40) / (float)(1ull << 23) * 2.0f - 1.0f;
}

void nro_rng_vec(uint64_t *s, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = nro_rng_f32(s);
}

void nro_rng_adversarial(uint64_t *s, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        switch (nro_rng_next(s) % 7) {
        case 0: out[i] = 0.0f; break;
        case 1: out[i] = 100.0f * nro_rng_f32(s); break;
        case 2: out[i] = 1e-4f * nro_rng_f32(s); break;
        case 3: out[i] = -50.0f + nro_rng_f32(s); break;
        default: out[i] = nro_rng_f32(s) * (float)(1 + i % 13); break;
        }
    }
}

static double rng_unit(uint64_t *s) { /* (0, 1] */
    return ((double)(nro_rng_next(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void nro_rng_normal(uint64_t *s, float *out, size_t n, float sigma) {
    for (size_t i = 0; i < n; i += 2) {
        double u1 = rng_unit(s), u2 = rng_unit(s);
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586 * u2;
        out[i] = (float)(r * cos(t)) * sigma;
        if (i + 1 < n) out[i + 1] = (float)(r * sin(t)) * sigma;
    }
}

void nro_rng_bytes(uint64_t *s, uint8_t *out, size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t v = nro_rng_next(s);
        memcpy(out + i, &v, 8);
    }
    if (i < n) {
        uint64_t v = nro_rng_next(s);
        memcpy(out + i, &v, n - i);
    }
}

void nro_gen_weights(int dtype, uint64_t seed, void *out, size_t nblocks) {
    uint64_t s = seed ? seed : 0x9E3779B97F4A7C15ull;
    uint8_t *o = (uint8_t *)out;
    float g[2];
    for (size_t b = 0; b < nblocks; b++) {
        if (dtype == NRO_Q8_0) {
            uint8_t *blk = o + b * NRO_Q8_0_BYTES;
            nro_rng_normal(&s, g, 1, 0.02f);
            uint16_t d = nro_f32_to_f16(fabsf(g[0]) / 127.0f);
            memcpy(blk, &d, 2);
            for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)((int)(nro_rng_next(&s) % 255) - 127);
        } else if (dtype == NRO_Q4K) {
            uint8_t *blk = o + b * NRO_Q4K_BYTES;
            nro_rng_normal(&s, g, 2, 0.01f);
            uint16_t d = nro_f32_to_f16(fabsf(g[0])), dm = nro_f32_to_f16(fabsf(g[1]));
            memcpy(blk, &d, 2);
            memcpy(blk + 2, &dm, 2);
            nro_rng_bytes(&s, blk + 4, 140);
        } else {
            uint8_t *blk = o + b * NRO_Q6K_BYTES;
            nro_rng_bytes(&s, blk, 208);
            nro_rng_normal(&s, g, 1, 0.01f);
            uint16_t d = nro_f32_to_f16(fabsf(g[0]));
            memcpy(blk + 208, &d, 2);
        }
    }
}
