/*
 * CPU oracle for the quantized matrix path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's nr-tensor kernels, used as the
 * checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg. Nothing in the product (libnrq) links, loads or calls it.
 *
 * Every function cites the reference file:line it restates. The reference
 * is Rust (crates/nr-tensor) and cannot be built in this image, so there is
 * no compiled reference build beside this restatement; each function is
 * pinned instead by the reference tests' known values, properties and
 * closed forms (see tests/test_oracle.py).
 *
 * Block layouts (little-endian, packed), identical to the reference:
 *   Q8_0 : d:f16@0  qs:i8[32]@2                                  34 B
 *   Q4_K : d:f16@0  dmin:f16@2  scales:u8[12]@4  qs:u8[128]@16    144 B
 *   Q6_K : ql:u8[128]@0  qh:u8[64]@128  scales:i8[16]@192  d:f16@208  210 B
 *   Q8_K : d:f32@0  qs:i8[256]@4  bsums:i16[16]@260              292 B
 */
#ifndef NRQ_ORACLE_H
#define NRQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NRO_QK8_0 32
#define NRO_QK_K 256
#define NRO_Q8_0_BYTES 34
#define NRO_Q4K_BYTES 144
#define NRO_Q6K_BYTES 210
#define NRO_Q8K_BYTES 292

/* dtype ids follow TensorDtype (crates/nr-model/src/format.rs:97-102) */
#define NRO_Q8_0 1
#define NRO_Q4K 2
#define NRO_Q6K 3

/* f32 summation order of the CPU kernel being restated */
#define NRO_ORDER_SCALAR 0 /* dot_*_scalar (== the NEON kernels bit for bit) */
#define NRO_ORDER_AVX2 1   /* dot_*_avx2 / dot_*_avx2_x4 */

/* f16.rs:3-23, f16.rs:25-56 */
float nro_f16_to_f32(uint16_t bits);
uint16_t nro_f32_to_f16(float v);

/* q8.rs:27-44 (quantize), q8.rs:47-55 (dequantize) */
void nro_quantize_q8_0(const float *src, size_t n, void *out);
void nro_dequantize_q8_0(const void *blocks, size_t nblocks, float *out);

/* kquant.rs:157-187 */
void nro_quantize_q8k(const float *src, size_t n, void *out);
/* kquant.rs:83-92 */
void nro_q4k_scale_min(const uint8_t *scales12, int j, uint8_t *sc, uint8_t *m);
/* kquant.rs:95-118, kquant.rs:121-142 */
void nro_dequant_q4k(const void *block, float *out256);
void nro_dequant_q6k(const void *block, float *out256);
/* kquant.rs:647-712, kquant.rs:715-771 (test-support quantizers) */
void nro_quantize_q4k_ref(const float *src256, void *out_block);
void nro_quantize_q6k_ref(const float *src256, void *out_block);

/* kernels.rs:72-82 */
float nro_dot_q8_scalar(const void *w, const void *x, size_t nblocks);
/* kernels.rs:263-286, kernels.rs:229-256 */
float nro_dot_q8_avx2(const void *w, const void *x, size_t nblocks);
void nro_dot_q8_avx2_x4(const void *w, const void *const xs[4], size_t nblocks, float out[4]);
/* kquant.rs:192-218, kquant.rs:260-305, kquant.rs:317-374 */
float nro_dot_q4k_scalar(const void *w, const void *x, size_t nblocks);
float nro_dot_q4k_avx2(const void *w, const void *x, size_t nblocks);
void nro_dot_q4k_avx2_x4(const void *w, const void *const xs[4], size_t nblocks, float out[4]);
/* kquant.rs:220-250, kquant.rs:454-510, kquant.rs:383-448 */
float nro_dot_q6k_scalar(const void *w, const void *x, size_t nblocks);
float nro_dot_q6k_avx2(const void *w, const void *x, size_t nblocks);
void nro_dot_q6k_avx2_x4(const void *w, const void *const xs[4], size_t nblocks, float out[4]);

/*
 * Row-parallel matvec / matmul, restating kernels.rs:36-70 / 91-143 and the
 * kquant_matvec!/kquant_matmul! macros (kquant.rs:536-639), with rows split
 * by a pool that follows parallel.rs:86-105 (chunk = max(total/((n+1)*4),16),
 * main thread participates, inline when n == 0 or total < 128).
 * `threads` counts the main thread (1 = inline). y is [batch][rows].
 */
void nro_matvec(int dtype, int order, float *y, const void *w, const void *x,
                size_t rows, size_t cols, int threads);
void nro_matmul(int dtype, int order, float *y, const void *w, const void *xs,
                size_t rows, size_t cols, size_t batch, int threads);

/*
 * Exact integer partial sums of one weight row against one activation row,
 * as the scalar kernels form them before any f32 step:
 *   Q8_0 : out[b]          = sum_32 w*x                  (kernels.rs:75-78)
 *   Q4_K : out[b*9 + j]    = sub_j (j<8), out[b*9+8] = sum_m (kquant.rs:200-214)
 *   Q6_K : out[b*16 + g]   = group_sums over 16 elements, g = 8*half + g'
 *                                                         (kquant.rs:232-242)
 * Returns the number of ints written.
 */
size_t nro_block_sums(int dtype, const void *w, const void *x, size_t nblocks, int32_t *out);

/* xorshift64 (13/7/17) as in the reference tests (tests/kernels.rs:9-29) */
uint64_t nro_rng_next(uint64_t *state);
float nro_rng_f32(uint64_t *state);          /* uniform [-1, 1) */
void nro_rng_vec(uint64_t *state, float *out, size_t n);
void nro_rng_adversarial(uint64_t *state, float *out, size_t n); /* tests/kquant.rs:28-38 */
/* N(0, sigma) by Box-Muller over the same xorshift stream */
void nro_rng_normal(uint64_t *state, float *out, size_t n, float sigma);
/* uniform random bytes from the same stream */
void nro_rng_bytes(uint64_t *state, uint8_t *out, size_t n);

/*
 * Synthetic weight generators for the benchmark shapes:
 *   Q8_0 : d = f16(|N(0,0.02)|/127), qs uniform in [-127,127]
 *   Q4_K : d, dmin = f16(|N(0,0.01)|), random scales[12] and qs[128]
 *   Q6_K : random ql[128], qh[64], scales i8[16], d = f16(|N(0,0.01)|)
 */
void nro_gen_weights(int dtype, uint64_t seed, void *out, size_t nblocks);

/* ---- forward pass (nrq_model_oracle.c) ----------------------------------------- */

/* libm restatements (musl algorithms the reference's libm crate ports) */
float nro_expf(float x);
void nro_sincosf(float x, float *s, float *c);
void nro_expf_n(const float *x, float *y, size_t n);
void nro_sincosf_n(const float *x, float *s, float *c, size_t n);
/* crates/nr-tensor/src/vec.rs:4-14, 30-42, 45-52, 80-90 */
void nro_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void nro_softmax(float *x, size_t n);
void nro_swiglu(float *gate, const float *up, size_t n);
uint32_t nro_argmax(const float *x, size_t n);
/* crates/nr-tensor/src/rope.rs:14-34 (no scaling), 49-65 (adjacent pairs) */
void nro_rope_freqs(float *out, size_t head_dim, float theta);
void nro_rope_apply(float *x, size_t n, size_t head_dim, const float *freqs, size_t pos);

/* InferCtx (crates/nr-model/src/infer.rs) for the Llama recipe.
 * dims = {dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx};
 * weights w[7] = {q, k, v, o, gate, up, down} with their dtype ids. */
typedef struct nro_model nro_model;
nro_model *nro_model_new(const int dims[8], float eps, float theta, int threads);
/* the kernels' f32 order: NRO_ORDER_SCALAR (default) or NRO_ORDER_AVX2, the
 * x86 host's AVX2 matvec dots and F16C attention (kernels.rs:174-220) */
void nro_model_set_order(nro_model *m, int order);
/* dot_f16 / axpy_f16 (kernels.rs:146-173) in the given order */
float nro_dot_f16(int order, const uint16_t *k, const float *q, size_t n);
void nro_axpy_f16(int order, float *out, float a, const uint16_t *v, size_t n);
void nro_model_free(nro_model *m);
void nro_model_set_recipe(nro_model *m, int neox, float embed_scale, float attn_scale, float residual_scale,
                          float logit_scale);
void nro_model_set_qk_norm(nro_model *m, int l, const float *q_norm, const float *k_norm);
void nro_rmsnorm_inplace(float *x, const float *w, size_t n, float eps);
void nro_rope_apply_style(float *x, size_t n, size_t head_dim, const float *freqs, size_t pos, int neox);
void nro_model_set_globals(nro_model *m, const void *embed, int embed_dt, const void *output, int output_dt,
                           const float *out_norm);
void nro_model_set_layer(nro_model *m, int l, const void *const w[7], const int dt[7], const float *attn_norm,
                         const float *ffn_norm);
const float *nro_model_forward(nro_model *m, uint32_t token);                        /* infer.rs:510-595 */
const float *nro_model_prefill_chunk(nro_model *m, const uint32_t *tokens, int n);   /* infer.rs:601-750 */
/* replaces the rope table (head_dim/2 floats), as InferCtx::new fills it (infer.rs:433-447) */
void nro_model_set_freqs(nro_model *m, const float *freqs);
int nro_model_pos(const nro_model *m);
void nro_model_reset(nro_model *m);
void nro_model_seek(nro_model *m, int pos); /* timing aid: skips computing the rows before pos */
const float *nro_model_logits(const nro_model *m);
const uint16_t *nro_model_kcache(const nro_model *m);
const uint16_t *nro_model_vcache(const nro_model *m);

/* Sampler (crates/nr-model/src/sample.rs:23-96); rng is the sampler's state
 * (Sampler::new sets seed | 1). Exact logit ties among the top 64 are ordered
 * by token id. */
float nro_sampler_next_f32(uint64_t *rng);
uint32_t nro_sample(float temperature, float top_p, uint64_t *rng, const float *logits, size_t n);

/* .nrm checksum (crates/nr-model/src/crc32.rs:6-79), zlib running-value
 * convention; the bitwise form is the classic algorithm of
 * crates/nr-model/tests/verify.rs:16-30. */
uint32_t nro_crc32(uint32_t crc, const void *data, size_t n);
uint32_t nro_crc32_bitwise(uint32_t crc, const void *data, size_t n);
/* InferCtx::new's rope table (infer.rs:433-447, rope.rs:14-34); factors may be NULL */
void nro_infer_freqs(float *out, size_t head_dim, float theta, float factor, float low, float high, float orig_ctx,
                     const float *factors);

#ifdef __cplusplus
}
#endif
#endif
