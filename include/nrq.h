/*
 * libnrq — MI355X (gfx950) quantized matrix kernels, C ABI.
 *
 * Drop-in for the quantized kernels of the reference's nr-tensor crate
 * (crates/nr-tensor). Plain pointers and sizes only; every function returns
 * an int status (NRQ_OK = 0) and never unwinds. On failure nrq_last_error()
 * returns a message; shape failures carry the text of the reference
 * assertion they replace, so a binding can re-panic with it.
 *
 * Lengths are element counts of the reference's Rust slices: `w_len`,
 * `x_len` count blocks (BlockQ8_0 = 34 B, BlockQ4K = 144 B, BlockQ6K =
 * 210 B, BlockQ8K = 292 B), `y_len` and `src_len` count f32 values.
 *
 * f32 results are bit-identical to one of the reference's CPU kernels,
 * selected with nrq_set_order():
 *   NRQ_ORDER_SCALAR : dot_q8_scalar / dot_q4k_scalar / dot_q6k_scalar
 *                      (also what the reference's NEON path returns)
 *   NRQ_ORDER_AVX2   : dot_q8_avx2 / dot_q4k_avx2 / dot_q6k_avx2 (x86 fast path)
 */
#ifndef NRQ_H
#define NRQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define NRQ_OK 0
#define NRQ_ERR_ARG (-1)         /* null pointer, unknown dtype/order, misaligned device pointer */
#define NRQ_ERR_SHAPE (-2)       /* a reference assert!/assert_eq! would have panicked */
#define NRQ_ERR_DEVICE (-3)      /* HIP error, or no gfx950 device */
#define NRQ_ERR_UNSUPPORTED (-4) /* row wider than the kernels' LDS tile */
#define NRQ_ERR_NOT_INIT (-5)    /* nrq_init was not called */
/* .nrm files: Model::parse's ParseError variants (crates/nr-model/src/format.rs:217-224)
 * and Model::verify_data's failure (format.rs:409-422, VerifyError::DataCrc) */
#define NRQ_ERR_NRM_TOO_SHORT (-10)      /* ParseError::TooShort */
#define NRQ_ERR_NRM_BAD_MAGIC (-11)      /* ParseError::BadMagic */
#define NRQ_ERR_NRM_BAD_VERSION (-12)    /* ParseError::BadVersion(v) */
#define NRQ_ERR_NRM_META_CRC (-13)       /* ParseError::MetaCrc { expect, got } */
#define NRQ_ERR_NRM_BAD_TABLE (-14)      /* ParseError::BadTable */
#define NRQ_ERR_NRM_MISSING_TENSOR (-15) /* ParseError::MissingTensor(name) */
#define NRQ_ERR_NRM_DATA_CRC (-16)       /* the data section's CRC does not match the header */

/* weight dtypes: TensorDtype ids (crates/nr-model/src/format.rs:97-102) */
#define NRQ_Q8_0 1
#define NRQ_Q4_K 2
#define NRQ_Q6_K 3

/* f32 accumulation order to reproduce */
#define NRQ_ORDER_SCALAR 0
#define NRQ_ORDER_AVX2 1

/* ---- lifecycle ------------------------------------------------------------ */

/* Selects HIP device `device`, checks it is gfx950, creates the library's
 * stream. Replaces the CPU-feature probe cpu::fast_path
 * (crates/nr-tensor/src/cpu.rs:46-49) and the worker-pool bring-up
 * POOL.activate (crates/nr-tensor/src/parallel.rs:47-50). Idempotent. */
int nrq_init(int device);
/* Frees every device buffer and the stream. */
int nrq_shutdown(void);
/* Message of the last failure on this thread ("" if none). */
const char *nrq_last_error(void);
/* "gfx950 <name>, <n> CUs, <bytes> HBM" into buf. */
int nrq_device_info(char *buf, size_t len);

/* Order used by the host-slice entry points below (default NRQ_ORDER_SCALAR).
 * The reference picks AVX2 vs scalar per call with cpu::fast_path()
 * (kernels.rs:58, kquant.rs:544); this is that switch. */
int nrq_set_order(int order);
int nrq_get_order(void);

/* ---- weight residency ------------------------------------------------------- */

/* Copies `bytes` of quantized weights at `host` into HBM once, in their
 * original block layout (no dequantized copy). Later calls whose `w` slice
 * lies inside [host, host+bytes) read the HBM copy. This is the device side
 * of InferCtx::new taking zero-copy weight views
 * (crates/nr-model/src/infer.rs:352-419, format.rs:201-214). Host slices that
 * are not registered are uploaded on every call. */
int nrq_register_weights(const void *host, size_t bytes);
int nrq_unregister_weights(const void *host);

/* ---- nr-tensor API over host slices (synchronous) ----------------------------- */

/* kernels::matvec_q8 (crates/nr-tensor/src/kernels.rs:36-47):
 * y[r] = dot(w[r,:], x); asserts y_len == rows, x_len == cols/32,
 * w_len >= rows*cols/32. */
int nrq_matvec_q8(float *y, size_t y_len, const void *w, size_t w_len, const void *x, size_t x_len, size_t rows,
                  size_t cols);
/* kernels::matmul_q8 (kernels.rs:91-143): y is [batch][rows], xs is
 * [batch][cols/32]; bit-identical to matvec_q8 per batch row. */
int nrq_matmul_q8(float *y, size_t y_len, const void *w, size_t w_len, const void *xs, size_t xs_len, size_t rows,
                  size_t cols, size_t batch);
/* kquant::matvec_q4k / matvec_q6k (crates/nr-tensor/src/kquant.rs:536-564) */
int nrq_matvec_q4k(float *y, size_t y_len, const void *w, size_t w_len, const void *x, size_t x_len, size_t rows,
                   size_t cols);
int nrq_matvec_q6k(float *y, size_t y_len, const void *w, size_t w_len, const void *x, size_t x_len, size_t rows,
                   size_t cols);
/* kquant::matmul_q4k / matmul_q6k (kquant.rs:566-639) */
int nrq_matmul_q4k(float *y, size_t y_len, const void *w, size_t w_len, const void *xs, size_t xs_len, size_t rows,
                   size_t cols, size_t batch);
int nrq_matmul_q6k(float *y, size_t y_len, const void *w, size_t w_len, const void *xs, size_t xs_len, size_t rows,
                   size_t cols, size_t batch);
/* q8::quantize (crates/nr-tensor/src/q8.rs:27-44); asserts src_len == out_len*32 */
int nrq_quantize(const float *src, size_t src_len, void *out, size_t out_len);
/* kquant::quantize_q8k (kquant.rs:157-187); asserts src_len == out_len*256 */
int nrq_quantize_q8k(const float *src, size_t src_len, void *out, size_t out_len);

/* ---- device-resident entry points (asynchronous on `stream`) --------------------
 * All pointers are device pointers; `stream` is a hipStream_t (NULL = the
 * library's stream). Weight pointers must be 16-byte aligned (any HIP
 * allocation is); a weight buffer must stay readable up to the next
 * 16-byte boundary past its end (true of every HIP allocation). */

/* matvec / matmul with an explicit dtype and order; same contracts as above */
int nrq_dev_matvec(int dtype, int order, float *y, const void *w, const void *x, size_t rows, size_t cols,
                   void *stream);
int nrq_dev_matmul(int dtype, int order, float *y, const void *w, const void *xs, size_t rows, size_t cols,
                   size_t batch, void *stream);
/* Acts::matmul_group (crates/nr-model/src/infer.rs:180-228) on the device: n
 * (1-3) matrices of one dtype and width over the same activation blocks,
 * ys[i] = [batch][rows[i]], each bitwise equal to nrq_dev_matmul of that
 * matrix in the scalar order. One launch covers the group where the prefill
 * kernel takes it (else one launch per matrix). */
int nrq_dev_matmul_group(int dtype, int n, float *const *ys, const void *const *ws, const size_t *rows,
                         const void *xs, size_t cols, size_t batch, void *stream);
/* q8::quantize / kquant::quantize_q8k over n f32 values already in HBM */
int nrq_dev_quantize_q8_0(const float *src, size_t n, void *out, void *stream);
int nrq_dev_quantize_q8k(const float *src, size_t n, void *out, void *stream);
/* Exact per-(row, block) integer sums the scalar kernels form before any f32
 * step (kernels.rs:75-78, kquant.rs:200-214, kquant.rs:232-242):
 *   Q8_0: 1 int per block; Q4_K: 8 sub-block sums + sum_m; Q6_K: 16 group sums.
 * out is [rows][cols/QK][1|9|16] int32. Diagnostic path for parity tests. */
int nrq_dev_block_sums(int dtype, const void *w, const void *x, int32_t *out, size_t rows, size_t cols,
                       void *stream);
/* The forward pass's math functions over n f32 values in HBM, for parity
 * tests: fn 0 = expf, 1 = the sine and 2 = the cosine of sincosf (restating
 * the musl algorithms the reference's libm crate ports; vec.rs:30-52,
 * rope.rs:49-65 call them). Diagnostic path. */
int nrq_dev_mathf(int fn, const float *x, float *y, size_t n, void *stream);
/* rmsnorm (crates/nr-tensor/src/vec.rs:4-14) of each of `rows` rows of n f32 in
 * HBM: ss += v*v in element order, scale = 1/sqrtf(ss/n + eps), out = x *
 * scale * w. The decode and prefill steps run the same kernel; n is a multiple
 * of 256, at most 8192. */
int nrq_dev_rmsnorm(const float *x, const float *w, float *out, size_t rows, size_t n, float eps, void *stream);
/* Waits for all work on `stream` (NULL = library stream). */
int nrq_sync(void *stream);
/* A plain streaming read of `bytes` (16-byte aligned units) of device memory,
 * xor-folded (out is written only on a 2^-32 chance): no reference
 * counterpart; the read rate the matvecs are measured against on the same
 * GPU. */
int nrq_dev_stream_read(const void *data, size_t bytes, uint32_t *out, void *stream);

/* ---- decode and prefill of a whole model on one GPU ---------------------------------
 * The forward pass of crates/nr-model/src/infer.rs (InferCtx) for the three
 * recipes it runs (infer.rs:447-461): Llama (adjacent-pair RoPE), Qwen3
 * (per-head q/k RMSNorm, NeoX pairs) and Granite (muP embed / attention /
 * residual / logit scales), with Llama-3 rope scaling or RopeFreqs factors
 * through nrq_model_set_rope_freqs. Layer matrices may be Q8_0, Q4_K or Q6_K
 * in any mix; the embedding (and an untied head) Q8_0, Q4_K or Q6_K. Every
 * tensor is resident in HBM; greedy (sample.rs:32-35) or top-p sampling
 * (sample.rs:36-96). The KV cache holds f16 bits, as the reference's does
 * (infer.rs:297-299).
 * The model always computes in the reference's scalar order, bit-identical to
 * dot_*_scalar (and so to the NEON path); nrq_set_order does not apply to it. */

#define NRQ_F32 0 /* dtype of f32 tensors (norm weights) */

/* tensor kinds: TensorKind ids (crates/nr-model/src/format.rs:53-69) */
#define NRQ_TENSOR_TOK_EMBED 1
#define NRQ_TENSOR_OUTPUT_NORM 2
#define NRQ_TENSOR_OUTPUT 3
#define NRQ_TENSOR_ROPE_FREQS 4
#define NRQ_TENSOR_ATTN_NORM 10
#define NRQ_TENSOR_ATTN_Q 11
#define NRQ_TENSOR_ATTN_K 12
#define NRQ_TENSOR_ATTN_V 13
#define NRQ_TENSOR_ATTN_O 14
#define NRQ_TENSOR_FFN_NORM 15
#define NRQ_TENSOR_FFN_GATE 16
#define NRQ_TENSOR_FFN_UP 17
#define NRQ_TENSOR_FFN_DOWN 18
#define NRQ_TENSOR_ATTN_Q_NORM 19 /* Qwen3 per-head RMSNorm weights, f32[head_dim] */
#define NRQ_TENSOR_ATTN_K_NORM 20

#define NRQ_ROPE_ADJACENT 0 /* RopeStyle (rope.rs:37-44): pairs (2i, 2i+1), Llama / Granite */
#define NRQ_ROPE_NEOX 1     /* pairs (i, i + head_dim/2), Qwen3 */

typedef struct nrq_model nrq_model;

/* Dims (crates/nr-model/src/infer.rs:60-73 Dims, format.rs:126-156 Meta). */
typedef struct {
  int dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx;
  float norm_eps, rope_theta;
} nrq_model_config;

/* InferCtx::new (infer.rs:352-492): device KV cache, scratch, rope table. */
int nrq_model_create(const nrq_model_config *cfg, nrq_model **out);
/* Binds one tensor already in HBM (matrices Q8_0/Q4_K/Q6_K in their block
 * layout; norms NRQ_F32; every tensor 16-byte aligned). The output head is tied to the
 * embedding until an NRQ_TENSOR_OUTPUT is set (infer.rs:415-419). A Q4_K or
 * Q6_K embedding needs dim % 256 == 0; its rows are dequantized as
 * QMat::dequant_row does (infer.rs:36-56). */
int nrq_model_set_tensor(nrq_model *m, int kind, int layer, int dtype, const void *dev_ptr);
/* Replaces the rope table (n = head_dim / 2 host floats), as InferCtx::new
 * fills it from Llama-3 scaling or a RopeFreqs tensor (infer.rs:433-447).
 * nrq_model_create sets the unscaled theta^(-2i/head_dim). */
int nrq_model_set_rope_freqs(nrq_model *m, const float *freqs, int n);
/* The recipe InferCtx::new derives from the file (infer.rs:447-461;
 * replaces its rope_style / embed_scale / att_score_scale / residual_scale /
 * logit_recip fields): rope pairs, muP embedding scale, attention score scale
 * (0 = 1/sqrtf(head_dim)), residual scale (x += s * branch) and logit scale
 * (logits /= s, as * (1/s)). nrq_model_create sets the Llama recipe
 * (NRQ_ROPE_ADJACENT, 1, 0, 1, 1). Qwen3's per-head q/k RMSNorm runs when a
 * layer has NRQ_TENSOR_ATTN_Q_NORM and NRQ_TENSOR_ATTN_K_NORM. */
int nrq_model_set_recipe(nrq_model *m, int rope_style, float embed_scale, float attn_scale, float residual_scale,
                         float logit_scale);
/* InferCtx::reset (infer.rs:494-496). */
int nrq_model_reset(nrq_model *m);
/* InferCtx::pos. */
int nrq_model_pos(const nrq_model *m);
/* InferCtx::forward (infer.rs:510-595): one token at the current position;
 * copies the logits to host `logits` (vocab floats) unless NULL. */
int nrq_model_forward(nrq_model *m, uint32_t token, float *logits);
/* InferCtx::prefill (infer.rs:753-759): the n prompt tokens in chunks of up to
 * 512 tokens (the reference's MAX_BATCH is 64: the KV cache and logits are the same
 * at any chunk size), each chunk as prefill_chunk (infer.rs:601-750) does it:
 * batched norms and matmuls (int8 MFMA), every row's rope and f16 KV append,
 * then causal attention for all (head, token) pairs in one launch. The KV
 * cache and the last token's logits (copied to host `logits`, vocab floats,
 * unless NULL) are bit-identical to n forward steps. */
int nrq_model_prefill(nrq_model *m, const uint32_t *tokens, int n, float *logits);
/* Greedy generation: n steps of forward + argmax (sample.rs:33-35), each
 * step's token feeding the next, device-resident (one HIP graph per step).
 * out_tokens gets the n sampled ids; last_logits (optional) the last step's
 * logits. */
int nrq_model_generate(nrq_model *m, uint32_t token, int n, uint32_t *out_tokens, float *last_logits);
/* One decode step of `token` (as nrq_model_forward, no logits copied back),
 * launched eagerly with a HIP event after each stage; stage_us[0..8] get the
 * microseconds per stage summed over the layers: embed, norm + q|k|v,
 * attention, o, norm + gate|up (+ swiglu), down, final norm, head, argmax or
 * sampler. No reference counterpart: the step's own timing, beside the graph
 * replays of nrq_model_generate. */
int nrq_model_step_profile(nrq_model *m, uint32_t token, float *stage_us, int n_stages);
/* Sampler::new (sample.rs:15-21) for nrq_model_generate: temperature <= 0 is
 * greedy (argmax, the default); otherwise each step draws from the 64 largest
 * logits at `temperature`, cut to the shortest prefix whose probability
 * reaches top_p (sample.rs:32-96), with the xorshift state seed | 1 kept on
 * the device. Exact logit ties among the candidates are ordered by token id. */
int nrq_model_set_sampler(nrq_model *m, float temperature, float top_p, uint64_t seed);
/* The sampler's state after the draws so far. */
int nrq_model_sampler_state(nrq_model *m, uint64_t *state);
/* Sampler::sample over n device logits: the drawn id to the device word
 * *token; *rng (device) is the state, advanced once per draw at temperature
 * > 0. Enqueued on `stream`. */
int nrq_dev_sample(const float *logits, int n, float temperature, float top_p, uint64_t *rng, uint32_t *token,
                   void *stream);
/* nrq_dev_sample without allocation. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The partial
 * top-64 lists go to a fixed 128 KiB array per device, held until the process
 * ends, instead of stream-ordered memory; n is at most 524288 logits (else
 * NRQ_ERR_UNSUPPORTED). The array belongs to the current device, and `stream`
 * (NULL = the null stream) must be on that device. Every call on a device
 * shares the array: calls that overlap on one device (different streams or
 * threads) race and must not run concurrently. Same results as nrq_dev_sample. */
int nrq_dev_sample_noalloc(const float *logits, int n, float temperature, float top_p, uint64_t *rng,
                           uint32_t *token, void *stream);
/* Copies the f16 KV cache ([n_layers][ctx][kv_dim] each) to host buffers. */
int nrq_model_kv_cache(nrq_model *m, void *k, void *v, size_t bytes);
int nrq_model_destroy(nrq_model *m);

/* ---- .nrm v3 model files (crates/nr-model/src/format.rs, crc32.rs) -------------------
 * Layout: 192-byte header | tokenizer blob | tensor table (32-byte entries) |
 * data section (each tensor 64-byte aligned). meta_crc covers the header (its
 * two CRC fields as zeros), the tokenizer blob and the table; data_crc the
 * data section. CRC-32 is IEEE (reflected 0xEDB88320). */

#define NRQ_ARCH_LLAMA3 1 /* Arch (format.rs:23-29) */
#define NRQ_ARCH_QWEN3 2
#define NRQ_ARCH_GRANITE 3
#define NRQ_NRM_FLAG_TIED_EMBEDDINGS 1 /* format.rs:21 */
#define NRQ_NRM_VERIFY_DATA 1          /* nrq_model_load_nrm flag: check data_crc on the device copy */

/* Meta (format.rs:126-156) and the header's section fields (format.rs:297-306). */
typedef struct {
  uint32_t arch, dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx_train;
  float rope_theta, norm_eps, rope_factor, rope_low, rope_high, rope_orig_ctx;
  uint32_t flags;
  float embed_scale, attn_scale, residual_scale, logit_scale;
  char name[48];
  uint64_t tok_off, tok_size, table_off;
  uint32_t tensor_count, data_crc, meta_crc, reserved;
  uint64_t data_off, data_size;
} nrq_nrm_meta;

/* TensorEntry (format.rs:159-169); offset is from the start of the data section. */
typedef struct {
  uint32_t kind, layer, dtype, rows, cols, reserved;
  uint64_t offset, size;
} nrq_nrm_tensor_info;

typedef struct nrq_nrm nrq_nrm;

/* Model::parse (format.rs:260-406): header, scale sanity, region bounds (no
 * wrapping sums), meta CRC, then every table entry (known dtype, inside the
 * data section, 64-byte aligned offset, size == dtype block math). Host only;
 * the blob must outlive the handle. Errors: NRQ_ERR_NRM_*, text in nrq_last_error. */
int nrq_nrm_open(const void *blob, size_t len, nrq_nrm **out);
int nrq_nrm_get_meta(const nrq_nrm *f, nrq_nrm_meta *out);
/* i-th table entry, in file order. */
int nrq_nrm_entry(const nrq_nrm *f, uint32_t i, nrq_nrm_tensor_info *out);
/* Model::tensor (format.rs:424-435): the first entry of this kind and layer,
 * else NRQ_ERR_NRM_MISSING_TENSOR naming it (format.rs:444-465). */
int nrq_nrm_tensor(const nrq_nrm *f, int kind, int layer, nrq_nrm_tensor_info *out);
/* Model::has_tensor (format.rs:437-439): 1 or 0. */
int nrq_nrm_has_tensor(const nrq_nrm *f, int kind);
/* Model::verify_data (format.rs:409-422) over a device copy of the data
 * section (data_size bytes): the CRC runs on the GPU; synchronous.
 * NRQ_ERR_NRM_DATA_CRC on a mismatch. */
int nrq_nrm_verify_data(const nrq_nrm *f, const void *dev_data, void *stream);
int nrq_nrm_close(nrq_nrm *f);

/* crc32::checksum / Crc32::update (crc32.rs:38-79) on host bytes, with zlib's
 * running-value convention: nrq_crc32(nrq_crc32(0, a), b) == nrq_crc32(0, a || b). */
uint32_t nrq_crc32(uint32_t crc, const void *data, size_t n);
/* The same CRC over n bytes in device memory (any alignment), enqueued on
 * `stream`; the result is written to the device word *out. Calls that overlap
 * on one device (different streams) share the library's partial-register
 * buffer and must not run concurrently. */
int nrq_dev_crc32(const void *data, size_t n, uint32_t crc, uint32_t *out, void *stream);

/* InferCtx::new (infer.rs:352-461) over a parsed file of any arch (Llama3,
 * Qwen3, Granite): checks that every tensor the recipe needs is present with
 * its shape, in the reference's order (MissingTensor errors as it reports
 * them, Qwen3's attn_q_norm / attn_k_norm included, and "unexpected
 * attn_q_norm for this arch" for the other families), uploads the data section
 * once, optionally verifies it on the device (NRQ_NRM_VERIFY_DATA), binds the
 * tensors (the head tied to the embedding under FLAG_TIED_EMBEDDINGS), sets the
 * rope table (RopeFreqs factors or the header's Llama-3 scaling) and the recipe
 * (NeoX pairs for Qwen3, the header's muP scales). The model owns the device
 * copy. Widths are checked in 64 bits; a model whose widths do not fit an int
 * is NRQ_ERR_UNSUPPORTED. */
int nrq_model_load_nrm(const nrq_nrm *f, int ctx, int flags, nrq_model **out);

#ifdef __cplusplus
}
#endif
#endif /* NRQ_H */
