/*
 * mcpm_hip.h -- C ABI of the MI355X (gfx950) decode engine for MiniCPM5-style
 * GGUF models.  Plain pointers and sizes; no C++ or torch types cross it.
 *
 * Three layers, mirroring the reference (astrowar/MiniCPM5.cpp):
 *   1. Context, device memory and weights (the reference keeps weights in one
 *      host buffer, src/model.cpp:44-69; here they are uploaded once to HBM).
 *   2. Per-op entry points, one per kernel of the backend seam
 *      (src/ops/ops_internal.h:13-72) and of the ops API (include/ops.h:112-160).
 *      Activations are device pointers; calls are ordered on the context's
 *      stream and return after enqueueing.  mcpm_sync() waits for them.
 *   3. The engine: load_model / init_kv_cache / forward of MiniCPM5Engine
 *      (include/model.h:37-45) plus the decode loop of ChatSession
 *      (src/chat_session.cpp:154-186).
 *
 * Every function returns MCPM_OK (0) or a negative MCPM_ERR_* code; nothing
 * throws across this boundary.  mcpm_last_error() returns the message of the
 * calling thread's last failure.  A context is used by one host thread at a
 * time (the reference engine is single-threaded, include/model.h:37-45).
 *
 * Block formats are ggml's (include/ops.h:33-65): Q8_0 34 B per 32 weights,
 * Q4_K 144 B per 256, Q6_K 210 B per 256, activation Q8_K 292 B per 256.
 */
#ifndef MCPM_HIP_H
#define MCPM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MCPM_OK 0
#define MCPM_ERR_HIP (-1)         /* a HIP runtime call failed */
#define MCPM_ERR_ARG (-2)         /* invalid argument (shape, null pointer) */
#define MCPM_ERR_UNSUPPORTED (-3) /* tensor type without a kernel */
#define MCPM_ERR_CONTEXT (-4)     /* pos >= max_seq_len, or KV cache missing */
#define MCPM_ERR_IO (-5)          /* file could not be read */
#define MCPM_ERR_FORMAT (-6)      /* malformed GGUF or missing tensor */
#define MCPM_ERR_NOMEM (-7)       /* device or host allocation failed */

/* ggml tensor type ids, as stored in GGUF. */
#define MCPM_TYPE_F32 0
#define MCPM_TYPE_Q8_0 8
#define MCPM_TYPE_Q4_K 12
#define MCPM_TYPE_Q6_K 14

#define MCPM_QK_K 256
#define MCPM_Q8K_BYTES 292

typedef struct mcpm_ctx mcpm_ctx;
typedef struct mcpm_tensor mcpm_tensor;
typedef struct mcpm_engine mcpm_engine;

/* ------------------------------------------------------------ context ---- */

/* Opens `device` and creates one HIP stream for all calls on the context. */
int mcpm_init(int device, mcpm_ctx **out);
void mcpm_destroy(mcpm_ctx *ctx);
const char *mcpm_last_error(void);
int mcpm_sync(mcpm_ctx *ctx);
/* Number of compute units and the device name (for reports). */
int mcpm_device_info(mcpm_ctx *ctx, int *n_cu, char *name, size_t name_len);

int mcpm_device_alloc(mcpm_ctx *ctx, size_t bytes, void **dptr);
int mcpm_device_free(mcpm_ctx *ctx, void *dptr);
/* Synchronous copies on the context stream. */
int mcpm_copy_to_device(mcpm_ctx *ctx, void *dst, const void *src, size_t bytes);
int mcpm_copy_to_host(mcpm_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device-to-device copy (reads and writes `bytes`: the kernel of known size
 * that scales the HBM byte counters in the measurements). */
int mcpm_copy_device(mcpm_ctx *ctx, void *dst, const void *src, size_t bytes);
int mcpm_fill_device(mcpm_ctx *ctx, void *dst, int byte_value, size_t bytes);
/* Read-only pass over `bytes` of device memory at `src` (a positive multiple
 * of 16, 16-byte aligned) by `grid` work groups of 256 lanes (1 .. 65536),
 * one word per work group written to `out` (device memory, `grid` words);
 * stream-ordered, timed like the per-op entries (mcpm_set_op_timing).  Its
 * duration is the floor of one launch that reads as many bytes as a GEMV.
 * No counterpart in the reference: a measurement kernel, as mcpm_copy_device
 * is for the byte counters. */
int mcpm_stream_read(mcpm_ctx *ctx, const void *src, size_t bytes, int grid, uint32_t *out);

/* ------------------------------------------------------------ weights ---- */

/* Uploads a weight matrix given in its native GGUF block layout (host memory),
 * cols = dims[0] (K), rows = dims[1] (include/ops.h:104-110).  The device copy
 * is re-laid out for coalesced loads (same bytes per block).  Replaces the
 * Tensor{type_str, dims, data_ptr} the reference's ops take. */
int mcpm_tensor_upload(mcpm_ctx *ctx, const void *host_blocks, size_t bytes, int ggml_type, int64_t cols,
                       int64_t rows, mcpm_tensor **out);
/* Writes the native block layout back to host memory (bytes == native size). */
int mcpm_tensor_download(mcpm_ctx *ctx, const mcpm_tensor *t, void *host_blocks, size_t bytes);
int mcpm_tensor_info(const mcpm_tensor *t, int *ggml_type, int64_t *cols, int64_t *rows);
void mcpm_tensor_free(mcpm_tensor *t);
/* Dequantizes rows [row0, row0+n_rows) to fp32 (device out, n_rows*cols). */
int mcpm_tensor_dequantize_rows(mcpm_ctx *ctx, const mcpm_tensor *t, int64_t row0, int64_t n_rows, float *out);

/* ------------------------------------------------------------ per-op ----- */

/* quantize_row_q8_K (src/ops/ops.cpp:300-308; AVX2 ties-to-even,
 * src/ops/ops_avx2.cpp:85-144).  n multiple of 256; y: n/256 Q8_K blocks. */
int mcpm_quantize_row_q8_K(mcpm_ctx *ctx, const float *x, int n, void *y);

/* gemv_q4_K_q8_K_avx2 / gemv_q6_K_q8_K_avx2 (src/ops/ops_internal.h:39-40). */
int mcpm_gemv_q4_K_q8_K(mcpm_ctx *ctx, const mcpm_tensor *w, const void *xq, float *out, int rows, int cols);
int mcpm_gemv_q6_K_q8_K(mcpm_ctx *ctx, const mcpm_tensor *w, const void *xq, float *out, int rows, int cols);

/* gemv_qkv_q4_K_q8_K_avx2 / gemv_qkv_q4_q4_q6_q8_K_avx2
 * (src/ops/ops_internal.h:43-50): q, k Q4_K; v Q4_K or Q6_K (wv's type). */
int mcpm_gemv_qkv_q8_K(mcpm_ctx *ctx, const mcpm_tensor *wq, const mcpm_tensor *wk, const mcpm_tensor *wv,
                       const void *xq, float *q, float *k, float *v, int q_rows, int kv_rows, int cols);

/* gemv_gate_up_q4_K_q8_K_avx2 (src/ops/ops_internal.h:51-54). */
int mcpm_gemv_gate_up_q4_K_q8_K(mcpm_ctx *ctx, const mcpm_tensor *wg, const mcpm_tensor *wu, const void *xq,
                                float *gate, float *up, int rows, int cols);

/* gemv_q4_K_avx2 / gemv_q6_K_avx2 (src/ops/ops_internal.h:35-36): fp32 input
 * quantized to Q8_K (ties-to-even), then the Q8_K GEMV. */
int mcpm_gemv_q4_K(mcpm_ctx *ctx, const mcpm_tensor *w, const float *x, float *out, int rows, int cols);
int mcpm_gemv_q6_K(mcpm_ctx *ctx, const mcpm_tensor *w, const float *x, float *out, int rows, int cols);

/* gemv_q8_0 / gemv_f32 (src/ops/ops.cpp:32-43, 58-79): fp32 activations. */
int mcpm_gemv_q8_0(mcpm_ctx *ctx, const mcpm_tensor *w, const float *x, float *out, int rows, int cols);
int mcpm_gemv_f32(mcpm_ctx *ctx, const mcpm_tensor *w, const float *x, float *out, int rows, int cols);

/* matmul (src/ops/ops.cpp:264-290): dispatch on w's type.  Unsupported types
 * fill out with 0.001f and return MCPM_ERR_UNSUPPORTED. */
int mcpm_matmul(mcpm_ctx *ctx, const mcpm_tensor *w, const float *x, float *out);
/* matmul_q8k (src/ops/ops.cpp:317-349): Q4_K or Q6_K; other types fill 0.0f
 * and return MCPM_ERR_UNSUPPORTED. */
int mcpm_matmul_q8k(mcpm_ctx *ctx, const mcpm_tensor *w, const void *xq, int num_cols, float *out);

/* rmsnorm (src/ops/ops.cpp:468-481). */
int mcpm_rmsnorm(mcpm_ctx *ctx, float *out, const float *x, const float *w, int dim, float eps);
/* rmsnorm_and_quantize_q8k (src/ops/ops.cpp:676-723), dim multiple of 256. */
int mcpm_rmsnorm_and_quantize_q8k(mcpm_ctx *ctx, void *out_q8k, const float *x, const float *w, int dim,
                                  float eps);
/* swiglu_and_quantize_q8k (src/ops/ops.cpp:725-765): dim/256 blocks. */
int mcpm_swiglu_and_quantize_q8k(mcpm_ctx *ctx, void *out_q8k, const float *gate, const float *up, int dim);
/* apply_rope for heads 0..n_heads-1 (src/ops/ops.cpp:502-516, loop
 * src/model.cpp:187-192), in place. */
int mcpm_apply_rope(mcpm_ctx *ctx, float *vec, int pos, int n_heads, int head_dim, float rope_base);
/* execute_attention (src/ops/ops.cpp:537-628) over caller-owned caches laid
 * out [max_seq_len][n_kv_heads][head_dim].  Returns MCPM_ERR_CONTEXT and
 * leaves attn_out untouched when pos >= max_seq_len. */
int mcpm_execute_attention(mcpm_ctx *ctx, float *attn_out, const float *q, const float *k_cur,
                           const float *v_cur, float *k_cache, float *v_cache, int pos, int max_seq_len,
                           int n_heads, int n_kv_heads, int head_dim);
/* mcpm_execute_attention with no allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the same kernels and results, with the chunk partials in a fixed per-GPU
 * device array (2.03 MiB, held until the process ends) instead of the
 * context's grow-on-demand buffer.  Limit: n_heads * ceil(max_seq_len / 64) *
 * (head_dim + 2) <= 532,480 floats (e.g. 64 heads of 128 up to 4096
 * positions, 32 heads of 64 up to 8192); larger shapes return MCPM_ERR_ARG.
 * Every call on one GPU shares the array, so calls that overlap on one GPU
 * (two contexts or threads at once) race. */
int mcpm_execute_attention_noalloc(mcpm_ctx *ctx, float *attn_out, const float *q, const float *k_cur,
                                   const float *v_cur, float *k_cache, float *v_cache, int pos, int max_seq_len,
                                   int n_heads, int n_kv_heads, int head_dim);
/* get_embedding (src/ops/ops.cpp:631-673) for Q4_K and Q6_K tables. */
int mcpm_get_embedding(mcpm_ctx *ctx, float *out, const mcpm_tensor *embd, int token);
/* First index of the maximum of x[0..n) into *out (device int). */
int mcpm_argmax(mcpm_ctx *ctx, const float *x, int n, int *out);
/* Sampler::sample (src/sampler.cpp:8-73) on device logits x[0..n) for the
 * uniform draw r in [0,1), token into *out (device int): temperature, softmax,
 * the top-p cut over the (p desc, id asc) order, the walk; its running sums
 * are taken in double over blocks of 256 positions (the reference's run
 * sequentially in float; see mcpm_sampler.hip), so its choice can differ
 * from mcpm_sample_logits only for draws within rounding of a boundary.
 * n up to 524,288 (larger: MCPM_ERR_ARG). */
int mcpm_sample_device(mcpm_ctx *ctx, const float *x, int n, float temperature, float top_p, float r, int *out);

/* Per-op kernel timing, a measurement aid with no counterpart in the
 * reference (its ops are timed with wall clocks around OpenMP regions).
 * While enabled, each launch of the single-kernel GEMV entries
 * (mcpm_gemv_q4_K_q8_K, mcpm_gemv_q6_K_q8_K, mcpm_gemv_qkv_q8_K,
 * mcpm_gemv_gate_up_q4_K_q8_K, mcpm_gemv_q4_K, mcpm_gemv_q6_K) records events
 * at its kernel's start and end.  mcpm_op_time waits for the stream, returns
 * the summed kernel time and the number of timed launches since the last
 * call (or since timing was enabled), and starts a new count. */
int mcpm_set_op_timing(mcpm_ctx *ctx, int enable);
int mcpm_op_time(mcpm_ctx *ctx, double *total_ms, int64_t *launches);

/* ------------------------------------------------------------ engine ----- */

typedef struct {
    int n_layers, dim, n_heads, n_kv_heads, head_dim;
    int ffn;     /* feed_forward_length */
    int ffn_pad; /* ffn rounded up to whole 256-blocks (the down-projection's K) */
    int vocab;
    float rope_base, eps;
    int tied_embeddings; /* 1 when token_embd also serves as the LM head */
} mcpm_model_config;

/* MiniCPM5Engine::load_model (src/model.cpp:33-133): parses the GGUF header
 * at run time (the reference bakes offsets at compile time) and uploads every
 * tensor once.  From a file or from a GGUF image in host memory. */
int mcpm_engine_load_gguf(mcpm_ctx *ctx, const char *path, mcpm_engine **out);
int mcpm_engine_load_gguf_memory(mcpm_ctx *ctx, const void *data, size_t bytes, mcpm_engine **out);
void mcpm_engine_free(mcpm_engine *e);
int mcpm_engine_config(const mcpm_engine *e, mcpm_model_config *out);
/* Weight bytes read per decode token (all layers, LM head, one embedding row). */
int64_t mcpm_engine_weight_bytes_per_token(const mcpm_engine *e);

/* MiniCPM5Engine::init_kv_cache (src/model.cpp:17-24): fp32 K and V,
 * [n_layers][max_seq_len][n_kv_heads*head_dim], zeroed. */
int mcpm_engine_init_kv_cache(mcpm_engine *e, int max_seq_len);

/* MiniCPM5Engine::forward (src/model.cpp:142-242): one token at position pos.
 * logits (vocab floats, host) and argmax (host int) may each be NULL.
 * MCPM_ERR_CONTEXT when pos >= the KV capacity or max_seq_len. */
int mcpm_engine_forward(mcpm_engine *e, int token, int pos, int max_seq_len, float *logits, int *argmax);

/* The prefill + greedy decode loop of ChatSession::generate_response
 * (src/chat_session.cpp:154-186) with argmax in place of the sampler: feeds
 * prompt[0..n_prompt) at positions 0.., then generates n_gen tokens
 * (out_tokens[0] is the argmax after the last prompt token).  Runs on the
 * device without host round trips between tokens. */
int mcpm_engine_generate_greedy(mcpm_engine *e, const int *prompt, int n_prompt, int n_gen, int *out_tokens);

/* Continues the greedy loop for n_steps more tokens from the device state the
 * previous generate/decode call left (the last argmax at the next position),
 * appending to the generated-token list; returns once the work is queued
 * (mcpm_sync waits for it).  MCPM_ERR_CONTEXT when the KV cache is full. */
int mcpm_engine_decode_steps(mcpm_engine *e, int n_steps);
/* Copies the first n generated tokens (since the last generate call). */
int mcpm_engine_tokens(mcpm_engine *e, int *out, int n);

/* Same loop with the reference's temperature / top-p sampler
 * (src/sampler.cpp:8-73) on the device (mcpm_sample_device's arithmetic),
 * drawing std::uniform_real_distribution<float> from std::mt19937(seed), one
 * draw per generated token. */
int mcpm_engine_generate_sampled(mcpm_engine *e, const int *prompt, int n_prompt, int n_gen, float temperature,
                                 float top_p, uint32_t seed, int *out_tokens);
/* Continues the last generate call by n_steps sampled tokens (draws from a
 * new std::mt19937(seed)); the token list must have room (mcpm_engine_tokens
 * reads it).  No counterpart in the reference: its chat loop
 * (src/chat_session.cpp:154-186) samples token by token. */
int mcpm_engine_decode_sampled(mcpm_engine *e, int n_steps, float temperature, float top_p, uint32_t seed);

/* The generate loops continuing a cached context: tokens[0..n) go at
 * positions pos0.. and the KV rows below pos0 are kept as they are (a previous
 * turn's), then n_gen tokens are generated as above.  For a chat driver that
 * keeps the cache across turns and processes only each turn's new tokens; the
 * reference re-runs forward() over the whole conversation from position 0
 * every turn (src/chat_session.cpp:126-160). */
int mcpm_engine_generate_greedy_at(mcpm_engine *e, const int *tokens, int n, int pos0, int n_gen, int *out_tokens);
int mcpm_engine_generate_sampled_at(mcpm_engine *e, const int *tokens, int n, int pos0, int n_gen,
                                    float temperature, float top_p, uint32_t seed, int *out_tokens);

/* Sampler::sample (src/sampler.cpp:8-73) on host logits for a given uniform
 * draw r in [0,1): returns the token id, or a negative error code. */
int mcpm_sample_logits(const float *logits, int n, float temperature, float top_p, float r);

/* 1: replay each token as one captured hipGraph (default); 0: eager launches. */
int mcpm_engine_set_graph(mcpm_engine *e, int enable);

/* Where every layer of a token runs in one persistent launch, the per-token
 * loop of MiniCPM5Engine::forward (src/model.cpp:171-226) as one kernel,
 * instead of five launches per layer.  Results are the same.
 *   1: wherever the model's shape and the KV capacity fit (8 kv heads of 64,
 *      4 query heads per kv head, a CU count that is a multiple of 8, at
 *      most 2 attention chunks of 64 positions per CU);
 *   2 (the default): only where the launch also has an instance compiled for
 *      the shape (every plan field a constant): the 2.4B-shaped decoder
 *      (hidden 2304, 32/8 heads of 64, FFN 5760, Q4_K q/k/o/gate/up, Q6_K
 *      v/down, any layer count) on 256 CUs with a KV capacity of at most
 *      4096 positions;
 *   0: never.
 * MCPM_PERSIST=0/1/2 in the environment at load sets the mode.  While the
 * launch is taken the engine holds its weight slab, the layer weights once
 * more in the launch's layout; mode 0 frees it, and so does mode 2 for a
 * shape it does not take.  MCPM_ERR_ARG for another mode. */
int mcpm_engine_set_persistent(mcpm_engine *e, int mode);
/* 1 when the next token runs its layers in one launch. */
int mcpm_engine_uses_persistent(const mcpm_engine *e);
/* 1 when that launch is the instance compiled for the model's shape.  No
 * counterpart in the reference. */
int mcpm_engine_persistent_fixed_shape(const mcpm_engine *e);
/* 1 when that launch also hands the records read on one XCD only (a kv
 * head's q/k/v rows, its attention chunks' partials) through that XCD's L2:
 * set up when every work group b runs on the XCD of work group b % 8
 * (checked at set-up, and by each launch, which otherwise fails with
 * MCPM_ERR_HIP); MCPM_PD_XCD_LOCAL=0 keeps every hand-off at agent scope.
 * No counterpart in the reference. */
int mcpm_engine_persistent_xcd_local(const mcpm_engine *e);
/* The spin limit of the waits inside the engine's launches: the fused
 * kernels' grid barrier (MCPM_FUSED_FFN / MCPM_FUSED_ATTN), the persistent
 * launch's hand-offs and the O projection's wait for its XCD's attention
 * records (contexts of at most 64 positions).  A wait that passes it gives up, every work group then
 * leaves, and the call returns MCPM_ERR_HIP with the wait state reset, so the
 * next call runs normally.  0 restores the defaults (1<<20 barrier polls,
 * 1<<18 hand-off polls).  No counterpart in the reference: it lets tests
 * drive the give-up path with a tiny limit. */
int mcpm_engine_set_spin_limit(mcpm_engine *e, unsigned limit);

/* Processes tokens[0..n) at positions pos0.. through every layer together
 * (MFMA GEMMs), leaving the KV cache exactly as n calls of
 * mcpm_engine_forward would; produces no logits.  Replaces the reference's
 * per-token prompt loop (src/chat_session.cpp:154-160). */
int mcpm_engine_prefill(mcpm_engine *e, const int *tokens, int n, int pos0);
/* 1 (default): generate calls send all prompt tokens but the last through
 * mcpm_engine_prefill; 0: one forward per prompt token.  Results are the same. */
int mcpm_engine_set_prefill(mcpm_engine *e, int enable);
int mcpm_engine_uses_prefill(const mcpm_engine *e);
/* Copies K and V cache rows [pos0, pos0+n) of one layer (n * n_kv_heads *
 * head_dim floats each) to host memory; k or v may be NULL. */
int mcpm_engine_read_kv(mcpm_engine *e, int layer, int pos0, int n, float *k, float *v);

/* Kernel-level timing for measurement.  Kernel classes: */
#define MCPM_KC_QKV 0
#define MCPM_KC_ATTN 1
#define MCPM_KC_OPROJ 2
#define MCPM_KC_GATE_UP 3
#define MCPM_KC_DOWN 4
#define MCPM_KC_LM_HEAD 5
#define MCPM_KC_LAYERS 6 /* the persistent launch of every layer */
#define MCPM_KC_COUNT 7
/* When enabled, HIP events bracket every launch of `kernel_class` on the
 * engine stream (inside the captured graph too); mcpm_engine_kernel_time
 * returns the summed milliseconds and launch count since the last reset. */
int mcpm_engine_set_kernel_timing(mcpm_engine *e, int kernel_class);
int mcpm_engine_kernel_time(mcpm_engine *e, double *total_ms, int64_t *launches);
/* Algorithmic bytes one launch of `kernel_class` moves (weights + activations). */
int64_t mcpm_engine_kernel_bytes(const mcpm_engine *e, int kernel_class);

/* ------------------------------------------------ synthetic GGUF models -- */

/* Writes a random-init MiniCPM5-shaped model as a GGUF v3 image: weights
 * N(0, 0.02) and norm gains 1 + N(0, 0.1) from a counter-based generator
 * keyed by (seed, tensor, index), quantized with this library's Q4_K / Q6_K /
 * Q8_0 encoders.  mix 0: Q6_K for every attn_v and ffn_down (literal
 * Q4_K_M reading); mix 1: llama.cpp's use_more_bits layers only; with
 * cfg->tied_embeddings one Q6_K token_embd serves as the LM head, else a
 * separate Q6_K output.weight follows it.  mix 2: the layout of the
 * reference's own file (include/minicpm_metadata.h:30-32): an untied Q6_K
 * output.weight, a Q4_K token_embd.weight, use_more_bits for attn_v and
 * ffn_down, tensors in that file's order, and a tokenizer.ggml.tokens
 * vocabulary the reference's tokenizer reads (src/tokenizer.cpp:10-60);
 * tied_embeddings is ignored.  A tensor's values depend on its name only, so
 * mixes and layouts agree wherever they store the same tensor with the same
 * type.  When path is NULL the image is returned in *image (free with
 * mcpm_free_host) and its size in *image_bytes. */
int mcpm_synth_gguf(const mcpm_model_config *cfg, uint64_t seed, int mix, const char *path, void **image,
                    size_t *image_bytes);
void mcpm_free_host(void *p);

/* Deterministic host-side generators, exposed for tests and benchmarks. */
void mcpm_synth_normal(uint64_t seed, uint64_t tensor_id, float mean, float stddev, float *out, size_t n);
/* Encode fp32 rows (cols multiple of the block size) into ggml blocks. */
int mcpm_quantize_rows(int ggml_type, const float *src, int64_t rows, int64_t cols, void *dst);
size_t mcpm_type_row_bytes(int ggml_type, int64_t cols);

#ifdef __cplusplus
}
#endif
#endif
