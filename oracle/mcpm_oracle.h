/*
 * mcpm_oracle.h -- CPU oracle for the MiniCPM5 batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library checks the product: it is loaded by the
 * tests, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by
 * the product library (minicpm5.cpp_amd/), which must fail loudly without its
 * HIP build instead of falling back here.
 *
 * It restates, in plain C11, the algorithms of the reference's CPU kernels
 * (astrowar/MiniCPM5.cpp):
 *   include/ops.h                    block formats, fp16, Q4_K scale unpack
 *   src/ops/ops.cpp                  dispatch, fused RMSNorm/SwiGLU quantizers,
 *                                    RoPE, attention, embedding, f32/Q8_0 GEMV
 *   src/ops/ops_avx2.cpp             Q8_K quantizer and Q4_K/Q6_K x Q8_K dots
 *   src/ops/ops_scalar_optimized.cpp the documented integer decomposition
 *   src/model.cpp                    forward() step order, residuals, KV layout
 *
 * Float evaluation order.  The reference is built with -O3 -march=native
 * -ffast-math, so its summation order in compiler-vectorised loops is not a
 * property of the source.  Where the reference's order is fixed by its source
 * (the AVX2 intrinsic kernels: eight integer lanes, one FMA per lane per block,
 * a fixed horizontal-sum tree) the oracle reproduces it exactly.  Where it is
 * not (sums of squares, attention dot products, softmax sums), the oracle fixes
 * one documented order, written out in each function below, which the HIP
 * kernels reproduce bit for bit.  The oracle is compiled with
 * -ffp-contract=off; every fused multiply-add below is an explicit fmaf().
 *
 * Pinning status of each function is listed in oracle/README.md.
 */
#ifndef MCPM_ORACLE_H
#define MCPM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK_K 256
#define OR_QK8_0 32

/* Block layouts (include/ops.h:33-65). */
typedef struct { uint16_t d; int8_t qs[32]; } or_block_q8_0;                                /* 34 B  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } or_block_q4_K;    /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } or_block_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } or_block_q8_K;               /* 292 B */

/* ggml type ids used by GGUF. */
enum { OR_F32 = 0, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14 };

/* Positions per split of the decode attention (online-softmax chunk). */
#define OR_ATTN_CHUNK 64

float or_fp16_to_fp32(uint16_t h);
void or_q4k_scales_mins(const uint8_t *q, uint8_t *sc, uint8_t *mn);
float or_expf(float x);

/* Q8_K activation quantizer; ties_away=0: nearest-even (quantize_row_q8_K),
 * ties_away=1: std::lround (fused RMSNorm / SwiGLU quantizers). */
void or_quantize_row_q8_K(const float *x, int n, or_block_q8_K *y, int ties_away);

/* Dequantize n values (a whole number of blocks) of a row. */
void or_dequant_row(int type, const void *blocks, int n, float *out);

/* Integer lanes of one block, as the AVX2 kernels form them (for tests). */
void or_q4k_block_lanes(const or_block_q4_K *w, const or_block_q8_K *a, int32_t isum[8], int32_t *minsum);
void or_q6k_block_lanes(const or_block_q6_K *w, const or_block_q8_K *a, int32_t isum[8]);

float or_dot_q4_K_q8_K(const or_block_q4_K *w, const or_block_q8_K *a, int nb);
float or_dot_q6_K_q8_K(const or_block_q6_K *w, const or_block_q8_K *a, int nb);

void or_gemv_q4_K_q8_K(const void *w, const or_block_q8_K *xq, float *out, int rows, int cols);
void or_gemv_q6_K_q8_K(const void *w, const or_block_q8_K *xq, float *out, int rows, int cols);
void or_gemv_qkv_q8_K(const void *wq, const void *wk, const void *wv, int v_type, const or_block_q8_K *xq,
                      float *q, float *k, float *v, int q_rows, int kv_rows, int cols);
void or_gemv_gate_up_q4_K_q8_K(const void *wg, const void *wu, const or_block_q8_K *xq, float *gate,
                               float *up, int rows, int cols);
void or_gemv_f32(const float *w, const float *x, float *out, int rows, int cols);
void or_gemv_q8_0(const void *w, const float *x, float *out, int rows, int cols);
void or_gemv_q4_K_f32act(const void *w, const float *x, float *out, int rows, int cols);
void or_gemv_q6_K_f32act(const void *w, const float *x, float *out, int rows, int cols);

/* matmul(out, x, tensor) of an AVX2 build (ops.cpp:264-290). Returns 0, or -1 for an
 * unsupported type (then out is filled with 0.001f as the reference does). */
int or_matmul(int type, const void *w, const float *x, float *out, int rows, int cols);
/* matmul_q8k (ops.cpp:317-349); -1 and zero fill for unsupported types. */
int or_matmul_q8k(int type, const void *w, const or_block_q8_K *xq, float *out, int rows, int cols);

float or_rms_scale(const float *x, int dim, float eps);
void or_rmsnorm(float *out, const float *x, const float *w, int dim, float eps);
void or_rmsnorm_and_quantize_q8k(or_block_q8_K *out, const float *x, const float *w, int dim, float eps);
void or_swiglu(float *h, const float *gate, const float *up, int dim);
void or_swiglu_and_quantize_q8k(or_block_q8_K *out, const float *gate, const float *up, int dim);
void or_apply_rope(float *vec, int pos, int n_heads, int head_dim, float base);
/* execute_attention: appends k_cur/v_cur at pos, then attends over 0..pos.
 * Returns -1 (and leaves out untouched) when pos >= max_seq_len. */
int or_attention(float *out, const float *q, const float *k_cur, const float *v_cur, float *k_cache,
                 float *v_cache, int pos, int max_seq_len, int n_heads, int n_kv_heads, int head_dim);
/* Returns -1 (zero fill) for unsupported embedding types. */
int or_get_embedding(float *out, int type, const void *embd, int dim, int token);
int or_argmax(const float *x, int n);
/* The OpenMP team of the oracle's parallel loops (a fixed team of n). */
void or_set_threads(int n);

/* ---- whole model ---- */
typedef struct {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, ffn_pad, vocab;
    float rope_base, eps;
} or_config;

typedef struct {
    const float *attn_norm;
    const void *wq, *wk, *wv;
    int wv_type;
    const void *wo;
    int wo_type;
    const float *ffn_norm;
    const void *wg, *wu, *wd;
    int wd_type;
} or_layer;

typedef struct or_model or_model;

or_model *or_model_create(const or_config *cfg, const void *embd, int embd_type, const float *out_norm,
                          const void *out_w, int out_type, const or_layer *layers);
int or_model_init_kv(or_model *m, int max_seq_len);
/* One token through the model; logits (vocab floats) may be NULL. Returns argmax. */
int or_model_forward(or_model *m, int token, int pos, float *logits);
/* The layers only (K/V rows into the cache), no LM head; 0 or -1. */
int or_model_forward_kv(or_model *m, int token, int pos);
/* Hidden state after the last layer (dim floats), for tests. */
const float *or_model_hidden(const or_model *m);
/* K and V cache rows [pos0, pos0+n) of one layer into k, v (either may be NULL); 0 or -1. */
int or_model_read_kv(const or_model *m, int layer, int pos0, int n, float *k, float *v);
void or_model_free(or_model *m);

/* mt19937 + uniform_real_distribution<float>(0,1) as libstdc++ computes it,
 * and the reference's temperature / top-p sampler (src/sampler.cpp:8-73)
 * given a draw r. */
typedef struct { uint32_t mt[624]; int idx; } or_mt19937;
void or_mt_seed(or_mt19937 *g, uint32_t seed);
uint32_t or_mt_next(or_mt19937 *g);
float or_mt_uniform01(or_mt19937 *g);
int or_sample(const float *logits, int n, float temperature, float top_p, float r);
/* The same steps with running sums in blocked double (the device sampler). */
int or_sample_blocked(const float *logits, int n, float temperature, float top_p, float r);

#ifdef __cplusplus
}
#endif
#endif
