// ref_harness.cpp -- extern "C" access to the reference's own CPU kernels.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's src/ops/{ops,ops_avx2,ops_scalar_optimized}.cpp, read where
// they lie in the reference's tree (nothing is copied), into
// oracle/_ref/librefops.so.  Tests use it to pin the oracle against the
// reference's compiled numerics; bench.py may time it as the CPU baseline.
//
// The functions below only marshal raw pointers into the reference's
// std::vector / Tensor API (include/ops.h:104-160).  ref_model_* restates the
// step order of MiniCPM5Engine::forward (src/model.cpp:142-242) with explicit
// shapes, because the reference's own forward() is fixed at compile time to
// its metadata header, and calls the reference's ops for every step.
#include <omp.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "ops.h"
#include "ops_internal.h"

// Defined in ops.cpp / ops_scalar_optimized.cpp without a header declaration.
void gemv_f32(const char* matrix_weights, const float* x, float* out, int num_rows, int num_cols);
void gemv_q8_0(const char* matrix_weights, const float* x, float* out, int num_rows, int num_cols);
void quantize_row_q8_K_scalar(const float* x, block_q8_K* y, int n);
float dot_row_q4_K_q8_K_scalar(const block_q4_K* w, const block_q8_K* xq, int num_blocks);
float dot_row_q6_K_q8_K_scalar(const block_q6_K* w, const block_q8_K* xq, int num_blocks);

namespace {

const char* type_name(int t) {
  switch (t) {
    case 0: return "F32";
    case 8: return "Q8_0";
    case 12: return "Q4_K";
    case 14: return "Q6_K";
    default: return "UNSUPPORTED";
  }
}

Tensor make_tensor(int type, const void* data, uint64_t cols, uint64_t rows) {
  Tensor t;
  t.type_str = type_name(type);
  t.data_ptr = static_cast<const char*>(data);
  t.dims = {cols, rows};
  return t;
}

}  // namespace

extern "C" {

void ref_set_threads(int n) { omp_set_dynamic(0); omp_set_num_threads(n); }

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }

void ref_decode_q4k_scales_mins(const uint8_t* q, uint8_t* sc, uint8_t* mn) { decode_q4k_scales_mins(q, sc, mn); }

void ref_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) { get_scale_min_k4(j, q, d, m); }

void ref_quantize_row_q8_K(const float* x, int n, block_q8_K* y) { quantize_row_q8_K(x, n, y); }

void ref_quantize_row_q8_K_scalar(const float* x, int n, block_q8_K* y) { quantize_row_q8_K_scalar(x, y, n); }

void ref_rmsnorm_and_quantize_q8k(block_q8_K* out, const float* x, const float* w, int dim, float eps) {
  std::vector<float> xv(x, x + dim);
  Tensor t = make_tensor(0, w, dim, 1);
  rmsnorm_and_quantize_q8k(out, xv, t, eps);
}

void ref_swiglu_and_quantize_q8k(block_q8_K* out, const float* g, const float* u, int dim) {
  std::vector<float> gv(g, g + dim), uv(u, u + dim);
  swiglu_and_quantize_q8k(out, gv, uv);
}

void ref_rmsnorm(float* out, const float* x, const float* w, int dim, float eps) {
  std::vector<float> xv(x, x + dim), ov;
  Tensor t = make_tensor(0, w, dim, 1);
  rmsnorm(ov, xv, t, eps);
  std::memcpy(out, ov.data(), sizeof(float) * dim);
}

float ref_silu(float x) { return silu(x); }

void ref_matmul(int type, const void* w, const float* x, float* out, int rows, int cols) {
  std::vector<float> xv(x, x + cols), ov;
  Tensor t = make_tensor(type, w, cols, rows);
  matmul(ov, xv, t);
  std::memcpy(out, ov.data(), sizeof(float) * rows);
}

void ref_matmul_q8k(int type, const void* w, const block_q8_K* xq, float* out, int rows, int cols) {
  std::vector<float> ov;
  Tensor t = make_tensor(type, w, cols, rows);
  matmul_q8k(ov, xq, cols, t);
  std::memcpy(out, ov.data(), sizeof(float) * rows);
}

void ref_matmul_qkv_q8k(const void* wq, const void* wk, const void* wv, int v_type, const block_q8_K* xq,
                        float* q, float* k, float* v, int q_rows, int kv_rows, int cols) {
  std::vector<float> qv, kv, vv;
  Tensor tq = make_tensor(12, wq, cols, q_rows), tk = make_tensor(12, wk, cols, kv_rows),
         tv = make_tensor(v_type, wv, cols, kv_rows);
  matmul_qkv_q8k(qv, kv, vv, xq, cols, tq, tk, tv);
  std::memcpy(q, qv.data(), sizeof(float) * q_rows);
  std::memcpy(k, kv.data(), sizeof(float) * kv_rows);
  std::memcpy(v, vv.data(), sizeof(float) * kv_rows);
}

void ref_matmul_gate_up_q8k(const void* wg, const void* wu, const block_q8_K* xq, float* g, float* u, int rows,
                            int cols) {
  std::vector<float> gv, uv;
  Tensor tg = make_tensor(12, wg, cols, rows), tu = make_tensor(12, wu, cols, rows);
  matmul_gate_up_q8k(gv, uv, xq, cols, tg, tu);
  std::memcpy(g, gv.data(), sizeof(float) * rows);
  std::memcpy(u, uv.data(), sizeof(float) * rows);
}

void ref_gemv_q4_K_scalar(const void* w, const float* x, float* out, int rows, int cols) {
  gemv_q4_K_scalar(static_cast<const char*>(w), x, out, rows, cols);
}
void ref_gemv_q6_K_scalar(const void* w, const float* x, float* out, int rows, int cols) {
  gemv_q6_K_scalar(static_cast<const char*>(w), x, out, rows, cols);
}
void ref_gemv_q4_K_q8_K_scalar(const void* w, const block_q8_K* xq, float* out, int rows, int cols) {
  gemv_q4_K_q8_K_scalar(static_cast<const char*>(w), xq, out, rows, cols);
}
void ref_gemv_q6_K_q8_K_scalar(const void* w, const block_q8_K* xq, float* out, int rows, int cols) {
  gemv_q6_K_q8_K_scalar(static_cast<const char*>(w), xq, out, rows, cols);
}
void ref_gemv_f32(const void* w, const float* x, float* out, int rows, int cols) {
  gemv_f32(static_cast<const char*>(w), x, out, rows, cols);
}
void ref_gemv_q8_0(const void* w, const float* x, float* out, int rows, int cols) {
  gemv_q8_0(static_cast<const char*>(w), x, out, rows, cols);
}

void ref_apply_rope(float* vec, int n, int pos, int n_heads, int head_dim, float base) {
  std::vector<float> v(vec, vec + n);
  for (int h = 0; h < n_heads; ++h) apply_rope(v, pos, h, head_dim, base);
  std::memcpy(vec, v.data(), sizeof(float) * n);
}

// execute_attention over a caller-owned cache of max_seq_len positions.
void ref_execute_attention(float* out, const float* q, const float* k_cur, const float* v_cur, float* k_cache,
                           float* v_cache, int pos, int max_seq_len, int n_heads, int n_kv_heads, int head_dim) {
  const int qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
  std::vector<float> ov(out, out + qd), qv(q, q + qd), kv(k_cur, k_cur + kvd), vv(v_cur, v_cur + kvd);
  KVCacheLayer cache;
  cache.k.assign(k_cache, k_cache + (size_t)max_seq_len * kvd);
  cache.v.assign(v_cache, v_cache + (size_t)max_seq_len * kvd);
  execute_attention(ov, qv, kv, vv, cache, pos, max_seq_len, n_heads, n_kv_heads, head_dim);
  std::memcpy(out, ov.data(), sizeof(float) * qd);
  std::memcpy(k_cache, cache.k.data(), sizeof(float) * (size_t)max_seq_len * kvd);
  std::memcpy(v_cache, cache.v.data(), sizeof(float) * (size_t)max_seq_len * kvd);
}

void ref_get_embedding(float* out, int type, const void* embd, int dim, int vocab, int token) {
  std::vector<float> ov;
  Tensor t = make_tensor(type, embd, dim, vocab);
  get_embedding(ov, t, token);
  std::memcpy(out, ov.data(), sizeof(float) * dim);
}

// ---------------------------------------------------------------- model ----

struct ref_layer {
  const float* attn_norm;
  const void *wq, *wk, *wv;
  int wv_type;
  const void* wo;
  int wo_type;
  const float* ffn_norm;
  const void *wg, *wu, *wd;
  int wd_type;
};

struct ref_config {
  int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, ffn_pad, vocab;
  float rope_base, eps;
};

struct ref_model {
  ref_config c;
  Tensor embd, out_norm, out;
  std::vector<ref_layer> L;
  std::vector<KVCacheLayer> kv;
  int max_seq = 0;
  std::vector<float> x, x_norm, q, k, v, attn_tmp, attn_out, gate, up, ffn_out, residual, logits;
  std::vector<block_q8_K> xq, hq;
};

ref_model* ref_model_create(const ref_config* c, const void* embd, int embd_type, const float* out_norm,
                            const void* out_w, int out_type, const ref_layer* layers) {
  auto* m = new ref_model();
  m->c = *c;
  // Tied Q6_K embedding is not supported by get_embedding (ops.cpp:635,669):
  // the harness takes the embedding row from the oracle in that case.
  m->embd = make_tensor(embd_type, embd, c->dim, c->vocab);
  m->out_norm = make_tensor(0, out_norm, c->dim, 1);
  m->out = make_tensor(out_type, out_w, c->dim, c->vocab);
  m->L.assign(layers, layers + c->n_layers);
  return m;
}

void ref_model_init_kv(ref_model* m, int max_seq_len) {
  const int kvd = m->c.n_kv_heads * m->c.head_dim;
  m->kv.resize(m->c.n_layers);
  for (auto& l : m->kv) {
    l.k.assign((size_t)max_seq_len * kvd, 0.0f);
    l.v.assign((size_t)max_seq_len * kvd, 0.0f);
  }
  m->max_seq = max_seq_len;
}

// forward() of src/model.cpp:142-242.  x_in: the embedding row (dim floats).
// Writes logits (vocab floats) and returns the first index of the maximum.
int ref_model_forward(ref_model* m, const float* x_in, int pos, float* logits) {
  const ref_config& c = m->c;
  const int qd = c.n_heads * c.head_dim;
  m->x.assign(x_in, x_in + c.dim);
  m->xq.resize(c.dim / QK_K);
  m->hq.resize(c.ffn_pad / QK_K);
  for (int l = 0; l < c.n_layers; ++l) {
    const ref_layer& L = m->L[l];
    Tensor an = make_tensor(0, L.attn_norm, c.dim, 1), fn = make_tensor(0, L.ffn_norm, c.dim, 1);
    Tensor tq = make_tensor(12, L.wq, c.dim, qd), tk = make_tensor(12, L.wk, c.dim, c.n_kv_heads * c.head_dim),
           tv = make_tensor(L.wv_type, L.wv, c.dim, c.n_kv_heads * c.head_dim),
           to = make_tensor(L.wo_type, L.wo, qd, c.dim), tg = make_tensor(12, L.wg, c.dim, c.ffn),
           tu = make_tensor(12, L.wu, c.dim, c.ffn), td = make_tensor(L.wd_type, L.wd, c.ffn_pad, c.dim);
    m->residual = m->x;
    rmsnorm_and_quantize_q8k(m->xq.data(), m->x, an, c.eps);
    matmul_qkv_q8k(m->q, m->k, m->v, m->xq.data(), c.dim, tq, tk, tv);
    for (int h = 0; h < c.n_heads; ++h) apply_rope(m->q, pos, h, c.head_dim, c.rope_base);
    for (int h = 0; h < c.n_kv_heads; ++h) apply_rope(m->k, pos, h, c.head_dim, c.rope_base);
    execute_attention(m->attn_tmp, m->q, m->k, m->v, m->kv[l], pos, m->max_seq, c.n_heads, c.n_kv_heads,
                      c.head_dim);
    matmul(m->attn_out, m->attn_tmp, to);
    for (int i = 0; i < c.dim; ++i) m->x[i] = m->residual[i] + m->attn_out[i];
    m->residual = m->x;
    rmsnorm_and_quantize_q8k(m->xq.data(), m->x, fn, c.eps);
    matmul_gate_up_q8k(m->gate, m->up, m->xq.data(), c.dim, tg, tu);
    // FFN width padded to whole Q8_K blocks with zeros (silu(0)*0 == 0).
    m->gate.resize(c.ffn_pad, 0.0f);
    m->up.resize(c.ffn_pad, 0.0f);
    swiglu_and_quantize_q8k(m->hq.data(), m->gate, m->up);
    matmul_q8k(m->ffn_out, m->hq.data(), c.ffn_pad, td);
    for (int i = 0; i < c.dim; ++i) m->x[i] = m->residual[i] + m->ffn_out[i];
  }
  rmsnorm(m->x_norm, m->x, m->out_norm, c.eps);
  matmul(m->logits, m->x_norm, m->out);
  int best = 0;
  for (int i = 1; i < c.vocab; ++i)
    if (m->logits[i] > m->logits[best]) best = i;
  if (logits) std::memcpy(logits, m->logits.data(), sizeof(float) * c.vocab);
  return best;
}

const float* ref_model_hidden(const ref_model* m) { return m->x.data(); }

void ref_model_free(ref_model* m) { delete m; }

}  // extern "C"
