// mcpm_engine.cpp -- the decode engine: GGUF load into HBM, KV cache, the
// per-token kernel sequence (captured as one hipGraph) and the decode loops.
//
// One token (src/model.cpp:142-242): where the shape fits, every layer in
// one persistent launch (mcpm_persist.hip); otherwise five fused kernels per
// layer:
//   qkv    RMSNorm+Q8_K (lround) prologue, Q/K/V GEMV, RoPE + KV append epilogue
//   attn   split softmax over 64-position chunks, last wave combines
//   oproj  Q8_K (ties-even) prologue, O GEMV, residual add epilogue
//   gateup RMSNorm+Q8_K (lround) prologue, gate/up GEMV, SwiGLU epilogue
//   down   Q8_K (lround) prologue, down GEMV, residual add epilogue
// then embedding at the start and RMSNorm+LM head+argmax at the end.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <random>
#include <vector>

#include "gguf.h"
#include "mcpm_host.h"
#include "mcpm_persist.h"

using namespace mcpm;

namespace {

struct Layer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  DevTensor wq, wk, wv, wo, wg, wu, wd;
};

struct TimedPair {
  hipEvent_t a, b;
};

// Scratch of the batched prompt path, for `cap` tokens at a time.
struct PrefillBufs {
  int cap = 0, max_chunks = 0;
  int* tokens = nullptr;
  float *x = nullptr, *q = nullptr, *g = nullptr, *u = nullptr, *part = nullptr;
  _Float16 *xh = nullptr, *xbs = nullptr;
  float* xd = nullptr;
};
// Tokens per batched pass (MCPM_PREFILL_CHUNK overrides, a tuning aid).
int prefill_chunk() {
  static const int v = [] {
    const char* e = std::getenv("MCPM_PREFILL_CHUNK");
    const int n = e ? std::atoi(e) : 0;
    return n >= 16 && n <= 4096 ? n : 1024;
  }();
  return v;
}

}  // namespace

struct mcpm_engine {
  mcpm_ctx* ctx = nullptr;
  mcpm_model_config cfg{};
  DevTensor embd, out_w;
  float* out_norm = nullptr;
  std::vector<Layer> L;
  // activations
  float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
  float2* argmax_part = nullptr;
  int lm_grid = 0;
  StepState* st = nullptr;
  StepState* h_st = nullptr;  // pinned staging, one per queued prefill token
  int h_st_cap = 0;
  int* out_tokens = nullptr;
  int out_cap = 0;
  int gen_count = 0;  // tokens generated since the last generate call
  int next_pos = 0;   // position the next decode step runs at
  // KV cache and attention scratch
  float *kc = nullptr, *vc = nullptr;
  int max_seq = 0;
  int max_chunks = 0;
  float2* rope = nullptr;
  float* attn_part = nullptr;
  bool attn_fused = false;  // the O-projection's prologue combines the attention partials
  // contexts of at most ATTN_Q8K_MAX_CHUNKS chunks: one attention work group
  // per kv head leaves the O projection's input as Q8_K blocks (att_q8); a
  // launch at a longer context sets attn_err
  bool attn_q8k = false;
  int attn_q8k_chunks = ATTN_Q8K_CHUNKS;  // up to this many chunks (MCPM_ATTN_Q8K=n: n)
  BlockQ8K* att_q8 = nullptr;
  unsigned* attn_err = nullptr;
  // contexts of one chunk (at most 64 positions): the O projection's
  // work groups form the attention themselves (PRO_ATTN_ONE: each XCD's work
  // groups split the heads and share them through tagged records in that
  // XCD's L2), with no attention launch.  Needs head_dim 64, 4 query heads
  // per kv head, at most 2048 query dims, work group b on the XCD of b % 8
  // (checked at set-up) and enough O work groups per XCD; MCPM_ATTN_IN_O=0
  // turns it off.
  bool attn_in_o = false;
  uint64_t* xo_rec = nullptr;  // [8][heads * 64] records of each XCD
  unsigned* xo_words = nullptr;  // [0] token epoch, [64] error word, [128..135] XCD of work groups b % 8
  // graph
  bool use_graph = true;
  // [greedy (argmax at the end), sampled][longer contexts, contexts the
  // per-kv-head attention covers, one-chunk contexts with the attention in
  // the O projection]
  hipGraphExec_t graph[2][3] = {{nullptr, nullptr, nullptr}, {nullptr, nullptr, nullptr}};
  // timing
  int timing_class = -1;
  std::vector<TimedPair> events;
  size_t events_used = 0;
  int64_t weight_bytes = 0;
  // batched prompt processing
  bool use_prefill = true;
  PrefillBufs pf;
  // sampled decode: the token graph ends at the logits and the device sampler
  // picks the next token
  bool sample_mode = false;
  void* d_sample = nullptr;
  size_t sample_cap = 0;
  // the sampled graph ends with the sampler's passes, for these settings,
  // when they need no sort (a cut at most 0.998, or none); the draws are
  // read on the device, d_draws[step], one per generated token
  float smp_T = 0.0f, smp_P = 0.0f;
  bool smp_in_graph = false;
  float* d_draws = nullptr;  // out_cap floats
  // the FFN block as one launch (gate/up, grid barrier, down)
  bool fused_ffn = false;
  unsigned spin_limit = 0;  // waits' spin limit; 0: each kernel's default
  bool fused_attn = false;  // QKV and attention in one launch (launch_qkv_attn)
  unsigned* gsync = nullptr;  // GRID_SYNC_WORDS words
  // every layer of a token in one persistent launch, where the shape fits:
  // the plan for the current KV cache, each work group's weight slabs, the
  // hand-off records, launch count and error word, and the launch's
  // arguments in device memory
  // 0 off, 1 wherever the shape fits, 2 (default) where the launch has a
  // compiled instance for the shape (MCPM_PERSIST, mcpm_engine_set_persistent)
  int pd_mode = 2;
  bool pd_ready = false;
  PdShape pd{};
  PdLayer* d_pd_layers = nullptr;
  uint8_t* pd_slab = nullptr;
  int pd_slab_stride = 0;  // layout the slab was built for
  uint64_t* pd_rec = nullptr;
  unsigned* pd_sync = nullptr;  // [0] launch count, [64] error word
  float* pd_norms = nullptr;    // [L][2][dim] RMSNorm gains
  int* pd_xcc = nullptr;        // [G] the XCD of each work group at set-up
  PdArgs pd_args{};
};

namespace {

// The context's stream is non-blocking: it does not wait for the null stream,
// where hipMemset and hipMemcpy run.  Every fill or copy that work on the
// context's stream reads is therefore complete before the call that made it
// returns (or runs on the context's stream itself).
int alloc_dev(void** p, size_t bytes) {
  MCPM_HIP(hipMalloc(p, bytes ? bytes : 4));
  MCPM_HIP(hipMemset(*p, 0, bytes ? bytes : 4));
  MCPM_HIP(hipStreamSynchronize(nullptr));
  return MCPM_OK;
}

void drop_graph(mcpm_engine* e) {
  for (auto& mode : e->graph)
    for (hipGraphExec_t& g : mode) {
      if (g) (void)hipGraphExecDestroy(g);
      g = nullptr;
    }
}

void free_prefill(PrefillBufs& b) {
  for (void* p : {static_cast<void*>(b.tokens), static_cast<void*>(b.x),
                  static_cast<void*>(b.q), static_cast<void*>(b.g),
                  static_cast<void*>(b.u), static_cast<void*>(b.part), static_cast<void*>(b.xh),
                  static_cast<void*>(b.xbs), static_cast<void*>(b.xd)})
    if (p) (void)hipFree(p);
  b = PrefillBufs{};
}

void free_engine(mcpm_engine* e) {
  if (!e) return;
  (void)hipStreamSynchronize(e->ctx->stream);
  drop_graph(e);
  for (auto& p : e->events) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  free_tensor(e->embd);
  free_tensor(e->out_w);
  if (e->out_norm) (void)hipFree(e->out_norm);
  for (auto& l : e->L) {
    if (l.attn_norm) (void)hipFree(l.attn_norm);
    if (l.ffn_norm) (void)hipFree(l.ffn_norm);
    for (DevTensor* t : {&l.wq, &l.wk, &l.wv, &l.wo, &l.wg, &l.wu, &l.wd}) free_tensor(*t);
  }
  for (void* p : {static_cast<void*>(e->x), static_cast<void*>(e->q), static_cast<void*>(e->att),
                  static_cast<void*>(e->h), static_cast<void*>(e->logits), static_cast<void*>(e->argmax_part),
                  static_cast<void*>(e->st), static_cast<void*>(e->out_tokens), static_cast<void*>(e->kc),
                  static_cast<void*>(e->vc), static_cast<void*>(e->rope), static_cast<void*>(e->attn_part),
                  e->d_sample, static_cast<void*>(e->gsync), static_cast<void*>(e->d_draws),
                  static_cast<void*>(e->att_q8), static_cast<void*>(e->attn_err), static_cast<void*>(e->d_pd_layers),
                  static_cast<void*>(e->pd_slab), static_cast<void*>(e->pd_rec), static_cast<void*>(e->pd_sync),
                  static_cast<void*>(e->pd_norms), static_cast<void*>(e->pd_xcc), static_cast<void*>(e->xo_rec),
                  static_cast<void*>(e->xo_words)})
    if (p) (void)hipFree(p);
  if (e->h_st) (void)hipHostFree(e->h_st);
  free_prefill(e->pf);
  delete e;
}

int load_f32(mcpm_ctx* ctx, const GgufTensor* t, int n, float** out) {
  if (!t || t->type != MCPM_TYPE_F32 || static_cast<int64_t>(t->dims[0]) != n ||
      t->bytes != static_cast<size_t>(n) * sizeof(float))
    return fail(MCPM_ERR_FORMAT, "missing or malformed F32 tensor " + (t ? t->name : std::string("?")));
  MCPM_HIP(hipMalloc(out, n * sizeof(float)));
  MCPM_HIP(hipMemcpyAsync(*out, t->data, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  MCPM_HIP(hipStreamSynchronize(ctx->stream));
  return MCPM_OK;
}

int load_mat(mcpm_ctx* ctx, const GgufTensor* t, int64_t cols, int64_t rows, std::initializer_list<int> types,
             DevTensor& out, int64_t& bytes) {
  if (!t) return fail(MCPM_ERR_FORMAT, "missing tensor");
  if (t->dims.size() < 2 || static_cast<int64_t>(t->dims[0]) != cols || static_cast<int64_t>(t->dims[1]) != rows)
    return fail(MCPM_ERR_FORMAT, "tensor " + t->name + " has unexpected dims");
  if (std::find(types.begin(), types.end(), static_cast<int>(t->type)) == types.end())
    return fail(MCPM_ERR_UNSUPPORTED, "tensor " + t->name + " has unsupported type " + std::to_string(t->type));
  bytes += static_cast<int64_t>(t->bytes);
  return upload_tensor(ctx, t->data, t->bytes, static_cast<int>(t->type), cols, rows, out);
}

int load_from_image(mcpm_ctx* ctx, const uint8_t* data, size_t size, mcpm_engine** out) {
  GgufFile f;
  std::string err;
  if (!gguf_parse(data, size, f, err)) return fail(MCPM_ERR_FORMAT, "GGUF: " + err);
  std::string arch = "llama";
  f.get_str("general.architecture", arch);
  auto geti = [&](const std::string& k, int64_t dflt) {
    int64_t v;
    return f.get_int(arch + "." + k, v) ? v : dflt;
  };
  auto getf = [&](const std::string& k, double dflt) {
    double v;
    return f.get_float(arch + "." + k, v) ? v : dflt;
  };
  mcpm_model_config c{};
  c.n_layers = static_cast<int>(geti("block_count", 0));
  c.dim = static_cast<int>(geti("embedding_length", 0));
  c.ffn = static_cast<int>(geti("feed_forward_length", 0));
  c.n_heads = static_cast<int>(geti("attention.head_count", 0));
  c.n_kv_heads = static_cast<int>(geti("attention.head_count_kv", c.n_heads));
  c.head_dim = c.n_heads ? static_cast<int>(geti("attention.key_length", c.dim / c.n_heads)) : 0;
  c.rope_base = static_cast<float>(getf("rope.freq_base", 10000.0));
  c.eps = static_cast<float>(getf("attention.layer_norm_rms_epsilon", 1e-6));
  const GgufTensor* te = f.find("token_embd.weight");
  if (!te || te->dims.size() < 2) return fail(MCPM_ERR_FORMAT, "GGUF: token_embd.weight missing");
  c.vocab = static_cast<int>(te->dims[1]);
  const GgufTensor* td0 = f.find("blk.0.ffn_down.weight");
  c.ffn_pad = td0 ? static_cast<int>(td0->dims[0]) : (c.ffn + 255) / 256 * 256;
  const GgufTensor* to = f.find("output.weight");
  c.tied_embeddings = to ? 0 : 1;
  const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  if (c.n_layers <= 0 || c.dim <= 0 || c.vocab <= 0 || c.n_heads <= 0 || c.head_dim <= 0 || qd <= 0 ||
      c.dim % QK_K || c.dim / QK_K > MAX_NB || qd % QK_K || qd / QK_K > MAX_NB ||
      c.ffn <= 0 || c.ffn_pad < c.ffn || c.ffn_pad % QK_K || c.ffn_pad / QK_K > MAX_NB || c.n_kv_heads <= 0 ||
      c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 8 || c.head_dim % 8 || c.head_dim > 128 ||
      kvd % 8 || c.n_kv_heads > 256)
    return fail(MCPM_ERR_FORMAT, "GGUF: model shape not supported by the engine");

  auto* e = new mcpm_engine();
  e->ctx = ctx;
  e->cfg = c;
  e->attn_fused = qd / QK_K <= 8 && c.head_dim % 8 == 0;
  int rc = MCPM_OK;
  int64_t wb = 0;
  auto T = [&](const std::string& n) { return f.find(n); };
  rc = load_mat(ctx, te, c.dim, c.vocab, {MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K}, e->embd, wb);
  const int64_t embd_bytes = wb;
  wb = 0;
  if (!rc) rc = load_f32(ctx, T("output_norm.weight"), c.dim, &e->out_norm);
  if (!rc && to) rc = load_mat(ctx, to, c.dim, c.vocab, {MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K}, e->out_w, wb);
  if (!rc && !to) {
    e->out_w = e->embd;
    e->out_w.owned = false;
    wb += embd_bytes;
  }
  e->L.resize(c.n_layers);
  for (int l = 0; l < c.n_layers && !rc; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Layer& L = e->L[l];
    rc = load_f32(ctx, T(p + "attn_norm.weight"), c.dim, &L.attn_norm);
    if (!rc) rc = load_f32(ctx, T(p + "ffn_norm.weight"), c.dim, &L.ffn_norm);
    if (!rc) rc = load_mat(ctx, T(p + "attn_q.weight"), c.dim, qd, {MCPM_TYPE_Q4_K}, L.wq, wb);
    if (!rc) rc = load_mat(ctx, T(p + "attn_k.weight"), c.dim, kvd, {MCPM_TYPE_Q4_K}, L.wk, wb);
    if (!rc) rc = load_mat(ctx, T(p + "attn_v.weight"), c.dim, kvd, {MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K}, L.wv, wb);
    if (!rc) rc = load_mat(ctx, T(p + "attn_output.weight"), qd, c.dim, {MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K}, L.wo, wb);
    if (!rc) rc = load_mat(ctx, T(p + "ffn_gate.weight"), c.dim, c.ffn, {MCPM_TYPE_Q4_K}, L.wg, wb);
    if (!rc) rc = load_mat(ctx, T(p + "ffn_up.weight"), c.dim, c.ffn, {MCPM_TYPE_Q4_K}, L.wu, wb);
    if (!rc) rc = load_mat(ctx, T(p + "ffn_down.weight"), c.ffn_pad, c.dim, {MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K}, L.wd, wb);
    wb += 2 * static_cast<int64_t>(c.dim) * 4;  // the two norm gains
  }
  // per token: every layer, LM head, output norm, one embedding row
  e->weight_bytes = wb + static_cast<int64_t>(c.dim) * 4 + static_cast<int64_t>(embd_bytes / c.vocab);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->x), c.dim * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->q), qd * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->att), qd * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->h), c.ffn_pad * 4);  // padding stays zero
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->logits), static_cast<size_t>(c.vocab) * 4);
  if (!rc) {
    GemvArgs a{};
    a.reg[0].w = view_of(e->out_w);  // the kernel instance (and its occupancy) follows the head's type
    a.total_rows = c.vocab;
    a.nreg = 1;
    a.nb = c.dim / QK_K;
    e->lm_grid = gemv_grid(a, ctx->n_cu);
    rc = alloc_dev(reinterpret_cast<void**>(&e->argmax_part), e->lm_grid * sizeof(float2));
  }
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->st), sizeof(StepState));
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->gsync), GRID_SYNC_WORDS * sizeof(unsigned));
  if (!rc && e->attn_fused && attn_q8k_fits(c.n_heads, c.n_kv_heads, c.head_dim)) {
    const char* v = std::getenv("MCPM_ATTN_Q8K");
    e->attn_q8k = !v || std::atoi(v) != 0;
    if (v && std::atoi(v) > 0) e->attn_q8k_chunks = std::min(std::atoi(v), ATTN_Q8K_MAX_CHUNKS);
    if (e->attn_q8k) rc = alloc_dev(reinterpret_cast<void**>(&e->att_q8), (qd / QK_K) * sizeof(BlockQ8K));
    if (!rc && e->attn_q8k) rc = alloc_dev(reinterpret_cast<void**>(&e->attn_err), sizeof(unsigned));
  }
  if (!rc && c.head_dim == 64 && c.n_heads == 4 * c.n_kv_heads && qd / QK_K <= 8 && qd % QK_K == 0 &&
      c.n_layers > 0) {
    const char* v = std::getenv("MCPM_ATTN_IN_O");
    GemvArgs o{};
    o.reg[0] = GemvRegion{view_of(e->L[0].wo), nullptr, 0, c.dim};
    o.nreg = 1;
    o.total_rows = c.dim;
    o.nb = qd / QK_K;
    bool same_types = true;
    for (const Layer& y : e->L) same_types = same_types && y.wo.type == e->L[0].wo.type;
    if ((!v || std::atoi(v) != 0) && same_types && gemv_attn_one_hpw(o, ctx->n_cu) > 0) {
      rc = alloc_dev(reinterpret_cast<void**>(&e->xo_words), 192 * sizeof(unsigned));
      if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->xo_rec), static_cast<size_t>(8) * qd * sizeof(uint64_t));
      int* probe = nullptr;
      if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&probe), 256 * sizeof(int));
      bool same = false;
      if (!rc && pd_probe_xcd(256, probe, ctx->stream, same) != hipSuccess) rc = MCPM_ERR_HIP;
      if (!rc && same) {
        rc = hipMemcpyAsync(e->xo_words + 128, probe, 8 * sizeof(int), hipMemcpyDeviceToDevice, ctx->stream) ==
                     hipSuccess && hipStreamSynchronize(ctx->stream) == hipSuccess
                 ? MCPM_OK
                 : MCPM_ERR_HIP;
        e->attn_in_o = !rc;
      }
      if (probe) (void)hipFree(probe);
    }
  }
  if (rc) {
    free_engine(e);
    return rc;
  }
  {
    const char* f = std::getenv("MCPM_FUSED_FFN");
    e->fused_ffn = f && std::atoi(f) != 0;
    const char* a = std::getenv("MCPM_FUSED_ATTN");
    e->fused_attn = a && std::atoi(a) != 0;
    const char* pv = std::getenv("MCPM_PERSIST");
    if (pv) e->pd_mode = std::atoi(pv) == 0 ? 0 : std::atoi(pv) == 2 ? 2 : 1;
  }
  *out = e;
  return MCPM_OK;
}

int ensure_out_tokens(mcpm_engine* e, int n) {
  if (n <= e->out_cap) return MCPM_OK;
  if (e->out_tokens || e->d_draws) MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  if (e->out_tokens) (void)hipFree(e->out_tokens);
  if (e->d_draws) (void)hipFree(e->d_draws);
  e->out_tokens = nullptr;
  e->d_draws = nullptr;
  e->out_cap = 0;
  drop_graph(e);  // the argmax and sampler nodes hold the arrays' pointers
  int rc = alloc_dev(reinterpret_cast<void**>(&e->out_tokens), n * sizeof(int));
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->d_draws), n * sizeof(float));
  if (rc) return rc;
  e->out_cap = n;
  return MCPM_OK;
}

int ensure_staging(mcpm_engine* e, int n) {
  if (n <= e->h_st_cap) return MCPM_OK;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  if (e->h_st) (void)hipHostFree(e->h_st);
  e->h_st = nullptr;
  e->h_st_cap = 0;
  MCPM_HIP(hipHostMalloc(reinterpret_cast<void**>(&e->h_st), n * sizeof(StepState), hipHostMallocDefault));
  e->h_st_cap = n;
  return MCPM_OK;
}

// Launch helper: when its class is timed, the launch records an event pair at
// its kernel's start and end.
template <class F>
hipError_t timed(mcpm_engine* e, int kc, F&& launch) {
  if (kc != e->timing_class) return launch();
  if (e->events_used == e->events.size()) {
    TimedPair p;
    hipError_t err = hipEventCreate(&p.a);
    if (err == hipSuccess) err = hipEventCreate(&p.b);
    if (err != hipSuccess) return err;
    e->events.push_back(p);
  }
  TimedPair& p = e->events[e->events_used++];
  g_launch_timing = LaunchTiming{p.a, p.b};
  const hipError_t err = launch();
  g_launch_timing = LaunchTiming{};
  return err;
}

// After the stream is idle: a grid barrier of a fused kernel that gave up
// (spin limit) left its error word set; report it and reset the barrier
// state for the next launches.
unsigned grid_spin_limit(const mcpm_engine* e) { return e->spin_limit ? e->spin_limit : 1u << 20; }
unsigned pd_spin_limit(const mcpm_engine* e) { return e->spin_limit ? e->spin_limit : 1u << 18; }

int check_grid_sync(mcpm_engine* e) {
  hipStream_t s = e->ctx->stream;
  // every error source is read and reset before the first one is reported,
  // so that the next call starts clean whichever waits gave up
  const char* msg = nullptr;
  auto note = [&](const char* m) {
    if (!msg) msg = m;
  };
  if (e->attn_in_o) {
    unsigned xerr = 0;
    MCPM_HIP(hipMemcpyAsync(&xerr, e->xo_words + 64, sizeof xerr, hipMemcpyDeviceToHost, s));
    MCPM_HIP(hipStreamSynchronize(s));
    if (xerr) {
      // the epoch advances every token, so no record of the abandoned
      // launches carries a later tag
      MCPM_HIP(hipMemsetAsync(e->xo_words + 64, 0, sizeof(unsigned), s));
      MCPM_HIP(hipStreamSynchronize(s));
      note("the O projection's attention hand-off gave up waiting (spin limit, or a work group on another XCD); "
           "results of the call are invalid (MCPM_ATTN_IN_O=0 runs the attention as its own launch)");
    }
  }
  if (e->attn_q8k) {
    unsigned aerr = 0;
    MCPM_HIP(hipMemcpyAsync(&aerr, e->attn_err, sizeof aerr, hipMemcpyDeviceToHost, s));
    MCPM_HIP(hipStreamSynchronize(s));
    if (aerr) {
      MCPM_HIP(hipMemsetAsync(e->attn_err, 0, sizeof(unsigned), s));
      MCPM_HIP(hipStreamSynchronize(s));
      note("the per-kv-head attention ran past its context limit; results of the call are invalid");
    }
  }
  if (e->pd_ready) {
    unsigned perr = 0;
    MCPM_HIP(hipMemcpyAsync(&perr, e->pd_sync + 64, sizeof perr, hipMemcpyDeviceToHost, s));
    MCPM_HIP(hipStreamSynchronize(s));
    if (perr) {
      // records of the abandoned launch may carry tags a later launch would
      // take: clear them and restart the launch count
      const unsigned init[1] = {1u};
      MCPM_HIP(hipMemsetAsync(e->pd_rec, 0, pd_records(e->pd) * sizeof(uint64_t), s));
      MCPM_HIP(hipMemsetAsync(e->pd_sync, 0, 128 * sizeof(unsigned), s));
      MCPM_HIP(hipMemcpyAsync(e->pd_sync, init, sizeof init, hipMemcpyHostToDevice, s));
      MCPM_HIP(hipStreamSynchronize(s));
      note(perr == 2u ? "the persistent decode launch ran a work group on another XCD than at set-up; results of "
                        "the call are invalid (MCPM_PD_XCD_LOCAL=0 keeps every hand-off at agent scope)"
                      : "the persistent decode launch gave up waiting (spin limit); results of the call are invalid");
    }
  }
  if (e->fused_ffn || e->fused_attn) {
    unsigned err = 0;
    MCPM_HIP(hipMemcpyAsync(&err, e->gsync + 8 * 64 + 64, sizeof err, hipMemcpyDeviceToHost, s));
    MCPM_HIP(hipStreamSynchronize(s));
    if (err) {
      MCPM_HIP(hipMemsetAsync(e->gsync, 0, GRID_SYNC_WORDS * sizeof(unsigned), s));
      MCPM_HIP(hipStreamSynchronize(s));
      note("a fused kernel's grid barrier timed out; results of the call are invalid");
    }
  }
  return msg ? fail(MCPM_ERR_HIP, msg) : MCPM_OK;
}

// All kernels of one token, reading token and pos from e->st.  short_ctx:
// the context (pos + 1) has at most ATTN_Q8K_MAX_CHUNKS chunks; one_chunk:
// at most one chunk, and the O projection forms the attention (attn_in_o).
int enqueue_token(mcpm_engine* e, bool short_ctx, bool one_chunk) {
  const mcpm_model_config& c = e->cfg;
  hipStream_t s = e->ctx->stream;
  const int n_cu = e->ctx->n_cu;
  const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  const int* st = reinterpret_cast<const int*>(e->st);
  const bool in_o = one_chunk && e->attn_in_o && !e->fused_attn;
  const bool q8k = short_ctx && e->attn_q8k && !e->fused_attn && !in_o;
  const bool persist = e->pd_ready && e->pd_mode != 0;
  if (persist)
    MCPM_HIP(timed(e, MCPM_KC_LAYERS, [&] { return launch_decode_persist(e->pd_args, s); }));
  else
    MCPM_HIP(launch_embedding(view_of(e->embd), st, c.dim, e->x, s, e->attn_in_o ? e->xo_words : nullptr));
  for (int l = 0; l < c.n_layers && !persist; ++l) {
    const Layer& L = e->L[l];
    float* kc = e->kc + static_cast<size_t>(l) * e->max_seq * kvd;
    float* vc = e->vc + static_cast<size_t>(l) * e->max_seq * kvd;
    const AttnPart part = attn_part_of(e->attn_part, c.n_heads, e->max_chunks, c.head_dim);
    {
      GemvArgs a{};
      a.reg[0] = GemvRegion{view_of(L.wq), e->q, 0, qd};
      a.reg[1] = GemvRegion{view_of(L.wk), nullptr, qd, kvd};
      a.reg[2] = GemvRegion{view_of(L.wv), nullptr, qd + kvd, kvd};
      a.nreg = 3;
      a.total_rows = qd + 2 * kvd;
      a.nb = c.dim / QK_K;
      a.x = e->x;
      a.gamma = L.attn_norm;
      a.eps = c.eps;
      a.state = st;
      a.rope_cs = e->rope;
      a.head_dim = c.head_dim;
      a.k_cache = kc;
      a.v_cache = vc;
      a.kvd = kvd;
      hipError_t fe = hipErrorNotSupported;
      if (e->fused_attn) {
        const GridSync gs{e->gsync, e->gsync + 8 * 64, e->gsync + 8 * 64 + 64, grid_spin_limit(e)};
        const AttnArgs at{e->q, kc, vc, st, c.n_heads, c.n_kv_heads, c.head_dim, e->max_chunks, part.o, part.mz};
        fe = timed(e, MCPM_KC_QKV, [&] { return launch_qkv_attn(a, at, n_cu, gs, s); });
        if (fe != hipSuccess && fe != hipErrorNotSupported) MCPM_HIP(fe);
      }
      if (fe == hipErrorNotSupported) {
        MCPM_HIP(timed(e, MCPM_KC_QKV, [&] { return launch_gemv(a, PRO_NORM_AWAY, EPI_QKV, n_cu, s); }));
        if (!in_o) MCPM_HIP(timed(e, MCPM_KC_ATTN, [&] {
          if (q8k)
            return launch_attention_q8k(e->q, kc, vc, st, c.n_heads, c.n_kv_heads, c.head_dim, e->att_q8,
                                        e->attn_err, s);
          return launch_attention(e->q, kc, vc, st, c.n_heads, c.n_kv_heads, c.head_dim, e->max_chunks, part, s);
        }));
      }
    }
    if (in_o) {
      // every head's attention over the one chunk, then its ties-even Q8_K,
      // in the O projection's prologue
      GemvArgs a{};
      a.reg[0] = GemvRegion{view_of(L.wo), nullptr, 0, c.dim};
      a.nreg = 1;
      a.total_rows = c.dim;
      a.nb = qd / QK_K;
      a.resid = e->x;
      a.x = e->q;
      a.state = st;
      a.head_dim = c.head_dim;
      a.k_cache = kc;
      a.v_cache = vc;
      a.kvd = kvd;
      a.xrec = e->xo_rec;
      a.epoch = e->xo_words;
      a.tag_mul = static_cast<unsigned>(c.n_layers + 1);
      a.tag_add = static_cast<unsigned>(l + 1);
      a.xcc = reinterpret_cast<const int*>(e->xo_words + 128);
      a.err = e->xo_words + 64;
      a.spin_limit = grid_spin_limit(e);
      MCPM_HIP(timed(e, MCPM_KC_OPROJ, [&] { return launch_gemv(a, PRO_ATTN_ONE, EPI_RESID, n_cu, s); }));
    } else if (q8k) {
      // the attention output is already the O projection's Q8_K input
      GemvArgs a{};
      a.reg[0] = GemvRegion{view_of(L.wo), nullptr, 0, c.dim};
      a.nreg = 1;
      a.total_rows = c.dim;
      a.nb = qd / QK_K;
      a.resid = e->x;
      a.xq = e->att_q8;
      MCPM_HIP(timed(e, MCPM_KC_OPROJ, [&] { return launch_gemv(a, PRO_Q8K, EPI_RESID, n_cu, s); }));
    } else {
      // the attention output is combined from its chunk partials in this
      // GEMV's prologue where the shape allows, else by its own kernel
      GemvArgs a{};
      a.reg[0] = GemvRegion{view_of(L.wo), nullptr, 0, c.dim};
      a.nreg = 1;
      a.total_rows = c.dim;
      a.nb = qd / QK_K;
      a.resid = e->x;
      if (e->attn_fused) {
        a.x = part.o;
        a.attn_mz = part.mz;
        a.attn_max_chunks = e->max_chunks;
        a.head_dim = c.head_dim;
        a.state = st;
        MCPM_HIP(timed(e, MCPM_KC_OPROJ, [&] { return launch_gemv(a, PRO_ATTN_EVEN, EPI_RESID, n_cu, s); }));
      } else {
        MCPM_HIP(launch_attn_combine(part, st, c.n_heads, c.head_dim, e->max_chunks, e->att, s));
        a.x = e->att;
        MCPM_HIP(timed(e, MCPM_KC_OPROJ, [&] { return launch_gemv(a, PRO_QUANT_EVEN, EPI_RESID, n_cu, s); }));
      }
    }
    {
      GemvArgs gu{};
      gu.reg[0] = GemvRegion{view_of(L.wg), nullptr, 0, c.ffn};
      gu.reg[1] = GemvRegion{view_of(L.wu), nullptr, 0, c.ffn};
      gu.nreg = 2;
      gu.pair = 1;
      gu.total_rows = c.ffn;
      gu.nb = c.dim / QK_K;
      gu.x = e->x;
      gu.gamma = L.ffn_norm;
      gu.eps = c.eps;
      gu.h_out = e->h;
      GemvArgs dn{};
      dn.reg[0] = GemvRegion{view_of(L.wd), nullptr, 0, c.dim};
      dn.nreg = 1;
      dn.total_rows = c.dim;
      dn.nb = c.ffn_pad / QK_K;
      dn.x = e->h;
      dn.resid = e->x;
      hipError_t fe = hipErrorNotSupported;
      if (e->fused_ffn) {
        const GridSync gs{e->gsync, e->gsync + 8 * 64, e->gsync + 8 * 64 + 64, grid_spin_limit(e)};
        fe = timed(e, MCPM_KC_GATE_UP, [&] { return launch_ffn_fused(gu, dn, n_cu, gs, s); });
        if (fe != hipSuccess && fe != hipErrorNotSupported) MCPM_HIP(fe);
      }
      if (fe == hipErrorNotSupported) {
        MCPM_HIP(timed(e, MCPM_KC_GATE_UP, [&] { return launch_gemv(gu, PRO_NORM_AWAY, EPI_SWIGLU, n_cu, s); }));
        MCPM_HIP(timed(e, MCPM_KC_DOWN, [&] { return launch_gemv(dn, PRO_QUANT_AWAY, EPI_RESID, n_cu, s); }));
      }
    }
  }
  {
    GemvArgs a{};
    a.reg[0] = GemvRegion{view_of(e->out_w), e->logits, 0, c.vocab};
    a.nreg = 1;
    a.total_rows = c.vocab;
    a.nb = c.dim / QK_K;
    a.x = e->x;
    a.gamma = e->out_norm;
    a.eps = c.eps;
    a.argmax_part = e->argmax_part;
    a.argmax_parts = e->lm_grid;
    MCPM_HIP(timed(e, MCPM_KC_LM_HEAD, [&] { return launch_gemv(a, PRO_NORM_EVEN, EPI_LOGITS, n_cu, s); }));
  }
  if (!e->sample_mode) MCPM_HIP(launch_argmax_final(e->argmax_part, e->lm_grid, nullptr, e->st, e->out_tokens, s));
  else if (e->smp_in_graph)
    MCPM_HIP(launch_sample(e->d_sample, e->sample_cap, e->logits, c.vocab, e->smp_T, e->smp_P, 0.0f, nullptr, e->st,
                           e->out_tokens, s, e->d_draws));
  return MCPM_OK;
}

// One token at position pos (the position the step state holds when the
// token's kernels run): the graph for its context length.
int run_token(mcpm_engine* e, int pos) {
  const bool short_ctx = pos / ATTN_CHUNK + 1 <= e->attn_q8k_chunks;
  const bool one_chunk = pos < ATTN_CHUNK;
  // Events recorded inside a captured graph cannot be read back with
  // hipEventElapsedTime, so a timed kernel class runs the same launches eagerly.
  if (!e->use_graph || e->timing_class >= 0) return enqueue_token(e, short_ctx, one_chunk);
  const int regime = one_chunk && e->attn_in_o ? 2 : short_ctx && e->attn_q8k ? 1 : 0;
  hipGraphExec_t& graph = e->graph[e->sample_mode ? 1 : 0][regime];
  if (!graph) {
    hipStream_t s = e->ctx->stream;
    MCPM_HIP(hipStreamSynchronize(s));
    MCPM_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_token(e, short_ctx, one_chunk);
    hipGraph_t g = nullptr;
    const hipError_t ce = hipStreamEndCapture(s, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (ce != hipSuccess) return hip_fail(ce, "hipStreamEndCapture");
    const hipError_t ie = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) {
      graph = nullptr;
      return hip_fail(ie, "hipGraphInstantiate");
    }
  }
  MCPM_HIP(hipGraphLaunch(graph, e->ctx->stream));
  return MCPM_OK;
}

// Queues a state write (token, pos) from pinned staging slot `slot`.
int queue_state(mcpm_engine* e, int slot, int token, int pos, int step) {
  StepState& hs = e->h_st[slot];
  hs.token = token;
  hs.pos = pos;
  hs.step = step;
  hs.n_out = e->out_cap;
  MCPM_HIP(hipMemcpyAsync(e->st, &hs, sizeof(StepState), hipMemcpyHostToDevice, e->ctx->stream));
  return MCPM_OK;
}

int ensure_prefill(mcpm_engine* e, int cap) {
  PrefillBufs& b = e->pf;
  if (cap <= b.cap && b.max_chunks == e->max_chunks) return MCPM_OK;
  free_prefill(b);
  const mcpm_model_config& c = e->cfg;
  const size_t qd = static_cast<size_t>(c.n_heads) * c.head_dim;
  const size_t kmax = std::max<size_t>({static_cast<size_t>(c.dim), qd, static_cast<size_t>(c.ffn_pad)});
  const size_t n = static_cast<size_t>(cap);
  int rc = alloc_dev(reinterpret_cast<void**>(&b.tokens), n * sizeof(int));
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.x), n * c.dim * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.q), n * qd * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.g), n * c.ffn * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.u), n * c.ffn * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.part), n * c.n_heads * e->max_chunks * (c.head_dim + 2) * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.xh), n * kmax * 2);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.xd), n * (kmax / QK_K) * 4);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&b.xbs), n * (kmax / QK_K) * 16 * 2);
  if (rc) {
    free_prefill(b);
    return rc;
  }
  b.cap = cap;
  b.max_chunks = e->max_chunks;
  return MCPM_OK;
}

// Every layer for tokens at positions pos0 .. pos0+n-1 (n <= the scratch
// capacity), leaving their K and V rows in the cache exactly as per-token
// decode leaves them.  The last layer stops after its K/V rows.
int prefill_pass(mcpm_engine* e, const int* tokens, int n, int pos0) {
  const mcpm_model_config& c = e->cfg;
  hipStream_t s = e->ctx->stream;
  PrefillBufs& b = e->pf;
  const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  const QuantBatch qb{b.xh, b.xd, b.xbs};
  MCPM_HIP(hipMemcpyAsync(b.tokens, tokens, n * sizeof(int), hipMemcpyHostToDevice, s));
  MCPM_HIP(launch_embed_batch(view_of(e->embd), b.tokens, n, c.dim, b.x, s));
  const AttnPart part = attn_part_of(b.part, n * c.n_heads, e->max_chunks, c.head_dim);
  const size_t tok_o = static_cast<size_t>(c.n_heads) * e->max_chunks * c.head_dim;
  const size_t tok_mz = static_cast<size_t>(c.n_heads) * e->max_chunks;
  for (int l = 0; l < c.n_layers; ++l) {
    const Layer& L = e->L[l];
    float* kc = e->kc + static_cast<size_t>(l) * e->max_seq * kvd;
    float* vc = e->vc + static_cast<size_t>(l) * e->max_seq * kvd;
    const int nbd = c.dim / QK_K;
    MCPM_HIP(launch_quant_batch(b.x, nullptr, c.dim, L.attn_norm, c.eps, c.dim, c.dim, PRO_NORM_AWAY, n, qb, s));
    // q rotated into b.q and k rotated into the cache rows by the GEMM's
    // RoPE epilogue, in one launch when q and k share a type (q's rows a
    // multiple of 64); v straight into the cache rows
    const WView wq = view_of(L.wq), wk = view_of(L.wk), wg = view_of(L.wg), wu = view_of(L.wu);
    const GemmRope rp{e->rope, c.head_dim, pos0};
    float* krows = kc + static_cast<size_t>(pos0) * kvd;
    float* vrows = vc + static_cast<size_t>(pos0) * kvd;
    if (wq.type == wk.type && qd % 64 == 0) {
      MCPM_HIP(launch_gemm_q8k(wq, qd, nbd, n, qb, b.q, qd, false, s, &wk, kvd, krows, kvd, &rp));
    } else {
      MCPM_HIP(launch_gemm_q8k(wq, qd, nbd, n, qb, b.q, qd, false, s, nullptr, 0, nullptr, 0, &rp));
      MCPM_HIP(launch_gemm_q8k(wk, kvd, nbd, n, qb, krows, kvd, false, s, nullptr, 0, nullptr, 0, &rp));
    }
    MCPM_HIP(launch_gemm_q8k(view_of(L.wv), kvd, nbd, n, qb, vrows, kvd, false, s));
    if (l == c.n_layers - 1) break;  // nothing after the last K/V rows reaches the cache
    MCPM_HIP(launch_attention_batch(b.q, kc, vc, c.n_heads, c.n_kv_heads, c.head_dim, e->max_chunks, part, tok_o,
                                    tok_mz, pos0, n, s));
    MCPM_HIP(launch_quant_batch_attn(part, tok_o, tok_mz, pos0, n, c.n_heads, c.head_dim, e->max_chunks, qb, s));
    MCPM_HIP(launch_gemm_q8k(view_of(L.wo), c.dim, qd / QK_K, n, qb, b.x, c.dim, true, s));
    MCPM_HIP(launch_quant_batch(b.x, nullptr, c.dim, L.ffn_norm, c.eps, c.dim, c.dim, PRO_NORM_AWAY, n, qb, s));
    if (wg.type == wu.type && c.ffn % 64 == 0) {
      // gate and up in one launch, h = silu(gate)*up written by its epilogue
      MCPM_HIP(launch_gemm_q8k(wg, c.ffn, nbd, n, qb, b.g, c.ffn, false, s, &wu, c.ffn, nullptr, 0, nullptr, true));
      MCPM_HIP(launch_quant_batch(b.g, nullptr, c.ffn, nullptr, 0.0f, c.ffn_pad, c.ffn, PRO_QUANT_AWAY, n, qb, s));
    } else {
      MCPM_HIP(launch_gemm_q8k(wg, c.ffn, nbd, n, qb, b.g, c.ffn, false, s));
      MCPM_HIP(launch_gemm_q8k(wu, c.ffn, nbd, n, qb, b.u, c.ffn, false, s));
      MCPM_HIP(launch_quant_batch_swiglu(b.g, b.u, c.ffn, c.ffn, c.ffn_pad, n, qb, s));
    }
    MCPM_HIP(launch_gemm_q8k(view_of(L.wd), c.dim, c.ffn_pad / QK_K, n, qb, b.x, c.dim, true, s));
  }
  return MCPM_OK;
}

// The persistent decode path for the current KV cache: plan, weight slabs
// (built once per layout), hand-off records, launch count and arguments.
// Leaves pd_ready false (the five-launch path) when the shape or the
// context does not fit.
// The persistent launch's large buffers (the weight slab: the model's layer
// weights once more) are held only while the launch is asked for.
void pd_release(mcpm_engine* e) {
  for (void** p : {reinterpret_cast<void**>(&e->pd_slab), reinterpret_cast<void**>(&e->d_pd_layers),
                   reinterpret_cast<void**>(&e->pd_rec), reinterpret_cast<void**>(&e->pd_xcc)}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  e->pd_slab_stride = 0;
  e->pd_ready = false;
}

int pd_setup(mcpm_engine* e) {
  e->pd_ready = false;
  const mcpm_model_config& c = e->cfg;
  if (e->pd_mode == 0) {
    pd_release(e);
    return MCPM_OK;
  }
  if (!e->kc || c.n_layers <= 0) return MCPM_OK;
  const Layer& L0 = e->L[0];
  PdShape s{};
  const char* why = nullptr;
  if (!pd_plan(c, e->ctx->n_cu, e->max_seq, L0.wq.type, L0.wk.type, L0.wv.type, L0.wo.type, L0.wd.type, s, &why) ||
      (e->pd_mode == 2 && !pd_fixed_shape(s))) {
    // the default mode holds no slab for a shape it does not take
    if (e->pd_mode == 2) pd_release(e);
    return MCPM_OK;
  }
  if (prepare_decode_persist(s) != hipSuccess) return MCPM_OK;
  // every layer must have the first layer's types (the slab layout's)
  for (const Layer& l : e->L)
    if (l.wq.type != s.sq.type || l.wk.type != s.sk.type || l.wv.type != s.sv.type || l.wo.type != s.so.type ||
        l.wd.type != s.sd.type || l.wg.type != MCPM_TYPE_Q4_K || l.wu.type != MCPM_TYPE_Q4_K)
      return MCPM_OK;
  hipStream_t st = e->ctx->stream;
  MCPM_HIP(hipStreamSynchronize(st));
  if (!e->pd_slab || e->pd_slab_stride != s.slab_stride || e->pd.G != s.G) {
    if (e->pd_slab) (void)hipFree(e->pd_slab);
    if (e->d_pd_layers) (void)hipFree(e->d_pd_layers);
    e->pd_slab = nullptr;
    e->d_pd_layers = nullptr;
    std::vector<PdLayer> hl(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
      const Layer& y = e->L[l];
      hl[l] = PdLayer{y.attn_norm, y.ffn_norm, view_of(y.wq), view_of(y.wk), view_of(y.wv), view_of(y.wo),
                      view_of(y.wg), view_of(y.wu), view_of(y.wd)};
    }
    const size_t slab_bytes = static_cast<size_t>(c.n_layers) * s.G * s.slab_stride;
    int rc = alloc_dev(reinterpret_cast<void**>(&e->d_pd_layers), hl.size() * sizeof(PdLayer));
    if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->pd_slab), slab_bytes);
    if (rc) return rc;
    MCPM_HIP(hipMemcpyAsync(e->d_pd_layers, hl.data(), hl.size() * sizeof(PdLayer), hipMemcpyHostToDevice, st));
    MCPM_HIP(launch_build_slab(s, e->d_pd_layers, e->pd_slab, st));
    MCPM_HIP(hipStreamSynchronize(st));
    e->pd_slab_stride = s.slab_stride;
  }
  if (e->pd_rec) (void)hipFree(e->pd_rec);
  if (e->pd_xcc) (void)hipFree(e->pd_xcc);
  e->pd_rec = nullptr;
  e->pd_xcc = nullptr;
  int rc = alloc_dev(reinterpret_cast<void**>(&e->pd_rec), pd_records(s) * sizeof(uint64_t));
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->pd_xcc), static_cast<size_t>(s.G) * sizeof(int));
  if (!rc && !e->pd_sync) rc = alloc_dev(reinterpret_cast<void**>(&e->pd_sync), 128 * sizeof(unsigned));
  if (!rc && !e->pd_norms)
    rc = alloc_dev(reinterpret_cast<void**>(&e->pd_norms), static_cast<size_t>(c.n_layers) * 2 * c.dim * sizeof(float));
  if (rc) return rc;
  for (int l = 0; l < c.n_layers; ++l) {
    float* dst = e->pd_norms + static_cast<size_t>(2 * l) * c.dim;
    MCPM_HIP(hipMemcpyAsync(dst, e->L[l].attn_norm, c.dim * sizeof(float), hipMemcpyDeviceToDevice, st));
    MCPM_HIP(hipMemcpyAsync(dst + c.dim, e->L[l].ffn_norm, c.dim * sizeof(float), hipMemcpyDeviceToDevice, st));
  }
  // XCD-local records (workgroup-scope stores read from the XCD's L2) need
  // every work group b on the XCD of b % 8; MCPM_PD_XCD_LOCAL=0 keeps every
  // record at agent scope
  bool same_xcd = false;
  MCPM_HIP(pd_probe_xcd(s.G, e->pd_xcc, st, same_xcd));
  const char* xv = std::getenv("MCPM_PD_XCD_LOCAL");
  const bool xcd_local = same_xcd && !(xv && std::atoi(xv) == 0);
  const unsigned init[2] = {1u, 0u};  // launch count 1: no record (all zero) carries a tag
  MCPM_HIP(hipMemsetAsync(e->pd_sync, 0, 128 * sizeof(unsigned), st));
  MCPM_HIP(hipMemcpyAsync(e->pd_sync, init, sizeof(unsigned), hipMemcpyHostToDevice, st));
  MCPM_HIP(hipStreamSynchronize(st));
  PdArgs a{};
  a.s = s;
  a.norms = e->pd_norms;
  a.slab = e->pd_slab;
  a.kc = e->kc;
  a.vc = e->vc;
  a.max_seq = e->max_seq;
  a.rope = e->rope;
  a.state = reinterpret_cast<const int*>(e->st);
  a.embd = view_of(e->embd);
  pd_bind_records(a, e->pd_rec);
  a.epoch = e->pd_sync;
  a.err = e->pd_sync + 64;
  a.spin_limit = pd_spin_limit(e);
  a.x_out = e->x;
  a.xcd_local = xcd_local ? 1 : 0;
  a.xcc = e->pd_xcc;
  e->pd_args = a;
  e->pd = s;
  e->pd_ready = true;
  return MCPM_OK;
}

}  // namespace

extern "C" {

int mcpm_engine_prefill(mcpm_engine* e, const int* tokens, int n, int pos0) {
  if (!e || (!tokens && n) || n < 0 || pos0 < 0) return fail(MCPM_ERR_ARG, "mcpm_engine_prefill: bad argument");
  if (!e->kc) return fail(MCPM_ERR_CONTEXT, "mcpm_engine_prefill: KV cache not initialised");
  if (pos0 + n > e->max_seq) return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= e->cfg.vocab) return fail(MCPM_ERR_ARG, "prefill token out of range");
  if (n == 0) return MCPM_OK;
  int rc = ensure_prefill(e, std::min(n, prefill_chunk()));
  if (rc) return rc;
  for (int i = 0; i < n && !rc; i += prefill_chunk())
    rc = prefill_pass(e, tokens + i, std::min(prefill_chunk(), n - i), pos0 + i);
  if (rc) return rc;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  return MCPM_OK;
}

int mcpm_engine_set_prefill(mcpm_engine* e, int enable) {
  if (!e) return fail(MCPM_ERR_ARG, "mcpm_engine_set_prefill: null engine");
  e->use_prefill = enable != 0;
  return MCPM_OK;
}

int mcpm_engine_uses_prefill(const mcpm_engine* e) { return e && e->use_prefill ? 1 : 0; }

int mcpm_engine_read_kv(mcpm_engine* e, int layer, int pos0, int n, float* k, float* v) {
  if (!e || layer < 0 || layer >= e->cfg.n_layers || pos0 < 0 || n < 0)
    return fail(MCPM_ERR_ARG, "mcpm_engine_read_kv: bad argument");
  if (!e->kc || pos0 + n > e->max_seq) return fail(MCPM_ERR_CONTEXT, "mcpm_engine_read_kv: rows outside the cache");
  const size_t kvd = static_cast<size_t>(e->cfg.n_kv_heads) * e->cfg.head_dim;
  const size_t off = (static_cast<size_t>(layer) * e->max_seq + pos0) * kvd, bytes = n * kvd * sizeof(float);
  if (k) MCPM_HIP(hipMemcpyAsync(k, e->kc + off, bytes, hipMemcpyDeviceToHost, e->ctx->stream));
  if (v) MCPM_HIP(hipMemcpyAsync(v, e->vc + off, bytes, hipMemcpyDeviceToHost, e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  return MCPM_OK;
}

int mcpm_engine_load_gguf(mcpm_ctx* ctx, const char* path, mcpm_engine** out) {
  if (!ctx || !path || !out) return fail(MCPM_ERR_ARG, "mcpm_engine_load_gguf: null argument");
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(MCPM_ERR_IO, std::string("Failed to open GGUF file: ") + path);
  struct stat sb;
  if (fstat(fd, &sb) != 0 || sb.st_size <= 0) {
    close(fd);
    return fail(MCPM_ERR_IO, std::string("Cannot stat GGUF file: ") + path);
  }
  void* m = mmap(nullptr, static_cast<size_t>(sb.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return fail(MCPM_ERR_IO, std::string("Cannot map GGUF file: ") + path);
  const int rc = load_from_image(ctx, static_cast<const uint8_t*>(m), static_cast<size_t>(sb.st_size), out);
  munmap(m, static_cast<size_t>(sb.st_size));
  return rc;
}

int mcpm_engine_load_gguf_memory(mcpm_ctx* ctx, const void* data, size_t bytes, mcpm_engine** out) {
  if (!ctx || !data || !out) return fail(MCPM_ERR_ARG, "mcpm_engine_load_gguf_memory: null argument");
  return load_from_image(ctx, static_cast<const uint8_t*>(data), bytes, out);
}

void mcpm_engine_free(mcpm_engine* e) { free_engine(e); }

int mcpm_engine_config(const mcpm_engine* e, mcpm_model_config* out) {
  if (!e || !out) return fail(MCPM_ERR_ARG, "mcpm_engine_config: null argument");
  *out = e->cfg;
  return MCPM_OK;
}

int64_t mcpm_engine_weight_bytes_per_token(const mcpm_engine* e) { return e ? e->weight_bytes : 0; }

int mcpm_engine_init_kv_cache(mcpm_engine* e, int max_seq_len) {
  if (!e || max_seq_len <= 0) return fail(MCPM_ERR_ARG, "mcpm_engine_init_kv_cache: bad argument");
  const mcpm_model_config& c = e->cfg;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  drop_graph(e);
  for (void** p : {reinterpret_cast<void**>(&e->kc), reinterpret_cast<void**>(&e->vc),
                   reinterpret_cast<void**>(&e->rope), reinterpret_cast<void**>(&e->attn_part)}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  e->max_seq = 0;
  const size_t kvd = static_cast<size_t>(c.n_kv_heads) * c.head_dim;
  const size_t kv_bytes = static_cast<size_t>(c.n_layers) * max_seq_len * kvd * sizeof(float);
  int rc = alloc_dev(reinterpret_cast<void**>(&e->kc), kv_bytes);
  if (!rc) rc = alloc_dev(reinterpret_cast<void**>(&e->vc), kv_bytes);
  if (rc) return rc;
  // RoPE (cos, sin) table for positions 0..max_seq_len-1 (src/ops/ops.cpp:503-508).
  std::vector<float2> tab(static_cast<size_t>(max_seq_len) * (c.head_dim / 2));
  for (int p = 0; p < max_seq_len; ++p) rope_row(p, c.head_dim, c.rope_base, tab.data() + static_cast<size_t>(p) * (c.head_dim / 2));
  MCPM_HIP(hipMalloc(&e->rope, tab.size() * sizeof(float2)));
  MCPM_HIP(hipMemcpyAsync(e->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice, e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  e->max_chunks = (max_seq_len + ATTN_CHUNK - 1) / ATTN_CHUNK;
  rc = alloc_dev(reinterpret_cast<void**>(&e->attn_part),
                 static_cast<size_t>(c.n_heads) * e->max_chunks * (2 + c.head_dim) * sizeof(float));
  if (rc) return rc;
  e->max_seq = max_seq_len;
  return pd_setup(e);
}

int mcpm_engine_set_graph(mcpm_engine* e, int enable) {
  if (!e) return fail(MCPM_ERR_ARG, "mcpm_engine_set_graph: null engine");
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  e->use_graph = enable != 0;
  drop_graph(e);
  return MCPM_OK;
}

int mcpm_engine_set_persistent(mcpm_engine* e, int mode) {
  if (!e || mode < 0 || mode > 2) return fail(MCPM_ERR_ARG, "mcpm_engine_set_persistent: bad argument");
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  drop_graph(e);
  if (mode == e->pd_mode && (e->pd_ready || !mode || !e->kc)) return MCPM_OK;
  e->pd_mode = mode;
  return pd_setup(e);  // builds the slab (with a KV cache) or releases it
}

int mcpm_engine_uses_persistent(const mcpm_engine* e) { return e && e->pd_ready && e->pd_mode ? 1 : 0; }

int mcpm_engine_persistent_fixed_shape(const mcpm_engine* e) {
  return mcpm_engine_uses_persistent(e) && pd_fixed_shape(e->pd) ? 1 : 0;
}

int mcpm_engine_persistent_xcd_local(const mcpm_engine* e) {
  return mcpm_engine_uses_persistent(e) && e->pd_args.xcd_local ? 1 : 0;
}

int mcpm_engine_set_spin_limit(mcpm_engine* e, unsigned limit) {
  if (!e) return fail(MCPM_ERR_ARG, "mcpm_engine_set_spin_limit: null engine");
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  e->spin_limit = limit;
  e->pd_args.spin_limit = pd_spin_limit(e);
  drop_graph(e);  // captured launches hold the old limit
  return MCPM_OK;
}

int mcpm_engine_forward(mcpm_engine* e, int token, int pos, int max_seq_len, float* logits, int* argmax) {
  if (!e) return fail(MCPM_ERR_ARG, "mcpm_engine_forward: null engine");
  if (!e->kc) return fail(MCPM_ERR_CONTEXT, "mcpm_engine_forward: KV cache not initialised");
  if (pos < 0 || pos >= max_seq_len || pos >= e->max_seq)
    return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  if (token < 0 || token >= e->cfg.vocab) return fail(MCPM_ERR_ARG, "mcpm_engine_forward: token out of range");
  int rc = ensure_out_tokens(e, 1);
  if (!rc) rc = ensure_staging(e, 1);
  if (rc) return rc;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  rc = queue_state(e, 0, token, pos, 0);
  if (!rc) rc = run_token(e, pos);
  if (rc) return rc;
  e->gen_count = 0;
  if (logits)
    MCPM_HIP(hipMemcpyAsync(logits, e->logits, static_cast<size_t>(e->cfg.vocab) * 4, hipMemcpyDeviceToHost,
                            e->ctx->stream));
  if (argmax) MCPM_HIP(hipMemcpyAsync(e->h_st, e->st, sizeof(StepState), hipMemcpyDeviceToHost, e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  if (const int rc2 = check_grid_sync(e)) return rc2;
  if (argmax) *argmax = e->h_st[0].token;
  return MCPM_OK;
}

// The token graph with the argmax at its end (greedy) or without it
// (sampled); each is captured once and kept.  The sampled graph also ends
// with the sampler's passes when its settings need no sort, and is captured
// again when the settings change.
static int set_sample_mode(mcpm_engine* e, bool on) {
  e->sample_mode = on;
  return MCPM_OK;
}

static void set_sampling(mcpm_engine* e, float temperature, float top_p) {
  if (e->smp_T != temperature || e->smp_P != top_p) {
    for (hipGraphExec_t& g : e->graph[1]) {
      if (g) (void)hipGraphExecDestroy(g);
      g = nullptr;
    }
  }
  e->smp_T = temperature;
  e->smp_P = top_p;
  const bool topp = top_p > 0.0f && top_p < 1.0f;
  e->smp_in_graph = !topp || top_p <= sampler_sort_free_top_p();
}

// Draws of std::uniform_real_distribution<float> over std::mt19937(seed)
// (src/sampler.cpp:5-6, 68-69), one per token, to d_draws[step0 ..].
static int upload_draws(mcpm_engine* e, uint32_t seed, int step0, int n) {
  std::mt19937 rng(seed);
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  std::vector<float> h(static_cast<size_t>(n));
  for (float& v : h) v = dist(rng);
  MCPM_HIP(hipMemcpyAsync(e->d_draws + step0, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice,
                          e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  return MCPM_OK;
}

static int ensure_sampler(mcpm_engine* e) {
  if (e->cfg.vocab > sampler_max_n())
    return fail(MCPM_ERR_UNSUPPORTED, "sampled decode: vocabulary larger than the device sampler's 524,288");
  const size_t need = sampler_bytes(e->cfg.vocab);
  if (need <= e->sample_cap) return MCPM_OK;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  if (e->d_sample) (void)hipFree(e->d_sample);
  e->d_sample = nullptr;
  e->sample_cap = 0;
  drop_graph(e);  // the sampler's nodes hold the scratch pointer
  int rc = alloc_dev(&e->d_sample, need);
  if (rc) return rc;
  e->sample_cap = need;
  return MCPM_OK;
}

// The next token from the logits of the step just queued: it becomes the
// next input token and the next entry of the generated list.
// Settings that need the sort run the sampler after the graph (its sort's
// launches are not captured); the others ran it inside the graph.
static int sample_step(mcpm_engine* e) {
  if (e->smp_in_graph) return MCPM_OK;
  MCPM_HIP(launch_sample(e->d_sample, e->sample_cap, e->logits, e->cfg.vocab, e->smp_T, e->smp_P, 0.0f, nullptr,
                         e->st, e->out_tokens, e->ctx->stream, e->d_draws));
  return MCPM_OK;
}

static bool bad_sampling(float temperature, float top_p) { return !(temperature == temperature) || !(top_p == top_p); }

// Tokens at positions pos0 .. pos0+n-1 (the KV rows below pos0 are kept as
// they are), then n_gen tokens: all given tokens but the last in batched
// passes, the last one (whose argmax or draw is the first generated token)
// through the per-token graph.  sampled: Sampler::sample on the device after
// each token with the draws of std::uniform_real_distribution<float> over
// std::mt19937(seed), one per generated token (src/sampler.cpp:5-6, seeded by
// the caller); else the greedy argmax.
static int generate_at(mcpm_engine* e, const int* toks, int n, int pos0, int n_gen, bool sampled, float temperature,
                       float top_p, uint32_t seed, int* out_tokens, const char* fn) {
  if (!e || !toks || !out_tokens || n <= 0 || n_gen <= 0 || pos0 < 0 ||
      (sampled && bad_sampling(temperature, top_p)))
    return fail(MCPM_ERR_ARG, std::string(fn) + ": bad argument");
  if (!e->kc) return fail(MCPM_ERR_CONTEXT, "KV cache not initialised");
  if (static_cast<int64_t>(pos0) + n + n_gen - 1 > e->max_seq)
    return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  for (int i = 0; i < n; ++i)
    if (toks[i] < 0 || toks[i] >= e->cfg.vocab) return fail(MCPM_ERR_ARG, "prompt token out of range");
  int rc = ensure_out_tokens(e, n_gen);
  if (!rc) rc = ensure_staging(e, n);
  if (!rc && sampled) rc = ensure_sampler(e);
  if (!rc) rc = set_sample_mode(e, sampled);
  if (rc) return rc;
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  if (sampled) {
    set_sampling(e, temperature, top_p);
    rc = upload_draws(e, seed, 0, n_gen);
  }
  const int first = (e->use_prefill && n > 1) ? n - 1 : 0;
  if (!rc && first) rc = mcpm_engine_prefill(e, toks, first, pos0);
  for (int i = first; i < n && !rc; ++i) {
    rc = queue_state(e, i, toks[i], pos0 + i, 0);
    if (!rc) rc = run_token(e, pos0 + i);
  }
  if (!rc && sampled) rc = sample_step(e);
  // generated token i runs at position pos0 + n - 1 + i
  for (int i = 1; i < n_gen && !rc; ++i) {
    rc = run_token(e, pos0 + n - 1 + i);
    if (!rc && sampled) rc = sample_step(e);
  }
  const int rc2 = set_sample_mode(e, false);
  if (rc) return rc;
  if (rc2) return rc2;
  e->gen_count = n_gen;
  e->next_pos = pos0 + n + n_gen - 1;
  MCPM_HIP(hipMemcpyAsync(out_tokens, e->out_tokens, n_gen * sizeof(int), hipMemcpyDeviceToHost, e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  return check_grid_sync(e);
}

int mcpm_engine_generate_greedy(mcpm_engine* e, const int* prompt, int n_prompt, int n_gen, int* out_tokens) {
  return generate_at(e, prompt, n_prompt, 0, n_gen, false, 0.0f, 0.0f, 0u, out_tokens, "mcpm_engine_generate_greedy");
}

int mcpm_engine_generate_greedy_at(mcpm_engine* e, const int* tokens, int n, int pos0, int n_gen, int* out_tokens) {
  return generate_at(e, tokens, n, pos0, n_gen, false, 0.0f, 0.0f, 0u, out_tokens, "mcpm_engine_generate_greedy_at");
}

int mcpm_engine_decode_steps(mcpm_engine* e, int n_steps) {
  if (!e || n_steps < 0) return fail(MCPM_ERR_ARG, "mcpm_engine_decode_steps: bad argument");
  if (e->gen_count == 0) return fail(MCPM_ERR_ARG, "mcpm_engine_decode_steps: no generate call to continue");
  if (e->next_pos + n_steps > e->max_seq) return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  if (e->gen_count + n_steps > e->out_cap) {
    // grow the token list, keeping what is there
    std::vector<int> keep(e->gen_count);
    MCPM_HIP(hipMemcpyAsync(keep.data(), e->out_tokens, keep.size() * sizeof(int), hipMemcpyDeviceToHost,
                            e->ctx->stream));
    MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
    int rc = ensure_out_tokens(e, e->gen_count + n_steps);
    if (rc) return rc;
    hipStream_t s = e->ctx->stream;
    MCPM_HIP(hipMemcpyAsync(e->out_tokens, keep.data(), keep.size() * sizeof(int), hipMemcpyHostToDevice, s));
    // the state's capacity field must follow the new array
    StepState st;
    MCPM_HIP(hipMemcpyAsync(&st, e->st, sizeof(st), hipMemcpyDeviceToHost, s));
    MCPM_HIP(hipStreamSynchronize(s));
    st.n_out = e->out_cap;
    MCPM_HIP(hipMemcpyAsync(e->st, &st, sizeof(st), hipMemcpyHostToDevice, s));
    MCPM_HIP(hipStreamSynchronize(s));
  }
  for (int i = 0; i < n_steps; ++i) {
    const int rc = run_token(e, e->next_pos + i);
    if (rc) return rc;
  }
  e->gen_count += n_steps;
  e->next_pos += n_steps;
  return MCPM_OK;
}

int mcpm_engine_generate_sampled(mcpm_engine* e, const int* prompt, int n_prompt, int n_gen, float temperature,
                                 float top_p, uint32_t seed, int* out_tokens) {
  return generate_at(e, prompt, n_prompt, 0, n_gen, true, temperature, top_p, seed, out_tokens,
                     "mcpm_engine_generate_sampled");
}

int mcpm_engine_generate_sampled_at(mcpm_engine* e, const int* tokens, int n, int pos0, int n_gen, float temperature,
                                    float top_p, uint32_t seed, int* out_tokens) {
  return generate_at(e, tokens, n, pos0, n_gen, true, temperature, top_p, seed, out_tokens,
                     "mcpm_engine_generate_sampled_at");
}

int mcpm_engine_decode_sampled(mcpm_engine* e, int n_steps, float temperature, float top_p, uint32_t seed) {
  if (!e || n_steps < 0 || bad_sampling(temperature, top_p))
    return fail(MCPM_ERR_ARG, "mcpm_engine_decode_sampled: bad argument");
  if (e->gen_count == 0) return fail(MCPM_ERR_ARG, "mcpm_engine_decode_sampled: no generate call to continue");
  if (e->next_pos + n_steps > e->max_seq) return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  if (e->gen_count + n_steps > e->out_cap) return fail(MCPM_ERR_ARG, "mcpm_engine_decode_sampled: token list full");
  int rc = ensure_sampler(e);
  if (!rc) rc = set_sample_mode(e, true);
  if (rc) return rc;
  set_sampling(e, temperature, top_p);
  rc = upload_draws(e, seed, e->gen_count, n_steps);
  for (int i = 0; i < n_steps && !rc; ++i) {
    rc = run_token(e, e->next_pos + i);
    if (!rc) rc = sample_step(e);
  }
  const int rc2 = set_sample_mode(e, false);
  if (rc) return rc;
  if (rc2) return rc2;
  e->gen_count += n_steps;
  e->next_pos += n_steps;
  return MCPM_OK;
}

int mcpm_engine_tokens(mcpm_engine* e, int* out, int n) {
  if (!e || !out || n < 0 || n > e->gen_count) return fail(MCPM_ERR_ARG, "mcpm_engine_tokens: bad argument");
  MCPM_HIP(hipMemcpyAsync(out, e->out_tokens, n * sizeof(int), hipMemcpyDeviceToHost, e->ctx->stream));
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  return check_grid_sync(e);
}

int mcpm_engine_set_kernel_timing(mcpm_engine* e, int kernel_class) {
  if (!e || kernel_class < -1 || kernel_class >= MCPM_KC_COUNT)
    return fail(MCPM_ERR_ARG, "mcpm_engine_set_kernel_timing: bad argument");
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  e->timing_class = kernel_class;
  e->events_used = 0;
  drop_graph(e);
  return MCPM_OK;
}

int mcpm_engine_kernel_time(mcpm_engine* e, double* total_ms, int64_t* launches) {
  if (!e || !total_ms || !launches) return fail(MCPM_ERR_ARG, "mcpm_engine_kernel_time: null argument");
  MCPM_HIP(hipStreamSynchronize(e->ctx->stream));
  double t = 0.0;
  for (size_t i = 0; i < e->events_used; ++i) {
    float ms = 0.0f;
    MCPM_HIP(hipEventElapsedTime(&ms, e->events[i].a, e->events[i].b));
    t += ms;
  }
  *total_ms = t;
  *launches = static_cast<int64_t>(e->events_used);
  return MCPM_OK;
}

int64_t mcpm_engine_kernel_bytes(const mcpm_engine* e, int kc) {
  if (!e) return 0;
  const mcpm_model_config& c = e->cfg;
  const int64_t qd = static_cast<int64_t>(c.n_heads) * c.head_dim, kvd = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
  const Layer& L = e->L[0];
  switch (kc) {
    case MCPM_KC_QKV:
      return static_cast<int64_t>(L.wq.bytes + L.wk.bytes + L.wv.bytes) + 8 * c.dim + 4 * (qd + 2 * kvd);
    case MCPM_KC_OPROJ:
      return static_cast<int64_t>(L.wo.bytes) + 4 * qd + 8 * c.dim;
    case MCPM_KC_GATE_UP:
      return static_cast<int64_t>(L.wg.bytes + L.wu.bytes) + 8 * c.dim + 4 * static_cast<int64_t>(c.ffn);
    case MCPM_KC_DOWN:
      return static_cast<int64_t>(L.wd.bytes) + 4 * static_cast<int64_t>(c.ffn_pad) + 8 * c.dim;
    case MCPM_KC_LM_HEAD:
      return static_cast<int64_t>(e->out_w.bytes) + 8 * c.dim + 4 * static_cast<int64_t>(c.vocab);
    case MCPM_KC_ATTN:
      // K and V rows of the current context, the query and the output
      return 2 * static_cast<int64_t>(e->next_pos + 1) * kvd * 4 + 8 * qd;
    case MCPM_KC_LAYERS: {
      // every layer's weights and norm gains, one embedding row, and the K
      // and V rows of the current context
      int64_t b = static_cast<int64_t>(e->embd.bytes / c.vocab);
      for (const Layer& y : e->L)
        b += static_cast<int64_t>(y.wq.bytes + y.wk.bytes + y.wv.bytes + y.wo.bytes + y.wg.bytes + y.wu.bytes +
                                  y.wd.bytes) +
             8 * static_cast<int64_t>(c.dim);
      return b + 2 * static_cast<int64_t>(e->next_pos + 1) * kvd * 4 * c.n_layers;
    }
    default:
      return 0;
  }
}

}  // extern "C"
