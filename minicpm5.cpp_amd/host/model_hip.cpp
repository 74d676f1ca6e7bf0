// model_hip.cpp -- MiniCPM5Engine (include/model.h:37-45) over the C ABI.
//
// The class keeps the reference's data members, none of which can hold a
// device handle, so each object's engine lives in a table keyed by the
// object's address.  The object's raw_gguf_buffer_ (the reference keeps the
// whole file there) holds an 8-byte id of its table entry instead: an object
// constructed at the address of a destroyed one has no buffer (or another
// id), so a stale entry left by the destroyed object is recognised and its
// engine released on first use.
#include "model.h"

#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

namespace {

struct EngineState {
    uint64_t id = 0;
    mcpm_ctx* ctx = nullptr;
    mcpm_engine* engine = nullptr;
    mcpm_model_config cfg{};
    int kv_capacity = 0;  // init_kv_cache's, applied at every load
};

std::mutex g_mu;
uint64_t g_next_id = 1;

// Never destroyed: no device call runs during static destruction at exit.
std::unordered_map<const MiniCPM5Engine*, EngineState*>& table() {
    static auto* t = new std::unordered_map<const MiniCPM5Engine*, EngineState*>();
    return *t;
}

void check(int rc, const char* what) {
    if (rc < 0) throw std::runtime_error(std::string(what) + ": " + mcpm_last_error());
}

void drop_engine(EngineState& s) {
    if (s.engine) mcpm_engine_free(s.engine);
    s.engine = nullptr;
    s.cfg = mcpm_model_config{};
}

}  // namespace

struct MiniCPM5EngineAccess {
    static uint64_t id_of(const MiniCPM5Engine& e) {
        uint64_t id = 0;
        if (e.raw_gguf_buffer_ && e.raw_gguf_buffer_->size() == sizeof id)
            std::memcpy(&id, e.raw_gguf_buffer_->data(), sizeof id);
        return id;
    }

    // The object's table entry, created on first use; an entry whose id the
    // object does not hold was left by a destroyed object at this address.
    static EngineState& state(MiniCPM5Engine& e) {
        std::lock_guard<std::mutex> lock(g_mu);
        EngineState*& s = table()[&e];
        if (!s) s = new EngineState();
        if (s->id != 0 && s->id != id_of(e)) {
            drop_engine(*s);
            s->kv_capacity = 0;
            s->id = 0;
        }
        if (s->id == 0) {
            s->id = g_next_id++;
            e.raw_gguf_buffer_ = std::make_unique<std::vector<char>>(sizeof s->id);
            std::memcpy(e.raw_gguf_buffer_->data(), &s->id, sizeof s->id);
        }
        if (!s->ctx) check(mcpm_init(0, &s->ctx), "mcpm_init");
        return *s;
    }

    static bool finish_load(MiniCPM5Engine& e, EngineState& s, int rc, bool verbose) {
        if (rc < 0) {
            std::fprintf(stderr, "[ERROR] load_model: %s\n", mcpm_last_error());
            s.engine = nullptr;
            return false;
        }
        check(mcpm_engine_config(s.engine, &s.cfg), "mcpm_engine_config");
        e.logits_.assign(static_cast<size_t>(s.cfg.vocab), 0.0f);
        if (s.kv_capacity > 0) check(mcpm_engine_init_kv_cache(s.engine, s.kv_capacity), "mcpm_engine_init_kv_cache");
        if (verbose) {
            std::printf("[INFO] model: %d layers, hidden %d, %d/%d heads of %d, ffn %d, vocab %d, %.3f GB per token\n",
                        s.cfg.n_layers, s.cfg.dim, s.cfg.n_heads, s.cfg.n_kv_heads, s.cfg.head_dim, s.cfg.ffn,
                        s.cfg.vocab, mcpm_engine_weight_bytes_per_token(s.engine) / 1e9);
        }
        return true;
    }

    static mcpm_engine* loaded(MiniCPM5Engine& e, const char* what) {
        EngineState& s = state(e);
        if (!s.engine) throw std::runtime_error(std::string(what) + ": no model loaded");
        return s.engine;
    }

    static void release(MiniCPM5Engine& e) {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = table().find(&e);
        if (it == table().end()) return;
        drop_engine(*it->second);
        if (it->second->ctx) mcpm_destroy(it->second->ctx);
        delete it->second;
        table().erase(it);
        e.raw_gguf_buffer_.reset();
        e.logits_.clear();
    }
};

using A = MiniCPM5EngineAccess;

void MiniCPM5Engine::init_kv_cache(int max_seq_len) {
    EngineState& s = A::state(*this);
    s.kv_capacity = max_seq_len;
    if (s.engine) check(mcpm_engine_init_kv_cache(s.engine, max_seq_len), "mcpm_engine_init_kv_cache");
}

bool MiniCPM5Engine::load_model(const std::string& gguf_path, bool verbose) {
    EngineState& s = A::state(*this);
    drop_engine(s);
    return A::finish_load(*this, s, mcpm_engine_load_gguf(s.ctx, gguf_path.c_str(), &s.engine), verbose);
}

const std::vector<float>& MiniCPM5Engine::forward(int token_id, int pos, int max_seq_len) {
    mcpm_engine* eng = A::loaded(*this, "forward");
    const int rc = mcpm_engine_forward(eng, token_id, pos, max_seq_len, logits_.data(), nullptr);
    if (rc == MCPM_ERR_CONTEXT) {
        std::fprintf(stderr, "[WARNING] Maximum context exceeded (pos >= max_seq_len).\n");
        return logits_;
    }
    check(rc, "mcpm_engine_forward");
    return logits_;
}

namespace mcpm_host {

bool load_synthetic(MiniCPM5Engine& engine, const mcpm_model_config& cfg, uint64_t seed, int mix, bool verbose) {
    EngineState& s = A::state(engine);
    void* image = nullptr;
    size_t bytes = 0;
    int rc = mcpm_synth_gguf(&cfg, seed, mix, nullptr, &image, &bytes);
    if (rc < 0) {
        std::fprintf(stderr, "[ERROR] synthetic model: %s\n", mcpm_last_error());
        return false;
    }
    drop_engine(s);
    rc = mcpm_engine_load_gguf_memory(s.ctx, image, bytes, &s.engine);
    mcpm_free_host(image);
    return A::finish_load(engine, s, rc, verbose);
}

mcpm_model_config config(MiniCPM5Engine& engine) { return A::state(engine).cfg; }

void prefill(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0) {
    check(mcpm_engine_prefill(A::loaded(engine, "prefill"), tokens.data(), static_cast<int>(tokens.size()), pos0),
          "mcpm_engine_prefill");
}

std::vector<int> generate_greedy(MiniCPM5Engine& engine, const std::vector<int>& prompt, int n_gen) {
    mcpm_engine* e = A::loaded(engine, "generate_greedy");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_greedy(e, prompt.data(), static_cast<int>(prompt.size()), n_gen, out.data()),
          "mcpm_engine_generate_greedy");
    return out;
}

std::vector<int> generate_sampled(MiniCPM5Engine& engine, const std::vector<int>& prompt, int n_gen,
                                  float temperature, float top_p, uint32_t seed) {
    mcpm_engine* e = A::loaded(engine, "generate_sampled");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_sampled(e, prompt.data(), static_cast<int>(prompt.size()), n_gen, temperature, top_p,
                                       seed, out.data()),
          "mcpm_engine_generate_sampled");
    return out;
}

std::vector<int> generate_greedy_at(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0, int n_gen) {
    mcpm_engine* e = A::loaded(engine, "generate_greedy_at");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_greedy_at(e, tokens.data(), static_cast<int>(tokens.size()), pos0, n_gen, out.data()),
          "mcpm_engine_generate_greedy_at");
    return out;
}

std::vector<int> generate_sampled_at(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0, int n_gen,
                                     float temperature, float top_p, uint32_t seed) {
    mcpm_engine* e = A::loaded(engine, "generate_sampled_at");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_sampled_at(e, tokens.data(), static_cast<int>(tokens.size()), pos0, n_gen, temperature,
                                          top_p, seed, out.data()),
          "mcpm_engine_generate_sampled_at");
    return out;
}

void release(MiniCPM5Engine& engine) { A::release(engine); }

}  // namespace mcpm_host
