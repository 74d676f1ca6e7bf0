// model_hip.cpp -- MiniCPM5Engine (include/model.h:37-45) over the C ABI.
#include "model.h"

#include <cstdio>
#include <stdexcept>
#include <string>

namespace {

void check(int rc, const char* what) {
    if (rc < 0) throw std::runtime_error(std::string(what) + ": " + mcpm_last_error());
}

}  // namespace

MiniCPM5Engine::MiniCPM5Engine() { check(mcpm_init(0, &ctx_), "mcpm_init"); }

MiniCPM5Engine::~MiniCPM5Engine() {
    if (engine_) mcpm_engine_free(engine_);
    if (ctx_) mcpm_destroy(ctx_);
}

bool MiniCPM5Engine::finish_load(int rc, bool verbose) {
    if (rc < 0) {
        std::fprintf(stderr, "[ERROR] load_model: %s\n", mcpm_last_error());
        engine_ = nullptr;
        return false;
    }
    check(mcpm_engine_config(engine_, &cfg_), "mcpm_engine_config");
    logits_.assign(static_cast<size_t>(cfg_.vocab), 0.0f);
    kv_capacity_ = 0;
    if (verbose) {
        std::printf("[INFO] model: %d layers, hidden %d, %d/%d heads of %d, ffn %d, vocab %d, %.3f GB per token\n",
                    cfg_.n_layers, cfg_.dim, cfg_.n_heads, cfg_.n_kv_heads, cfg_.head_dim, cfg_.ffn, cfg_.vocab,
                    mcpm_engine_weight_bytes_per_token(engine_) / 1e9);
    }
    return true;
}

bool MiniCPM5Engine::load_model(const std::string& gguf_path, bool verbose) {
    if (engine_) mcpm_engine_free(engine_);
    engine_ = nullptr;
    return finish_load(mcpm_engine_load_gguf(ctx_, gguf_path.c_str(), &engine_), verbose);
}

bool MiniCPM5Engine::load_synthetic(const mcpm_model_config& cfg, uint64_t seed, int mix, bool verbose) {
    void* image = nullptr;
    size_t bytes = 0;
    int rc = mcpm_synth_gguf(&cfg, seed, mix, nullptr, &image, &bytes);
    if (rc < 0) {
        std::fprintf(stderr, "[ERROR] synthetic model: %s\n", mcpm_last_error());
        return false;
    }
    if (engine_) mcpm_engine_free(engine_);
    engine_ = nullptr;
    rc = mcpm_engine_load_gguf_memory(ctx_, image, bytes, &engine_);
    mcpm_free_host(image);
    return finish_load(rc, verbose);
}

void MiniCPM5Engine::init_kv_cache(int max_seq_len) {
    if (!engine_) throw std::runtime_error("init_kv_cache: no model loaded");
    check(mcpm_engine_init_kv_cache(engine_, max_seq_len), "mcpm_engine_init_kv_cache");
    kv_capacity_ = max_seq_len;
}

const std::vector<float>& MiniCPM5Engine::forward(int token_id, int pos, int max_seq_len) {
    if (!engine_) throw std::runtime_error("forward: no model loaded");
    const int rc = mcpm_engine_forward(engine_, token_id, pos, max_seq_len, logits_.data(), nullptr);
    if (rc == MCPM_ERR_CONTEXT) {
        std::fprintf(stderr, "[WARNING] Maximum context exceeded (pos >= max_seq_len).\n");
        return logits_;
    }
    check(rc, "mcpm_engine_forward");
    return logits_;
}

void MiniCPM5Engine::prefill(const std::vector<int>& tokens, int pos0) {
    if (!engine_) throw std::runtime_error("prefill: no model loaded");
    check(mcpm_engine_prefill(engine_, tokens.data(), static_cast<int>(tokens.size()), pos0), "mcpm_engine_prefill");
}

std::vector<int> MiniCPM5Engine::generate_sampled(const std::vector<int>& prompt, int n_gen, float temperature,
                                                 float top_p, uint32_t seed) {
    if (!engine_) throw std::runtime_error("generate_sampled: no model loaded");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_sampled(engine_, prompt.data(), static_cast<int>(prompt.size()), n_gen, temperature,
                                       top_p, seed, out.data()),
          "mcpm_engine_generate_sampled");
    return out;
}

std::vector<int> MiniCPM5Engine::generate_greedy(const std::vector<int>& prompt, int n_gen) {
    if (!engine_) throw std::runtime_error("generate_greedy: no model loaded");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_greedy(engine_, prompt.data(), static_cast<int>(prompt.size()), n_gen, out.data()),
          "mcpm_engine_generate_greedy");
    return out;
}

std::vector<int> MiniCPM5Engine::generate_greedy_at(const std::vector<int>& tokens, int pos0, int n_gen) {
    if (!engine_) throw std::runtime_error("generate_greedy_at: no model loaded");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_greedy_at(engine_, tokens.data(), static_cast<int>(tokens.size()), pos0, n_gen,
                                         out.data()),
          "mcpm_engine_generate_greedy_at");
    return out;
}

std::vector<int> MiniCPM5Engine::generate_sampled_at(const std::vector<int>& tokens, int pos0, int n_gen,
                                                     float temperature, float top_p, uint32_t seed) {
    if (!engine_) throw std::runtime_error("generate_sampled_at: no model loaded");
    std::vector<int> out(static_cast<size_t>(n_gen > 0 ? n_gen : 0));
    check(mcpm_engine_generate_sampled_at(engine_, tokens.data(), static_cast<int>(tokens.size()), pos0, n_gen,
                                          temperature, top_p, seed, out.data()),
          "mcpm_engine_generate_sampled_at");
    return out;
}
