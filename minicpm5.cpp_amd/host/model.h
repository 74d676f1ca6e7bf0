// model.h -- MiniCPM5Engine (include/model.h:37-45) served by the HIP engine:
// the weights and the KV cache live in HBM, the per-token forward runs as one
// graph replay, and forward() returns the logits in host memory like the
// reference.  generate_greedy() is the device-side loop for callers that need
// only token ids (no logits copy per token).
#pragma once

#include <string>
#include <vector>

#include "mcpm_hip.h"

class MiniCPM5Engine {
public:
    MiniCPM5Engine();
    ~MiniCPM5Engine();
    MiniCPM5Engine(const MiniCPM5Engine&) = delete;
    MiniCPM5Engine& operator=(const MiniCPM5Engine&) = delete;

    void init_kv_cache(int max_seq_len);
    bool load_model(const std::string& gguf_path, bool verbose = false);
    // Logits of the token at position pos; the reference stays valid until
    // the next call.  Past the KV capacity it warns and returns the previous
    // logits (the reference's execute_attention warns and continues).
    const std::vector<float>& forward(int token_id, int pos, int max_seq_len);

    // Feeds prompt at positions 0.., then returns n_gen greedy tokens (all
    // prompt tokens but the last go through prefill()).
    std::vector<int> generate_greedy(const std::vector<int>& prompt, int n_gen);
    // The same loop with Sampler::sample (src/sampler.cpp:8-73) on the device
    // after each token: temperature, top-p, draws from std::mt19937(seed).
    std::vector<int> generate_sampled(const std::vector<int>& prompt, int n_gen, float temperature, float top_p,
                                      uint32_t seed);
    // The same two loops continuing a cached context: tokens go at positions
    // pos0.., the KV rows below pos0 are kept (a previous turn's).
    std::vector<int> generate_greedy_at(const std::vector<int>& tokens, int pos0, int n_gen);
    std::vector<int> generate_sampled_at(const std::vector<int>& tokens, int pos0, int n_gen, float temperature,
                                         float top_p, uint32_t seed);
    // Fills the KV cache for tokens at positions pos0.. in batched passes
    // (MFMA GEMMs), exactly as forward() per token would, without logits.  A
    // chat driver keeps the cache across turns and prefills only the new
    // tokens (pos0 = tokens already cached) instead of re-running the history.
    void prefill(const std::vector<int>& tokens, int pos0);
    // A synthetic model image (seeded random weights, the benchmark's shapes).
    bool load_synthetic(const mcpm_model_config& cfg, uint64_t seed, int mix, bool verbose = false);
    const mcpm_model_config& config() const { return cfg_; }

private:
    bool finish_load(int rc, bool verbose);

    mcpm_ctx* ctx_ = nullptr;
    mcpm_engine* engine_ = nullptr;
    mcpm_model_config cfg_{};
    int kv_capacity_ = 0;
    std::vector<float> logits_;
};
