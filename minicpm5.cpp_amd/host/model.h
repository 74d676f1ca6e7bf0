// model.h -- MiniCPM5Engine (include/model.h) served by the HIP engine.
//
// The class is the reference's, member for member: the same public calls and
// the same private data, so code compiled against the reference's own
// include/model.h (src/main.cpp, src/chat_session.cpp) links against
// libmcpm_model.so in place of src/model.cpp and src/ops/*.cpp with no change
// to its sources or headers, and constructs and destroys the object itself.
// The weights and the KV cache live in HBM, the per-token forward runs as one
// graph replay, and forward() returns the logits in host memory like the
// reference; the private vectors other than logits_ stay empty.
//
// Differences from the reference engine:
//  - the GGUF header is parsed at run time (the reference bakes one file's
//    offsets, src/model.cpp:78-133), so other layer counts and head
//    geometries load too;
//  - init_kv_cache may come before or after load_model (the reference CLI
//    calls it first, src/main.cpp:107-111); the capacity applies at load;
//  - forward() past the KV capacity warns and returns the previous logits;
//  - the reference's class has no destructor, so the device memory of an
//    engine is released by mcpm_host::release(), by a later load into an
//    object at the same address, or at process exit.
//
// Device-side loops and batched prefill for callers that need only token ids
// are free functions in namespace mcpm_host below (no logits copy per token).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "mcpm_hip.h"
#include "ops.h"

// include/model.h:13-31
struct LayerWeights {
    int layer_id;
    Tensor attn_norm;
    Tensor attn_q;
    Tensor attn_k;
    Tensor attn_v;
    Tensor attn_output;
    Tensor ffn_norm;
    Tensor ffn_gate;
    Tensor ffn_up;
    Tensor ffn_down;
};

struct ModelWeights {
    Tensor token_embd;
    Tensor output_norm;
    Tensor output;  // LM head
    std::vector<LayerWeights> layers;
};

// include/model.h:37-69
class MiniCPM5Engine {
public:
    // 42 layer slots, as the reference's constructor sizes them (its
    // MODEL_LAYERS); unused here, where the layer count comes from the file.
    MiniCPM5Engine() { weights_.layers.resize(42); }

    void init_kv_cache(int max_seq_len);
    bool load_model(const std::string& gguf_path, bool verbose = false);
    // Logits of the token at position pos; the reference stays valid until
    // the next call.
    const std::vector<float>& forward(int token_id, int pos, int max_seq_len);

private:
    bool load_gguf_file(const std::string& gguf_path, bool verbose);
    void map_tensors(bool verbose);

    std::unique_ptr<std::vector<char>> raw_gguf_buffer_;
    ModelWeights weights_;
    std::vector<KVCacheLayer> kv_caches_;

    std::vector<float> x_;
    std::vector<float> x_norm_;
    std::vector<float> q_;
    std::vector<float> k_;
    std::vector<float> v_;
    std::vector<float> attn_out_temp_;
    std::vector<float> attn_output_;
    std::vector<float> gate_;
    std::vector<float> up_;
    std::vector<float> ffn_intermediate_;
    std::vector<float> ffn_output_;
    std::vector<float> residual_;
    std::vector<float> logits_;
    std::vector<block_q8_K> x_norm_q8k_;
    std::vector<block_q8_K> ffn_intermediate_q8k_;

    // The one line that is not the reference's: this library's free
    // functions below reach the engine through it.  It changes neither the
    // layout nor any symbol.
    friend struct MiniCPM5EngineAccess;
};

namespace mcpm_host {

// A synthetic model image (seeded random weights; mcpm_synth_gguf's mix).
bool load_synthetic(MiniCPM5Engine& engine, const mcpm_model_config& cfg, uint64_t seed, int mix,
                    bool verbose = false);
// The loaded model's shape (zeros before a load).
mcpm_model_config config(MiniCPM5Engine& engine);
// Feeds prompt at positions 0.., then returns n_gen greedy tokens (all
// prompt tokens but the last go through the batched prefill).
std::vector<int> generate_greedy(MiniCPM5Engine& engine, const std::vector<int>& prompt, int n_gen);
// The same loop with Sampler::sample (src/sampler.cpp:8-73) on the device
// after each token: temperature, top-p, draws from std::mt19937(seed).
std::vector<int> generate_sampled(MiniCPM5Engine& engine, const std::vector<int>& prompt, int n_gen,
                                  float temperature, float top_p, uint32_t seed);
// The same two loops continuing a cached context: tokens go at positions
// pos0.., the KV rows below pos0 are kept (a previous turn's).
std::vector<int> generate_greedy_at(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0, int n_gen);
std::vector<int> generate_sampled_at(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0, int n_gen,
                                     float temperature, float top_p, uint32_t seed);
// Fills the KV cache for tokens at positions pos0.. in batched passes (MFMA
// GEMMs), exactly as forward() per token would, without logits.
void prefill(MiniCPM5Engine& engine, const std::vector<int>& tokens, int pos0);
// Releases the engine's device memory now (a later load_model starts over).
void release(MiniCPM5Engine& engine);

}  // namespace mcpm_host
