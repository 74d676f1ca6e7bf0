// kv_session.cpp -- KVSession over the engine's generate_*_at calls (mcpm_host).
#include "kv_session.h"

#include <algorithm>
#include <stdexcept>
#include <string>

KVSession::KVSession(MiniCPM5Engine& engine, int context_size) : engine_(engine), context_size_(context_size) {
    if (context_size < 2) throw std::invalid_argument("KVSession: context_size < 2");
    engine_.init_kv_cache(context_size);
}

std::vector<int> KVSession::generate_response(const std::vector<int>& conversation, int max_gen,
                                              const std::unordered_set<int>& stop_ids,
                                              const SessionSampling& sampling) {
    const int n = static_cast<int>(conversation.size());
    if (n == 0 || max_gen < 1) throw std::invalid_argument("KVSession: empty conversation or max_gen < 1");
    if (n >= context_size_)
        throw std::length_error("Context overflow: " + std::to_string(n) + " prompt tokens >= context_size " +
                                std::to_string(context_size_));
    // generated token g (g >= 1) is fed back at position n + g - 1
    const int n_gen = std::min(max_gen, context_size_ - n + 1);
    // the longest cached prefix, leaving at least the last token to run (its
    // logits give the first generated token)
    const size_t lim = std::min(cached_.size(), conversation.size() - 1);
    size_t keep = 0;
    while (keep < lim && cached_[keep] == conversation[keep]) ++keep;
    const std::vector<int> rest(conversation.begin() + static_cast<std::ptrdiff_t>(keep), conversation.end());
    const int pos0 = static_cast<int>(keep);
    std::vector<int> out =
        sampling.greedy ? mcpm_host::generate_greedy_at(engine_, rest, pos0, n_gen)
                        : mcpm_host::generate_sampled_at(engine_, rest, pos0, n_gen, sampling.temperature,
                                                         sampling.top_p, sampling.seed + static_cast<uint32_t>(turns_));
    // rows now valid: the conversation, then every generated token but the last
    cached_.assign(conversation.begin(), conversation.end());
    cached_.insert(cached_.end(), out.begin(), out.end() - 1);
    reused_ = pos0;
    processed_ = n - pos0;
    ++turns_;
    for (size_t i = 0; i < out.size(); ++i) {
        if (stop_ids.count(out[i])) {
            out.resize(i);
            break;
        }
    }
    return out;
}
