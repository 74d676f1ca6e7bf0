// kv_session.h -- the turn loop of ChatSession::generate_response
// (src/chat_session.cpp:117-186) at the token level, with the KV cache kept
// across turns.  The reference renders the whole conversation every turn and
// feeds all of its tokens through forward() from position 0 (:154-160).  Here
// each turn's tokens are compared with the tokens whose KV rows are in the
// cache; the rows of the longest shared prefix are kept and only the rest of
// the conversation runs through the model (batched prefill, then the
// per-token graph).  Kept rows are bit-identical to the rows a run from
// position 0 writes, so a turn generates the tokens that run would.
// Tokenizer, chat template and tool calls stay with the caller.
#pragma once

#include <cstdint>
#include <unordered_set>
#include <vector>

#include "model.h"

struct SessionSampling {
    bool greedy = true;
    float temperature = 1.0f;
    float top_p = 0.95f;
    uint32_t seed = 0;  // turn t draws from std::mt19937(seed + t)
};

class KVSession {
public:
    // The engine's KV cache is (re)initialised to context_size positions.
    KVSession(MiniCPM5Engine& engine, int context_size);

    // Up to max_gen tokens after `conversation` (every token of the rendered
    // conversation so far, the new turn included), cut before the first
    // token in stop_ids (which is not returned, as in the reference's loop).
    // Throws std::length_error when the conversation does not fit the context.
    std::vector<int> generate_response(const std::vector<int>& conversation, int max_gen,
                                       const std::unordered_set<int>& stop_ids = {},
                                       const SessionSampling& sampling = SessionSampling{});

    int reused_tokens() const { return reused_; }        // conversation tokens whose rows the last turn kept
    int processed_tokens() const { return processed_; }  // conversation tokens the last turn ran
    int cached_tokens() const { return static_cast<int>(cached_.size()); }
    // Forget the cached rows: the next turn runs its conversation from position 0.
    void clear() { cached_.clear(); }

private:
    MiniCPM5Engine& engine_;
    int context_size_;
    std::vector<int> cached_;  // the token at each position whose KV rows are valid
    int reused_ = 0, processed_ = 0, turns_ = 0;
};
