// mcpm_decode -- greedy decode through MiniCPM5Engine (host/model.h), the way
// the reference's driver calls forward() (src/chat_session.cpp:154-186):
// every prompt token at positions 0.., then the argmax of each step's logits
// fed back.  --device-loop runs the same decode with the argmax on the GPU
// (no logits copy per token); --prefill sends all prompt tokens but the last
// through the batched prefill before the per-token loop; --sample T,P,SEED
// samples each token on the GPU (temperature T, top-p P, mt19937 seeded with
// SEED) in the device loop.  --turns N1,N2,... runs a multi-turn exchange
// through KVSession (host/kv_session.h): turn 0 sends the prompt, turn i
// appends the previous response and Ni new random ids, and each turn
// generates --tokens tokens, keeping the KV rows of the conversation so far;
// --no-reuse forgets them before every turn (the reference's behaviour, the
// same tokens).
//
//   mcpm_decode (--gguf FILE | --synth SEED [--layers N] [--vocab N])
//               [--prompt N | --prompt-ids ID,ID,...] [--tokens N] [--device-loop] [--prefill]
//               [--sample T,P,SEED] [--turns N1,N2,... [--no-reuse]] [--verbose]
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "kv_session.h"
#include "model.h"

static void usage() {
    std::fprintf(stderr,
                 "usage: mcpm_decode (--gguf FILE | --synth SEED [--layers N] [--vocab N])\n"
                 "                   [--prompt N | --prompt-ids ID,ID,...] [--tokens N] [--device-loop] [--prefill]\n"
                 "                   [--sample T,P,SEED] [--turns N1,N2,... [--no-reuse]] [--verbose]\n");
}

int main(int argc, char** argv) {
    std::string gguf;
    long long synth_seed = -1;
    int layers = 40, vocab = 130560, n_prompt = 32, n_tokens = 64;
    bool device_loop = false, verbose = false, use_prefill = false, sample = false, reuse = true;
    std::vector<int> turns;
    float temperature = 1.0f, top_p = 1.0f;
    unsigned sample_seed = 0;
    std::vector<int> prompt_ids;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) {
                usage();
                std::exit(2);
            }
            return argv[++i];
        };
        if (a == "--gguf") gguf = next();
        else if (a == "--synth") synth_seed = std::atoll(next());
        else if (a == "--layers") layers = std::atoi(next());
        else if (a == "--vocab") vocab = std::atoi(next());
        else if (a == "--prompt") n_prompt = std::atoi(next());
        else if (a == "--prompt-ids") {
            for (const char* p = next(); *p;) {
                char* end = nullptr;
                prompt_ids.push_back(static_cast<int>(std::strtol(p, &end, 10)));
                if (end == p) {
                    usage();
                    return 2;
                }
                p = (*end == ',') ? end + 1 : end;
            }
            n_prompt = static_cast<int>(prompt_ids.size());
        }
        else if (a == "--tokens") n_tokens = std::atoi(next());
        else if (a == "--device-loop") device_loop = true;
        else if (a == "--prefill") use_prefill = true;
        else if (a == "--sample") {
            if (std::sscanf(next(), "%f,%f,%u", &temperature, &top_p, &sample_seed) != 3) {
                usage();
                return 2;
            }
            sample = device_loop = true;
        }
        else if (a == "--turns") {
            for (const char* p = next(); *p;) {
                char* end = nullptr;
                const long v = std::strtol(p, &end, 10);
                if (end == p || v < 1) {
                    usage();
                    return 2;
                }
                turns.push_back(static_cast<int>(v));
                p = (*end == ',') ? end + 1 : end;
            }
        }
        else if (a == "--no-reuse") reuse = false;
        else if (a == "--verbose") verbose = true;
        else {
            usage();
            return a == "--help" || a == "-h" ? 0 : 2;
        }
    }
    if (gguf.empty() == (synth_seed < 0) || n_prompt < 1 || n_tokens < 1 || layers < 1 || vocab < 256) {
        usage();
        return 2;
    }

    // The reference CLI's order (src/main.cpp:107-111): the KV cache first,
    // then the model.
    int max_seq = n_prompt + n_tokens;
    for (int t : turns) max_seq += t + n_tokens;
    MiniCPM5Engine engine;
    engine.init_kv_cache(max_seq);
    bool ok;
    if (!gguf.empty()) {
        ok = engine.load_model(gguf, verbose);
    } else {
        // the 2.4B shape: hidden 2304, 32/8 heads of 64, FFN 5760, tied Q6_K head
        mcpm_model_config c{};
        c.n_layers = layers;
        c.dim = 2304;
        c.n_heads = 32;
        c.n_kv_heads = 8;
        c.head_dim = 64;
        c.ffn = 5760;
        c.ffn_pad = 5888;
        c.vocab = vocab;
        c.rope_base = 10000.0f;
        c.eps = 1e-6f;
        c.tied_embeddings = 1;
        ok = mcpm_host::load_synthetic(engine, c, static_cast<uint64_t>(synth_seed), 0, verbose);
    }
    if (!ok) return 1;
    const mcpm_model_config cfg = mcpm_host::config(engine);

    std::vector<int> prompt = prompt_ids;
    if (prompt.empty()) {
        std::mt19937 gen(1234);
        std::uniform_int_distribution<int> pick(0, cfg.vocab - 1);
        prompt.resize(static_cast<size_t>(n_prompt));
        for (int& t : prompt) t = pick(gen);
    }
    for (int t : prompt) {
        if (t < 0 || t >= cfg.vocab) {
            std::fprintf(stderr, "prompt id %d outside [0, %d)\n", t, cfg.vocab);
            return 2;
        }
    }

    if (!turns.empty()) {
        // turn 0: the prompt; turn i: the previous response and turns[i-1] new ids
        KVSession session(engine, max_seq);
        SessionSampling sp;
        sp.greedy = !sample;
        sp.temperature = temperature;
        sp.top_p = top_p;
        sp.seed = sample_seed;
        std::mt19937 gen(4321);
        std::uniform_int_distribution<int> pick(0, cfg.vocab - 1);
        std::vector<int> conversation = prompt;
        for (size_t t = 0; t <= turns.size(); ++t) {
            if (t > 0)
                for (int k = 0; k < turns[t - 1]; ++k) conversation.push_back(pick(gen));
            if (!reuse) session.clear();
            const auto ts = std::chrono::steady_clock::now();
            const std::vector<int> resp = session.generate_response(conversation, n_tokens, {}, sp);
            const double ms = std::chrono::duration<double>(std::chrono::steady_clock::now() - ts).count() * 1e3;
            std::printf("turn %zu: conversation %zu, reused %d, processed %d, %.1f ms, tokens:", t,
                        conversation.size(), session.reused_tokens(), session.processed_tokens(), ms);
            for (int tok : resp) std::printf(" %d", tok);
            std::printf("\n");
            conversation.insert(conversation.end(), resp.begin(), resp.end());
        }
        return 0;
    }

    std::vector<int> out;
    const auto t0 = std::chrono::steady_clock::now();
    double decode_s = 0.0;
    if (device_loop) {
        out = sample ? mcpm_host::generate_sampled(engine, prompt, n_tokens, temperature, top_p, sample_seed)
                     : mcpm_host::generate_greedy(engine, prompt, n_tokens);
        decode_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    } else {
        auto argmax = [](const std::vector<float>& v) {
            size_t b = 0;
            for (size_t i = 1; i < v.size(); ++i)
                if (v[i] > v[b]) b = i;
            return static_cast<int>(b);
        };
        int pos = 0, next = 0;
        if (use_prefill && prompt.size() > 1) {
            mcpm_host::prefill(engine, std::vector<int>(prompt.begin(), prompt.end() - 1), 0);
            pos = static_cast<int>(prompt.size()) - 1;
        }
        for (size_t i = static_cast<size_t>(pos); i < prompt.size(); ++i)
            next = argmax(engine.forward(prompt[i], pos++, max_seq));
        const auto t1 = std::chrono::steady_clock::now();
        out.push_back(next);
        while (static_cast<int>(out.size()) < n_tokens) {
            next = argmax(engine.forward(next, pos++, max_seq));
            out.push_back(next);
        }
        decode_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    }
    std::printf("tokens:");
    for (int t : out) std::printf(" %d", t);
    std::printf("\n");
    std::printf("decode: %d tokens in %.1f ms (%.1f tok/s, %s)\n", n_tokens, decode_s * 1e3,
                (device_loop ? n_tokens : n_tokens - 1) / decode_s,
                device_loop ? "device loop incl. prompt" : "forward() per token");
    return 0;
}
