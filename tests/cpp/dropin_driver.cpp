// dropin_driver -- MiniCPM5Engine driven in the reference CLI's order
// (src/main.cpp:107-111, then the token loop of src/chat_session.cpp:154-186):
// init_kv_cache, load_model, forward() for every prompt token, then the
// argmax of each step's logits fed back.  It uses only the engine's public
// calls, so it compiles against either model.h: this build's
// (minicpm5.cpp_amd/host/model.h) or the reference's own include/model.h.
// oracle/Makefile links it three ways: this build's header with
// libmcpm_model.so; the reference's header with libmcpm_model.so (the engine
// drop-in); the reference's header and its own src/model.cpp with
// libmcpm_ops.so (the operator drop-in).  All three must print the tokens of
// the native engine.
//
//   dropin_driver GGUF CONTEXT N_GEN ID,ID,... [LOGITS_OUT]
//
// Prints "tokens: t0 t1 ..."; LOGITS_OUT receives the fp32 logits of the
// first generated step.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "model.h"

int main(int argc, char** argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: dropin_driver GGUF CONTEXT N_GEN ID,ID,... [LOGITS_OUT]\n");
        return 2;
    }
    const std::string path = argv[1];
    const int ctx = std::atoi(argv[2]);
    const int n_gen = std::atoi(argv[3]);
    std::vector<int> prompt;
    for (const char* p = argv[4]; *p;) {
        char* end = nullptr;
        const long v = std::strtol(p, &end, 10);
        if (end == p || (*end != ',' && *end != '\0')) return 2;
        prompt.push_back(static_cast<int>(v));
        p = *end == ',' ? end + 1 : end;
    }
    if (ctx < 1 || n_gen < 1 || prompt.empty() || static_cast<int>(prompt.size()) + n_gen > ctx + 1) return 2;

    MiniCPM5Engine engine;
    engine.init_kv_cache(ctx);
    if (!engine.load_model(path, false)) {
        std::fprintf(stderr, "load_model failed\n");
        return 1;
    }
    auto argmax = [](const std::vector<float>& v) {
        size_t b = 0;
        for (size_t i = 1; i < v.size(); ++i)
            if (v[i] > v[b]) b = i;
        return static_cast<int>(b);
    };
    int pos = 0, next = 0;
    for (int t : prompt) next = argmax(engine.forward(t, pos++, ctx));
    if (argc > 5) {
        const std::vector<float>& lg = engine.forward(prompt.back(), pos - 1, ctx);  // same position, same logits
        FILE* f = std::fopen(argv[5], "wb");
        if (!f || std::fwrite(lg.data(), sizeof(float), lg.size(), f) != lg.size()) return 1;
        std::fclose(f);
    }
    std::vector<int> out{next};
    while (static_cast<int>(out.size()) < n_gen) {
        next = argmax(engine.forward(next, pos++, ctx));
        out.push_back(next);
    }
    std::printf("tokens:");
    for (int t : out) std::printf(" %d", t);
    std::printf("\n");
    return 0;
}
