// Drives every function of the C++ operator mirror (minicpm5.cpp_amd/host/
// ops.h) on seeded inputs and writes each result to a file, which
// tests/test_gpu_host_wrapper.py compares with the oracle.  Inputs come from
// mcpm_synth_normal and mcpm_quantize_rows (host-side, deterministic), so the
// test regenerates them exactly.
//
//   ops_wrapper_check OUT_FILE
//
// Record format: u32 name length, name, u64 byte count, bytes.
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "mcpm_hip.h"
#include "ops.h"

namespace {

constexpr uint64_t SEED = 99;
constexpr int COLS = 512;

std::vector<float> normal(uint64_t id, size_t n, float mean = 0.0f, float sd = 1.0f) {
    std::vector<float> v(n);
    mcpm_synth_normal(SEED, id, mean, sd, v.data(), n);
    return v;
}

struct Owned {
    std::vector<char> bytes;
    Tensor t;
};

Owned weight(uint64_t id, const char* type, int ggml, int rows, int cols = COLS) {
    Owned o;
    const std::vector<float> w = normal(id, static_cast<size_t>(rows) * cols, 0.0f, 0.02f);
    if (ggml == MCPM_TYPE_F32) {
        o.bytes.assign(reinterpret_cast<const char*>(w.data()), reinterpret_cast<const char*>(w.data() + w.size()));
    } else {
        o.bytes.resize(mcpm_type_row_bytes(ggml, cols) * rows);
        mcpm_quantize_rows(ggml, w.data(), rows, cols, o.bytes.data());
    }
    o.t.name = std::string("w") + std::to_string(id);
    o.t.type_str = type;
    o.t.dims = {static_cast<uint64_t>(cols), static_cast<uint64_t>(rows)};
    o.t.data_ptr = o.bytes.data();
    o.t.size_bytes = o.bytes.size();
    return o;
}

Tensor vec_tensor(const std::vector<float>& v) {
    Tensor t;
    t.name = "gamma";
    t.type_str = "F32";
    t.dims = {v.size()};
    t.data_ptr = reinterpret_cast<const char*>(v.data());
    t.size_bytes = v.size() * 4;
    return t;
}

FILE* out_file = nullptr;

void put(const std::string& name, const void* data, uint64_t n) {
    const uint32_t len = static_cast<uint32_t>(name.size());
    std::fwrite(&len, 4, 1, out_file);
    std::fwrite(name.data(), 1, len, out_file);
    std::fwrite(&n, 8, 1, out_file);
    std::fwrite(data, 1, n, out_file);
}
void put(const std::string& name, const std::vector<float>& v) { put(name, v.data(), v.size() * 4); }

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: ops_wrapper_check OUT_FILE\n");
        return 2;
    }
    out_file = std::fopen(argv[1], "wb");
    if (!out_file) return 1;

    const std::vector<float> x = normal(5, COLS), gamma = normal(6, COLS, 1.0f, 0.1f);
    const std::vector<float> g = normal(7, COLS), u = normal(8, COLS);
    std::vector<float> y;

    const Owned w4 = weight(1, "Q4_K", MCPM_TYPE_Q4_K, 300), w6 = weight(2, "Q6_K", MCPM_TYPE_Q6_K, 300);
    const Owned w8 = weight(3, "Q8_0", MCPM_TYPE_Q8_0, 300), wf = weight(4, "F32", MCPM_TYPE_F32, 40);
    matmul(y, x, w4.t);
    put("matmul_q4k", y);
    matmul(y, x, w6.t);
    put("matmul_q6k", y);
    matmul(y, x, w8.t);
    put("matmul_q8_0", y);
    matmul(y, x, wf.t);
    put("matmul_f32", y);
    Owned bad = weight(1, "Q4_K", MCPM_TYPE_Q4_K, 300);
    bad.t.type_str = "Q5_K";
    matmul(y, x, bad.t);
    put("matmul_unsupported", y);

    std::vector<block_q8_K> xq(COLS / 256);
    quantize_row_q8_K(x.data(), COLS, xq.data());
    put("quantize_row_q8_K", xq.data(), xq.size() * sizeof(block_q8_K));
    matmul_q8k(y, xq.data(), COLS, w4.t);
    put("matmul_q8k_q4k", y);
    matmul_q8k(y, xq.data(), COLS, w6.t);
    put("matmul_q8k_q6k", y);

    const Owned wq = weight(9, "Q4_K", MCPM_TYPE_Q4_K, 256), wk = weight(10, "Q4_K", MCPM_TYPE_Q4_K, 64);
    const Owned wv = weight(11, "Q6_K", MCPM_TYPE_Q6_K, 64);
    std::vector<float> q, k, v;
    matmul_qkv_q8k(q, k, v, xq.data(), COLS, wq.t, wk.t, wv.t);
    put("qkv_q", q);
    put("qkv_k", k);
    put("qkv_v", v);

    const Owned wg = weight(12, "Q4_K", MCPM_TYPE_Q4_K, 300), wu = weight(13, "Q4_K", MCPM_TYPE_Q4_K, 300);
    std::vector<float> gate, up;
    matmul_gate_up_q8k(gate, up, xq.data(), COLS, wg.t, wu.t);
    put("gate", gate);
    put("up", up);

    const Tensor gt = vec_tensor(gamma);
    rmsnorm(y, x, gt);
    put("rmsnorm", y);
    std::vector<block_q8_K> nq(COLS / 256);
    rmsnorm_and_quantize_q8k(nq.data(), x, gt);
    put("rmsnorm_and_quantize_q8k", nq.data(), nq.size() * sizeof(block_q8_K));
    swiglu_and_quantize_q8k(nq.data(), g, u);
    put("swiglu_and_quantize_q8k", nq.data(), nq.size() * sizeof(block_q8_K));

    std::vector<float> rv = normal(14, 4 * 64);
    apply_rope(rv, 17, 2, 64, 10000.0f);
    put("apply_rope", rv);

    const int pos = 70, max_seq = 96, nh = 8, nkv = 2, hd = 64, kvd = nkv * hd;
    KVCacheLayer kv;
    kv.k = normal(18, static_cast<size_t>(max_seq) * kvd);
    kv.v = normal(19, static_cast<size_t>(max_seq) * kvd);
    const std::vector<float> aq = normal(15, nh * hd), kc = normal(16, kvd), vc = normal(17, kvd);
    std::vector<float> att;
    execute_attention(att, aq, kc, vc, kv, pos, max_seq, nh, nkv, hd);
    put("attention", att);
    put("attention_kcache_row", kv.k.data() + static_cast<size_t>(pos) * kvd, kvd * 4);

    const Owned emb = weight(20, "Q6_K", MCPM_TYPE_Q6_K, 50);
    get_embedding(y, emb.t, 5);
    put("embedding", y);

    std::fclose(out_file);
    std::printf("ops_wrapper_check: wrote %s\n", argv[1]);
    return 0;
}
