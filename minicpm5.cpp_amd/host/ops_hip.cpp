// ops_hip.cpp -- include/ops.h (the reference's operator API) over the C ABI.
// Host vectors are staged through per-thread device buffers; each call
// synchronizes before it returns, so outputs are filled on return as with the
// reference's CPU kernels.
#include "ops.h"

#include "mcpm_hip.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>

namespace {

struct ThreadState {
    mcpm_ctx* ctx = nullptr;
    std::unordered_map<const void*, mcpm_tensor*> tensors;  // by host data pointer
    std::unordered_map<const void*, void*> f32;             // F32 weight vectors
    void* buf[8] = {};
    size_t cap[8] = {};

    ~ThreadState() {
        for (auto& t : tensors) mcpm_tensor_free(t.second);
        if (ctx) {
            for (auto& w : f32) mcpm_device_free(ctx, w.second);
            for (int i = 0; i < 8; ++i)
                if (buf[i]) mcpm_device_free(ctx, buf[i]);
            mcpm_destroy(ctx);
        }
    }
};

thread_local ThreadState ts;

void check(int rc, const char* what) {
    if (rc < 0) throw std::runtime_error(std::string(what) + ": " + mcpm_last_error());
}

mcpm_ctx* ctx() {
    if (!ts.ctx) check(mcpm_init(0, &ts.ctx), "mcpm_init");
    return ts.ctx;
}

// Device scratch slot i with room for `bytes` (grow-only).
void* scratch(int i, size_t bytes) {
    if (bytes == 0) bytes = 4;
    if (ts.cap[i] < bytes) {
        if (ts.buf[i]) mcpm_device_free(ctx(), ts.buf[i]);
        ts.buf[i] = nullptr;
        ts.cap[i] = 0;
        check(mcpm_device_alloc(ctx(), bytes, &ts.buf[i]), "mcpm_device_alloc");
        ts.cap[i] = bytes;
    }
    return ts.buf[i];
}

void* upload(int slot, const void* host, size_t bytes) {
    void* d = scratch(slot, bytes);
    if (bytes) check(mcpm_copy_to_device(ctx(), d, host, bytes), "mcpm_copy_to_device");
    return d;
}

void download(void* host, const void* dev, size_t bytes) {
    check(mcpm_sync(ctx()), "mcpm_sync");
    if (bytes) check(mcpm_copy_to_host(ctx(), host, dev, bytes), "mcpm_copy_to_host");
}

int ggml_type(const std::string& s) {
    if (s == "Q4_K") return MCPM_TYPE_Q4_K;
    if (s == "Q6_K") return MCPM_TYPE_Q6_K;
    if (s == "Q8_0") return MCPM_TYPE_Q8_0;
    if (s == "F32") return MCPM_TYPE_F32;
    return -1;
}

int64_t cols_of(const Tensor& t) { return t.dims.empty() ? 0 : static_cast<int64_t>(t.dims[0]); }
int64_t rows_of(const Tensor& t) { return t.dims.size() > 1 ? static_cast<int64_t>(t.dims[1]) : 1; }

// The tensor in HBM (uploaded on first use); nullptr for types the engine
// does not hold.
const mcpm_tensor* device_tensor(const Tensor& t) {
    auto it = ts.tensors.find(t.data_ptr);
    if (it != ts.tensors.end()) return it->second;
    const int type = ggml_type(t.type_str);
    if (type < 0 || !t.data_ptr) return nullptr;
    mcpm_tensor* d = nullptr;
    check(mcpm_tensor_upload(ctx(), t.data_ptr, t.size_bytes, type, cols_of(t), rows_of(t), &d),
          ("mcpm_tensor_upload " + t.name).c_str());
    ts.tensors.emplace(t.data_ptr, d);
    return d;
}

// An F32 vector tensor (norm weights) in HBM.
const float* device_f32(const Tensor& t, size_t n) {
    auto it = ts.f32.find(t.data_ptr);
    if (it != ts.f32.end()) return static_cast<const float*>(it->second);
    void* d = nullptr;
    check(mcpm_device_alloc(ctx(), n * sizeof(float), &d), "mcpm_device_alloc");
    check(mcpm_copy_to_device(ctx(), d, t.data_ptr, n * sizeof(float)), "mcpm_copy_to_device");
    ts.f32.emplace(t.data_ptr, d);
    return static_cast<const float*>(d);
}

void warn_once(const std::string& key, const char* msg) {
    static thread_local std::unordered_map<std::string, bool> seen;
    if (!seen[key]) {
        seen[key] = true;
        std::fprintf(stderr, "[WARNING] %s (%s)\n", msg, key.c_str());
    }
}

template <class T>
void fit(std::vector<T>& v, size_t n) {
    if (v.size() != n) v.resize(n);
}

}  // namespace


float silu(float x) { return x / (1.0f + std::exp(-x)); }

void rmsnorm(std::vector<float>& out, const std::vector<float>& x, const Tensor& w, float eps) {
    const size_t n = x.size();
    fit(out, n);
    float* dx = static_cast<float*>(upload(0, x.data(), n * 4));
    float* dout = static_cast<float*>(scratch(1, n * 4));
    check(mcpm_rmsnorm(ctx(), dout, dx, device_f32(w, n), static_cast<int>(n), eps), "mcpm_rmsnorm");
    download(out.data(), dout, n * 4);
}

void rmsnorm_and_quantize_q8k(block_q8_K* out, const std::vector<float>& x, const Tensor& w, float eps) {
    const size_t n = x.size(), nb = n / 256;
    float* dx = static_cast<float*>(upload(0, x.data(), n * 4));
    void* dq = scratch(1, nb * sizeof(block_q8_K));
    check(mcpm_rmsnorm_and_quantize_q8k(ctx(), dq, dx, device_f32(w, n), static_cast<int>(n), eps),
          "mcpm_rmsnorm_and_quantize_q8k");
    download(out, dq, nb * sizeof(block_q8_K));
}

void swiglu_and_quantize_q8k(block_q8_K* out, const std::vector<float>& gate, const std::vector<float>& up) {
    const size_t n = gate.size(), nb = n / 256;
    float* dg = static_cast<float*>(upload(0, gate.data(), n * 4));
    float* du = static_cast<float*>(upload(1, up.data(), n * 4));
    void* dq = scratch(2, nb * sizeof(block_q8_K));
    check(mcpm_swiglu_and_quantize_q8k(ctx(), dq, dg, du, static_cast<int>(n)), "mcpm_swiglu_and_quantize_q8k");
    download(out, dq, nb * sizeof(block_q8_K));
}

void apply_rope(std::vector<float>& vec, int pos, int head_idx, int head_dim, float rope_base) {
    float* head = vec.data() + static_cast<size_t>(head_idx) * head_dim;
    float* d = static_cast<float*>(upload(0, head, static_cast<size_t>(head_dim) * 4));
    check(mcpm_apply_rope(ctx(), d, pos, 1, head_dim, rope_base), "mcpm_apply_rope");
    download(head, d, static_cast<size_t>(head_dim) * 4);
}

void matmul(std::vector<float>& output, const std::vector<float>& input, const Tensor& tensor) {
    const size_t rows = static_cast<size_t>(rows_of(tensor));
    fit(output, rows);
    const mcpm_tensor* w = device_tensor(tensor);
    if (!w) {
        warn_once(tensor.type_str, "matmul: tensor type not implemented");
        for (float& o : output) o = 0.001f;
        return;
    }
    float* dx = static_cast<float*>(upload(0, input.data(), input.size() * 4));
    float* dout = static_cast<float*>(scratch(1, rows * 4));
    const int rc = mcpm_matmul(ctx(), w, dx, dout);
    if (rc == MCPM_ERR_UNSUPPORTED) warn_once(tensor.type_str, "matmul: tensor type not implemented");
    else check(rc, "mcpm_matmul");
    download(output.data(), dout, rows * 4);
}

void quantize_row_q8_K(const float* x, int n, block_q8_K* y) {
    const size_t nb = static_cast<size_t>(n) / 256;
    float* dx = static_cast<float*>(upload(0, x, static_cast<size_t>(n) * 4));
    void* dq = scratch(1, nb * sizeof(block_q8_K));
    check(mcpm_quantize_row_q8_K(ctx(), dx, n, dq), "mcpm_quantize_row_q8_K");
    download(y, dq, nb * sizeof(block_q8_K));
}

void matmul_q8k(std::vector<float>& output, const block_q8_K* input_q8k, int num_cols, const Tensor& tensor) {
    const size_t rows = static_cast<size_t>(rows_of(tensor));
    fit(output, rows);
    const mcpm_tensor* w = device_tensor(tensor);
    if (!w) {
        warn_once(tensor.type_str, "matmul_q8k: tensor type not supported");
        for (float& o : output) o = 0.0f;
        return;
    }
    void* dq = upload(0, input_q8k, static_cast<size_t>(num_cols / 256) * sizeof(block_q8_K));
    float* dout = static_cast<float*>(scratch(1, rows * 4));
    const int rc = mcpm_matmul_q8k(ctx(), w, dq, num_cols, dout);
    if (rc == MCPM_ERR_UNSUPPORTED) warn_once(tensor.type_str, "matmul_q8k: tensor type not supported");
    else check(rc, "mcpm_matmul_q8k");
    download(output.data(), dout, rows * 4);
}

void matmul_qkv_q8k(std::vector<float>& q, std::vector<float>& k, std::vector<float>& v, const block_q8_K* input_q8k,
                    int num_cols, const Tensor& tq, const Tensor& tk, const Tensor& tv) {
    const size_t qr = static_cast<size_t>(rows_of(tq)), kr = static_cast<size_t>(rows_of(tk));
    fit(q, qr);
    fit(k, kr);
    fit(v, kr);
    const mcpm_tensor *wq = device_tensor(tq), *wk = device_tensor(tk), *wv = device_tensor(tv);
    void* dq = upload(0, input_q8k, static_cast<size_t>(num_cols / 256) * sizeof(block_q8_K));
    float* o = static_cast<float*>(scratch(1, (qr + 2 * kr) * 4));
    const int rc = (wq && wk && wv) ? mcpm_gemv_qkv_q8_K(ctx(), wq, wk, wv, dq, o, o + qr, o + qr + kr,
                                                        static_cast<int>(qr), static_cast<int>(kr), num_cols)
                                    : MCPM_ERR_UNSUPPORTED;
    if (rc == MCPM_ERR_UNSUPPORTED) {
        warn_once(tv.type_str, "matmul_qkv_q8k: tensor type not supported");
        std::fill(q.begin(), q.end(), 0.0f);
        std::fill(k.begin(), k.end(), 0.0f);
        std::fill(v.begin(), v.end(), 0.0f);
        return;
    }
    check(rc, "mcpm_gemv_qkv_q8_K");
    download(q.data(), o, qr * 4);
    download(k.data(), o + qr, kr * 4);
    download(v.data(), o + qr + kr, kr * 4);
}

void matmul_gate_up_q8k(std::vector<float>& gate, std::vector<float>& up, const block_q8_K* input_q8k, int num_cols,
                        const Tensor& tg, const Tensor& tu) {
    const size_t rows = static_cast<size_t>(rows_of(tg));
    fit(gate, rows);
    fit(up, rows);
    const mcpm_tensor *wg = device_tensor(tg), *wu = device_tensor(tu);
    void* dq = upload(0, input_q8k, static_cast<size_t>(num_cols / 256) * sizeof(block_q8_K));
    float* o = static_cast<float*>(scratch(1, 2 * rows * 4));
    const int rc = (wg && wu) ? mcpm_gemv_gate_up_q4_K_q8_K(ctx(), wg, wu, dq, o, o + rows, static_cast<int>(rows),
                                                            num_cols)
                              : MCPM_ERR_UNSUPPORTED;
    if (rc == MCPM_ERR_UNSUPPORTED) {
        warn_once(tg.type_str, "matmul_gate_up_q8k: tensor type not supported");
        std::fill(gate.begin(), gate.end(), 0.0f);
        std::fill(up.begin(), up.end(), 0.0f);
        return;
    }
    check(rc, "mcpm_gemv_gate_up_q4_K_q8_K");
    download(gate.data(), o, rows * 4);
    download(up.data(), o + rows, rows * 4);
}

void get_embedding(std::vector<float>& out, const Tensor& embd, int token_id) {
    const size_t dim = static_cast<size_t>(cols_of(embd));
    fit(out, dim);
    const mcpm_tensor* e = device_tensor(embd);
    float* d = static_cast<float*>(scratch(0, dim * 4));
    const int rc = e ? mcpm_get_embedding(ctx(), d, e, token_id) : MCPM_ERR_UNSUPPORTED;
    if (rc == MCPM_ERR_UNSUPPORTED) {
        warn_once(embd.type_str, "get_embedding: tensor type not supported");
        std::fill(out.begin(), out.end(), 0.0f);
        return;
    }
    check(rc, "mcpm_get_embedding");
    download(out.data(), d, dim * 4);
}

void execute_attention(std::vector<float>& attn_out, const std::vector<float>& q, const std::vector<float>& k_curr,
                       const std::vector<float>& v_curr, KVCacheLayer& kv, int pos, int max_seq_len, int num_heads,
                       int num_kv_heads, int head_dim) {
    fit(attn_out, static_cast<size_t>(num_heads) * head_dim);
    if (pos >= max_seq_len) {
        std::fprintf(stderr, "[WARNING] Maximum context exceeded (pos >= max_seq_len).\n");
        return;
    }
    const size_t kvd = static_cast<size_t>(num_kv_heads) * head_dim;
    // the host cache is authoritative: positions 0..pos-1 go up, the new row
    // is appended on both sides
    const size_t cache_bytes = static_cast<size_t>(max_seq_len) * kvd * 4;
    float* dk = static_cast<float*>(scratch(0, cache_bytes));
    float* dv = static_cast<float*>(scratch(1, cache_bytes));
    const size_t hist = static_cast<size_t>(pos) * kvd * 4;
    if (hist) {
        check(mcpm_copy_to_device(ctx(), dk, kv.k.data(), hist), "mcpm_copy_to_device");
        check(mcpm_copy_to_device(ctx(), dv, kv.v.data(), hist), "mcpm_copy_to_device");
    }
    float* dq = static_cast<float*>(upload(2, q.data(), q.size() * 4));
    float* dkc = static_cast<float*>(upload(3, k_curr.data(), kvd * 4));
    float* dvc = static_cast<float*>(upload(4, v_curr.data(), kvd * 4));
    float* dout = static_cast<float*>(scratch(5, attn_out.size() * 4));
    check(mcpm_execute_attention(ctx(), dout, dq, dkc, dvc, dk, dv, pos, max_seq_len, num_heads, num_kv_heads,
                                 head_dim),
          "mcpm_execute_attention");
    download(attn_out.data(), dout, attn_out.size() * 4);
    const size_t need = (static_cast<size_t>(pos) + 1) * kvd;
    if (kv.k.size() < need) kv.k.resize(need);
    if (kv.v.size() < need) kv.v.resize(need);
    std::memcpy(kv.k.data() + static_cast<size_t>(pos) * kvd, k_curr.data(), kvd * 4);
    std::memcpy(kv.v.data() + static_cast<size_t>(pos) * kvd, v_curr.data(), kvd * 4);
}
