// ops.h -- the operator API of MiniCPM5.cpp (include/ops.h:104-160) served by
// the HIP engine.  Same names, argument meaning and host-vector contract:
// outputs are resized when their size differs, results are in place when the
// call returns, unsupported tensor types warn once and fill a constant
// (src/ops/ops.cpp:288,347).  Each host thread gets its own GPU context on
// first use; weight tensors are uploaded to HBM once, keyed by their host
// data pointer, so a Tensor's bytes must not change after its first use.
// A GPU failure throws std::runtime_error (the reference never fails, but this
// build does not fall back to the CPU).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "mcpm_hip.h"

// Q8_K activation block (include/ops.h:58-65): 256 int8 codes, scale, and the
// sums of each group of 16 codes.
struct block_q8_K {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
static_assert(sizeof(block_q8_K) == 292, "block_q8_K is 292 bytes");

// A tensor of the model file (include/ops.h:104-110): dims[0] = columns,
// dims[1] = rows; data_ptr points at the native (GGUF) bytes in host memory.
struct Tensor {
    std::string name;
    std::string type_str;  // "Q4_K", "Q6_K", "Q8_0" or "F32"
    std::vector<uint64_t> dims;
    const char* data_ptr = nullptr;
    uint64_t size_bytes = 0;
};

float silu(float x);
void rmsnorm(std::vector<float>& out, const std::vector<float>& x, const Tensor& weight_tensor, float eps = 1e-6f);
void rmsnorm_and_quantize_q8k(block_q8_K* out_q8k, const std::vector<float>& x, const Tensor& weight_tensor,
                              float eps = 1e-6f);
void swiglu_and_quantize_q8k(block_q8_K* out_q8k, const std::vector<float>& gate, const std::vector<float>& up);
void apply_rope(std::vector<float>& vec, int pos, int head_idx, int head_dim, float rope_base);
void matmul(std::vector<float>& output, const std::vector<float>& input, const Tensor& tensor);
void quantize_row_q8_K(const float* x, int n, block_q8_K* y);
void matmul_q8k(std::vector<float>& output, const block_q8_K* input_q8k, int num_cols, const Tensor& tensor);
void matmul_qkv_q8k(std::vector<float>& q, std::vector<float>& k, std::vector<float>& v, const block_q8_K* input_q8k,
                    int num_cols, const Tensor& tensor_q, const Tensor& tensor_k, const Tensor& tensor_v);
void matmul_gate_up_q8k(std::vector<float>& gate, std::vector<float>& up, const block_q8_K* input_q8k, int num_cols,
                        const Tensor& tensor_gate, const Tensor& tensor_up);
void get_embedding(std::vector<float>& out, const Tensor& embd_tensor, int token_id);

// One layer's KV cache (include/ops.h:147-150): fp32 [max_seq][kv_heads][head_dim].
struct KVCacheLayer {
    std::vector<float> k;
    std::vector<float> v;
};

void execute_attention(std::vector<float>& attn_out, const std::vector<float>& q, const std::vector<float>& k_curr,
                       const std::vector<float>& v_curr, KVCacheLayer& kv_cache, int pos, int max_seq_len,
                       int num_heads, int num_kv_heads, int head_dim);

namespace mcpm_host {
// This thread's GPU context (device 0), created on first use.
mcpm_ctx* context();
}  // namespace mcpm_host
