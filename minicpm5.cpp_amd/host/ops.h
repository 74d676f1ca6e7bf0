// ops.h -- the operator API of MiniCPM5.cpp (include/ops.h) served by the HIP
// engine.  The declarations, types and block layouts are the reference's,
// member for member and signature for signature, so code compiled against
// the reference's own include/ops.h links against libmcpm_ops.so in place of
// src/ops/*.cpp with no change to its sources or headers, and code compiled
// against this header sees the same types.
//
// Behaviour follows the reference's host-vector contract: outputs are resized
// when their size differs, results are in place when the call returns,
// unsupported tensor types warn once and fill a constant
// (src/ops/ops.cpp:288,347).  Each host thread gets its own GPU context on
// first use; weight tensors are uploaded to HBM once, keyed by their host
// data pointer, so a Tensor's bytes must not change after its first use.  A
// GPU failure throws std::runtime_error (the reference never fails, but this
// build does not fall back to the CPU).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

// ------------------------------------------------ ggml block formats ------
// include/ops.h:11-97: the file's block layouts and helpers.

typedef uint16_t ggml_fp16_t;

// IEEE binary16 -> binary32, exact for every input, subnormals, infinities
// and NaN payloads included (the conversion of include/ops.h:14-31).
static inline float fp16_to_fp32(ggml_fp16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);  // inf / NaN, payload kept
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;  // signed zero
    } else {
        // subnormal: normalise the mantissa, one exponent step per shift
        uint32_t shifts = 0;
        while (!(m & 0x400u)) {
            m <<= 1;
            ++shifts;
        }
        bits = sign | ((113u - shifts) << 23) | ((m & 0x3ffu) << 13);
    }
    union {
        uint32_t u;
        float f;
    } v;
    v.u = bits;
    return v.f;
}

#define QK8_0 32
#define QK_K 256
#define K_SCALE_SIZE 12

// Q8_0: 32 weights, 34 bytes.
struct block_q8_0 {
    ggml_fp16_t d;
    int8_t qs[QK8_0];
};

// Q4_K: 256 weights in 8 sub-blocks of 32, 144 bytes: w = d*sc*q - dmin*mn.
struct block_q4_K {
    ggml_fp16_t d;
    ggml_fp16_t dmin;
    uint8_t scales[K_SCALE_SIZE];  // 6-bit scales and mins, packed
    uint8_t qs[QK_K / 2];          // 4-bit codes
};

// Q6_K: 256 weights in 16 sub-blocks of 16, 210 bytes: w = d*sc*(q - 32).
struct block_q6_K {
    uint8_t ql[QK_K / 2];      // low 4 bits of each code
    uint8_t qh[QK_K / 4];      // high 2 bits
    int8_t scales[QK_K / 16];  // sub-block scales
    ggml_fp16_t d;
};

// Q8_K activation block: 256 int8 codes, scale, and the sums of each group
// of 16 codes.
struct block_q8_K {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
};
static_assert(sizeof(block_q8_0) == 34, "block_q8_0 is 34 bytes");
static_assert(sizeof(block_q4_K) == 144, "block_q4_K is 144 bytes");
static_assert(sizeof(block_q6_K) == 210, "block_q6_K is 210 bytes");
static_assert(sizeof(block_q8_K) == 292, "block_q8_K is 292 bytes");

// Scale and min of Q4_K sub-block j (0..7) from the 12 packed bytes q: the
// low 6 bits of bytes j and j+4 for j < 4; otherwise the nibbles of byte j+4
// completed by the top two bits of bytes j-4 (scale) and j (min).
static inline void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = static_cast<uint8_t>(q[j] & 0x3f);
        *m = static_cast<uint8_t>(q[j + 4] & 0x3f);
    } else {
        *d = static_cast<uint8_t>((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = static_cast<uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// All eight scales and mins of a Q4_K block.
static inline void decode_q4k_scales_mins(const uint8_t* q, uint8_t* sc, uint8_t* mn) {
    for (int j = 0; j < 8; ++j) get_scale_min_k4(j, q, &sc[j], &mn[j]);
}

// ------------------------------------------------------- operators -------

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
