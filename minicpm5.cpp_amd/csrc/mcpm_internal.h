// mcpm_internal.h -- definitions shared by the HIP kernels and the host code of
// libmcpm_hip.so.  Not installed; the public surface is include/mcpm_hip.h.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>

#include "mcpm_hip.h"

namespace mcpm {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int MAX_NB = 32;        // largest K / 256 the Q8_K GEMVs accept (K <= 8192)
constexpr int ATTN_CHUNK = 64;    // positions per attention split
constexpr int ATTN_MAX_GROUP = 8;  // query heads per kv head the attention kernels take, at most
constexpr int ATTN_CPW = 8;        // chunks one attention split takes, at most
constexpr int GEMV_MAX_WAVES = 8;  // GEMV work groups: 4..8 waves (ROW shape)
constexpr int GEMV_TILE_WAVES = 4;  // TILE shape: one wave per SIMD
constexpr int ROWS_PER_GROUP = 8; // output rows per GEMV work item (8 lanes each)

// ggml block layouts (include/ops.h:33-65).  Byte images only; the kernels
// read the re-laid-out planes described in DevTensor.
struct BlockQ8_0 { uint16_t d; int8_t qs[32]; };
struct BlockQ4K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct BlockQ6K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; };
struct BlockQ8K { float d; int8_t qs[256]; int16_t bsums[16]; };
static_assert(sizeof(BlockQ8_0) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(BlockQ4K) == 144, "Q4_K block is 144 bytes");
static_assert(sizeof(BlockQ6K) == 210, "Q6_K block is 210 bytes");
static_assert(sizeof(BlockQ8K) == 292, "Q8_K block is 292 bytes");

// IEEE binary16 -> binary32, exact for every input (the conversion of
// include/ops.h:14-31 and of F16C's _cvtsh_ss).
__host__ __device__ inline float fp16_to_fp32(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
#else
  uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  int32_t exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { mant <<= 1; e++; } while (!(mant & 0x400u));
      bits = sign | (static_cast<uint32_t>(112 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else {
    bits = sign | (static_cast<uint32_t>(exp + 112) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
#endif
}

// fp32 -> binary16, round to nearest even (used by the weight encoders).
uint16_t fp32_to_fp16(float f);

// exp(x) in fp32 from the mathematics: k = nearest integer to x/ln2, r = x -
// k*ln2 with ln2 split in two parts (Cody-Waite), exp(r) by its Taylor series
// to degree 7 (Horner, fused multiply-adds), times 2^k.  Host and device run
// the same operation sequence, so they round identically.  Used where the
// reference calls std::exp (SiLU ops.cpp:740, softmax ops.cpp:601,
// sampler.cpp:30,36).
__host__ __device__ inline float exp_f32(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -103.972084045410156f) return 0.0f;
  const float inv_ln2 = 1.44269502162933349609375f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.428606765330187045e-06f;
  const float k = __builtin_rintf(x * inv_ln2);
  float r = __builtin_fmaf(-k, ln2_hi, x);
  r = __builtin_fmaf(-k, ln2_lo, r);
  float p = 1.98412698412698412526e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888894189e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333321769e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666643537e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666657415e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(k));
}

// A weight matrix in HBM.  Each block's bytes are split into planes, and a
// plane is cut into 16-byte chunks stored chunk-major then row-major: chunk c
// of block b of row r at ((b*nc + c)*rows + r)*16 (nc chunks per block), so
// a load instruction over consecutive rows reads consecutive memory.
//   Q4_K  p0: the 128 quant bytes, nc = 8;  p1: 16 B header (d, dmin, 12
//             scale bytes) at (b*rows + r)*16.
//   Q6_K  p0: 128 B ql, nc = 8;  p1: 64 B qh, nc = 4;  p2: 16 B int8 scales
//             at (b*rows + r)*16;  p3: 2 B d at (b*rows + r)*2.
//   Q8_0  p0: 32 B quants at (b*rows + r)*32;  p1: 2 B d at (b*rows + r)*2.
//   F32   p0: row-major floats.
// Chunks keep the block's native byte order and bytes per block are unchanged
// (144 / 210 / 34), so dequantized values are bit-identical to the GGUF blocks.
struct DevTensor {
  int type = -1;
  int64_t rows = 0, cols = 0;
  int nb = 0;  // blocks per row
  void* base = nullptr;
  size_t bytes = 0;  // native (GGUF) size == device size
  const uint8_t* p0 = nullptr;
  const uint8_t* p1 = nullptr;
  const uint8_t* p2 = nullptr;
  const uint8_t* p3 = nullptr;
  bool owned = true;
};

// Kernel-side view of one weight matrix.
struct WView {
  int type;
  int rows;
  int nb;
  const uint8_t* p0;
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
};

inline WView view_of(const DevTensor& t) {
  return WView{t.type, static_cast<int>(t.rows), t.nb, t.p0, t.p1, t.p2, t.p3};
}

size_t type_row_bytes(int type, int64_t cols);
int type_block_elems(int type);
// Host-side plane layout: native GGUF bytes <-> device image.
void repack_to_device_image(int type, int64_t rows, int64_t cols, const uint8_t* native, uint8_t* image);
void repack_from_device_image(int type, int64_t rows, int64_t cols, const uint8_t* image, uint8_t* native);
void set_planes(DevTensor& t);

// ------------------------------------------------------------ errors -------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define MCPM_HIP(call)                                      \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return ::mcpm::hip_fail(e_, #call); \
  } while (0)

// ------------------------------------------------------------ launches -----
// Prologue modes of the Q8_K GEMV: how the WG obtains its Q8_K activations.
enum Prologue : int {
  PRO_Q8K = 0,        // native Q8_K blocks in global memory
  PRO_QUANT_EVEN = 1, // quantize an fp32 vector, ties to even (quantize_row_q8_K)
  PRO_QUANT_AWAY = 2, // quantize an fp32 vector, ties away (lround)
  PRO_NORM_AWAY = 3,  // RMSNorm then quantize, ties away (rmsnorm_and_quantize_q8k)
  PRO_NORM_EVEN = 4,  // RMSNorm then quantize, ties to even (rmsnorm + matmul)
  PRO_ATTN_EVEN = 5,  // combine the attention partials, then quantize ties to even
  PRO_ATTN_ONE = 6,   // attention of every head over a one-chunk context (q in x, K and V
                      // rows in k_cache / v_cache), shared among each XCD's work groups
                      // through tagged records, then quantize ties to even
};

// Epilogue modes.
enum Epilogue : int {
  EPI_STORE = 0,   // out[row] = v
  EPI_QKV = 1,     // RoPE on q,k; q -> out0, k,v -> KV cache at pos
  EPI_RESID = 2,   // x[row] += v
  EPI_SWIGLU = 3,  // gate/up pairs -> h = silu(g)*u
  EPI_LOGITS = 4,  // out[row] = v plus per-WG argmax
};

struct GemvRegion {
  WView w;
  float* out;
  int row0;  // first virtual row of this region
  int rows;
};

// Per-chunk attention partials of every head (see k_attention): o_c values
// [n_heads][max_chunks][head_dim] and (m_c, z_c) [n_heads][max_chunks], in
// one allocation of n_heads*max_chunks*(head_dim+2) floats, o first.
struct AttnPart {
  float* o;
  float2* mz;
};
inline AttnPart attn_part_of(float* base, int n_heads, int max_chunks, int head_dim) {
  return AttnPart{base, reinterpret_cast<float2*>(base + static_cast<size_t>(n_heads) * max_chunks * head_dim)};
}

struct GemvArgs {
  GemvRegion reg[3];
  int nreg;
  int total_rows;  // virtual rows (pair mode: rows of one matrix)
  int nb;
  int pair;        // 1: slots 0-3 from reg[0], 4-7 from reg[1], same rows
  // prologue inputs
  const BlockQ8K* xq;
  const float* x;
  const float* gamma;
  float eps;
  const float2* attn_mz;  // PRO_ATTN_EVEN: x is the partials' o, these their (m, z)
  int attn_max_chunks;
  // epilogue inputs
  const int* state;      // [0] token, [1] pos
  const float2* rope_cs; // [max_seq][head_dim/2] (cos, sin)
  int head_dim;
  float* k_cache;        // layer base, [max_seq][kvd]
  float* v_cache;
  int kvd;
  float* resid;
  float* h_out;
  float2* argmax_part;   // per wave (value, index as float bits)
  int argmax_parts;      // EPI_LOGITS: entries of argmax_part (the launch must write exactly these)
  // PRO_ATTN_ONE: work group j of an XCD computes query heads j*attn_hpw ..
  // and stores them as (value, tag) records in its XCD's array of xrec
  // ([8][heads*64]); tag = epoch[0] * tag_mul + tag_add.  xcc[x]: the XCD
  // that work groups b % 8 == x ran on at set-up.  A wait past spin_limit
  // polls, or a work group on another XCD, sets err.
  uint64_t* xrec;
  const unsigned* epoch;
  unsigned tag_mul, tag_add;
  int attn_hpw;
  const int* xcc;
  unsigned* err;
  unsigned spin_limit;
};

// Device step state shared by the engine's kernels.
struct StepState {
  int token;
  int pos;
  int step;       // index of the next generated token
  int n_out;      // capacity of the generated-token array
};

hipError_t launch_gemv(const GemvArgs& a, int prologue, int epilogue, int n_cu, hipStream_t s);
// The query heads per work group a PRO_ATTN_ONE / EPI_RESID launch of a would
// take (its grid's work groups per XCD covering every head), 0 when it
// cannot run.
int gemv_attn_one_hpw(const GemvArgs& a, int n_cu);

// The grid barrier state of the fused kernels (device memory, zeroed at
// allocation): ctr[64 * x] arrivals of XCD x, the launch count, and an error
// word set when a wait passed spin_limit polls.
struct GridSync {
  unsigned* ctr;
  unsigned* gen;
  unsigned* err;
  unsigned spin_limit;
};
constexpr size_t GRID_SYNC_WORDS = 8 * 64 + 64 + 64;
// The FFN block (gate/up, then down) of one layer in one launch; gu and dn as
// for launch_gemv's PRO_NORM_AWAY/EPI_SWIGLU and PRO_QUANT_AWAY/EPI_RESID.
// hipErrorNotSupported when a phase's shape does not fit one resident round
// of work groups (the caller launches the two kernels then).
hipError_t launch_ffn_fused(const GemvArgs& gu, const GemvArgs& dn, int n_cu, const GridSync& gs, hipStream_t s);

// The attention inputs of the QKV + attention launch: q, the layer's K and V
// cache, the step state (position at state[1]) and the chunk partials, as
// for launch_attention.
struct AttnArgs {
  const float* q;
  const float* kc;
  const float* vc;
  const int* state;
  int n_heads, n_kv_heads, head_dim, max_chunks;
  float* part_o;
  float2* part_mz;
};
// QKV (as launch_gemv's PRO_NORM_AWAY/EPI_QKV) and the attention of one
// layer in one launch, with a grid barrier between them.
// hipErrorNotSupported when the QKV shape does not fit one resident round of
// work groups (the caller launches the two kernels then).
hipError_t launch_qkv_attn(const GemvArgs& qkv, const AttnArgs& at, int n_cu, const GridSync& gs, hipStream_t s);

// The temperature / top-p sampler on the device (mcpm_sampler.hip): scratch
// bytes for n logits, and its passes for one uniform draw r.  The token goes
// to *out_token (device) when given, and when st is given it becomes the next
// input token, is appended to out_tokens and pos advances (as the argmax does).
size_t sampler_bytes(int n);
int sampler_max_n();  // largest n launch_sample takes
float sampler_sort_free_top_p();  // cuts up to this top_p need no sort
// draws (with st): the draw is read on the device, draws[st->step], in place
// of r, so the launches can be captured once and replayed for every token.
hipError_t launch_sample(void* scratch, size_t scratch_bytes, const float* logits, int n, float temperature,
                         float top_p, float r, int* out_token, StepState* st, int* out_tokens, hipStream_t s,
                         const float* draws = nullptr);

// When `start` is set, the GEMV and attention launch helpers record these
// events at their kernel's start and end (hipExtLaunchKernel), so the elapsed
// time is the kernel's own duration.  Set around one launch by the engine's
// per-class timing; launches are eager then.
struct LaunchTiming {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
extern thread_local LaunchTiming g_launch_timing;

template <typename K, typename... Args>
void launch_kernel(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  if (g_launch_timing.start)
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s, g_launch_timing.start,
                          g_launch_timing.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}
int gemv_grid(const GemvArgs& a, int n_cu);

hipError_t launch_quantize_q8k(const float* x, const float* gamma, float eps, int dim, int mode, BlockQ8K* out,
                               hipStream_t s);
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, int dim, float* out, hipStream_t s);
hipError_t launch_swiglu_quant(const float* g, const float* u, int dim, BlockQ8K* out, hipStream_t s);
hipError_t launch_rope(float* vec, const float2* cs, int n_heads, int head_dim, hipStream_t s);
hipError_t launch_kv_append(const float* k, const float* v, float* kc, float* vc, const int* state, int kvd,
                            hipStream_t s);
hipError_t launch_attention(const float* q, const float* kc, const float* vc, const int* state, int n_heads,
                            int n_kv_heads, int head_dim, int max_chunks, const AttnPart& part, hipStream_t s);
// Decode attention for contexts of at most ATTN_Q8K_MAX_CHUNKS chunks (512
// positions), head_dim 64, one work group per kv head, its output combined and quantized ties-even into Q8_K blocks
// (for the O projection); shapes whose query group covers whole blocks.
// A longer context sets *err and writes nothing.
constexpr int ATTN_Q8K_MAX_CHUNKS = 8;
constexpr int ATTN_Q8K_CHUNKS = 3;  // the decode engine's default limit
inline bool attn_q8k_fits(int n_heads, int n_kv_heads, int head_dim) {
  return n_kv_heads > 0 && head_dim == 64 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 8 &&
         (n_heads / n_kv_heads * head_dim) % 256 == 0;
}
hipError_t launch_attention_q8k(const float* q, const float* kc, const float* vc, const int* state, int n_heads,
                                int n_kv_heads, int head_dim, BlockQ8K* out, unsigned* err, hipStream_t s);
hipError_t launch_attn_combine(const AttnPart& part, const int* state, int n_heads, int head_dim, int max_chunks,
                               float* out, hipStream_t s);

// ---- prefill (batched prompt tokens; csrc/mcpm_prefill.hip) ----
// Per-token Q8_K activations: fp16 codes [t][dim], d [t][dim/256], fp16
// bsums [t][dim/256][16].
struct QuantBatch {
  _Float16* xh;
  float* xd;
  _Float16* xbs;
};
hipError_t launch_embed_batch(const WView& w, const int* tokens, int n_tok, int dim, float* x, hipStream_t s);
hipError_t launch_quant_batch(const float* x, const float* u, int ld_x, const float* gamma, float eps, int dim,
                              int n_valid, int mode, int n_tok, QuantBatch q, hipStream_t s);
hipError_t launch_quant_batch_swiglu(const float* g, const float* u, int ld, int n_valid, int dim, int n_tok,
                                     QuantBatch q, hipStream_t s);
// RoPE applied to a GEMM's row pairs before they are stored: the (cos, sin)
// table (head_dim/2 pairs per position), token t at position pos0 + t.
struct GemmRope {
  const float2* table;
  int head_dim, pos0;
};
// w2 / rows2 / out2 / ld_out2: a second matrix of w's type on the same
// activations in the same launch (rows % 64 == 0).
hipError_t launch_gemm_q8k(const WView& w, int rows, int nb, int n_tok, const QuantBatch& q, float* out, int ld_out,
                           bool add, hipStream_t s, const WView* w2 = nullptr, int rows2 = 0, float* out2 = nullptr,
                           int ld_out2 = 0, const GemmRope* rope = nullptr, bool swiglu = false);
hipError_t launch_attention_batch(const float* q, const float* kc, const float* vc, int n_heads, int n_kv_heads,
                                  int head_dim, int max_chunks, const AttnPart& part, size_t tok_o, size_t tok_mz,
                                  int pos0, int n_tok, hipStream_t s);
// The attention output of each token from its chunk partials, quantized
// ties-even into q (the O projection's input), in one pass.
hipError_t launch_quant_batch_attn(const AttnPart& part, size_t tok_stride_o, size_t tok_stride_mz, int pos0,
                                   int n_tok, int n_heads, int head_dim, int max_chunks, QuantBatch q, hipStream_t s);
// epoch (optional): advanced by one (the tags of the token's XCD records).
hipError_t launch_embedding(const WView& w, const int* state, int dim, float* out, hipStream_t s,
                            unsigned* epoch = nullptr);
hipError_t launch_dequant_rows(const WView& w, int row0, int n_rows, int cols, float* out, hipStream_t s);
hipError_t launch_gemv_f32(const float* w, const float* x, float* out, int rows, int cols, hipStream_t s);
hipError_t launch_stream_read(const void* src, size_t bytes, int grid, uint32_t* out, hipStream_t s);
hipError_t launch_gemv_q8_0(const WView& w, const float* x, float* out, int rows, int cols, hipStream_t s);
hipError_t launch_argmax_partial(const float* x, int n, float2* part, int nparts, hipStream_t s);
hipError_t launch_argmax_final(const float2* part, int nparts, int* out_token, StepState* st, int* out_tokens,
                               hipStream_t s);
hipError_t launch_fill_f32(float* p, float v, size_t n, hipStream_t s);

}  // namespace mcpm
