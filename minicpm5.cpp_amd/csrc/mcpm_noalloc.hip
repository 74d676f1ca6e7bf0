// mcpm_noalloc.hip -- execute_attention for callers that cannot allocate
// device memory (code under graph capture, tight serving loops, harnesses
// that forbid hipMalloc): mcpm_execute_attention_noalloc runs the kernels of
// mcpm_execute_attention with its chunk partials in a fixed device array
// instead of the context's grow-on-demand buffer, and calls no allocating
// routine.
//
// The array, `scratch`, is one per GPU (each device holds its own copy at its
// own address) and lives until the process ends.  Its device address is
// looked up once per device when mcpm_init opens that device
// (mcpm_noalloc_setup); host code uses that address, never the array's name.
// Every call on a GPU shares the array: calls that overlap on one GPU (two
// contexts or threads at once) race.  No part of it must start at zero: the
// attention kernel writes every chunk record that the combine reads.
#include <mutex>

#include "mcpm_host.h"

namespace mcpm {

namespace {

// Chunk records of n_heads x ceil(max_seq_len / 64) chunks, head_dim + 2 floats
// each: at most 64 heads x 64 chunks (4096 positions) x 130 floats, 2.03 MiB.
constexpr size_t kScratchFloats = size_t{64} * 64 * (128 + 2);
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
float* g_scratch[kMaxDevices] = {};  // device address of `scratch` per GPU
std::mutex g_mu;

}  // namespace

// With `device` current (mcpm_init): the device address of this GPU's copy.
int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(MCPM_ERR_ARG, "mcpm_init: device id beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[device]) return MCPM_OK;
  void* p = nullptr;
  MCPM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  if (!p) return fail(MCPM_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
  g_scratch[device] = static_cast<float*>(p);
  return MCPM_OK;
}

}  // namespace mcpm

using namespace mcpm;

extern "C" int mcpm_execute_attention_noalloc(mcpm_ctx* c, float* out, const float* q, const float* k_cur,
                                              const float* v_cur, float* k_cache, float* v_cache, int pos,
                                              int max_seq_len, int n_heads, int n_kv_heads, int head_dim) {
  if (!c || !out || !q || !k_cur || !v_cur || !k_cache || !v_cache || pos < 0 || n_heads <= 0 ||
      n_kv_heads <= 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 8 || head_dim <= 0 || head_dim > 128 ||
      head_dim % 4 || n_kv_heads > 256)
    return fail(MCPM_ERR_ARG, "mcpm_execute_attention_noalloc: bad argument");
  if (pos >= max_seq_len) return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  const int max_chunks = (max_seq_len + ATTN_CHUNK - 1) / ATTN_CHUNK;
  const size_t need = static_cast<size_t>(n_heads) * max_chunks * (2 + head_dim);
  if (need > kScratchFloats)
    return fail(MCPM_ERR_ARG, "mcpm_execute_attention_noalloc: n_heads * ceil(max_seq_len/64) * (head_dim+2) = " +
                                  std::to_string(need) + " floats exceeds the fixed scratch of " +
                                  std::to_string(kScratchFloats));
  float* base = (c->device >= 0 && c->device < kMaxDevices) ? g_scratch[c->device] : nullptr;
  if (!base) return fail(MCPM_ERR_CONTEXT, "mcpm_execute_attention_noalloc: scratch not set up for this device");
  // the position, through the context's pinned staging (allocated at mcpm_init)
  c->h_state->token = 0;
  c->h_state->pos = pos;
  c->h_state->step = 0;
  c->h_state->n_out = 0;
  MCPM_HIP(hipMemcpyAsync(c->d_state, c->h_state, sizeof(StepState), hipMemcpyHostToDevice, c->stream));
  const int kvd = n_kv_heads * head_dim;
  const int* st = reinterpret_cast<const int*>(c->d_state);
  MCPM_HIP(launch_kv_append(k_cur, v_cur, k_cache, v_cache, st, kvd, c->stream));
  const AttnPart part = attn_part_of(base, n_heads, max_chunks, head_dim);
  MCPM_HIP(launch_attention(q, k_cache, v_cache, st, n_heads, n_kv_heads, head_dim, max_chunks, part, c->stream));
  MCPM_HIP(launch_attn_combine(part, st, n_heads, head_dim, max_chunks, out, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}
