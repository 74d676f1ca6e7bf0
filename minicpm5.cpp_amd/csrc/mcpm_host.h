// mcpm_host.h -- host-side objects behind the C ABI handles.
#pragma once

#include <utility>
#include <vector>

#include "mcpm_internal.h"

struct mcpm_ctx {
  int device = 0;
  int n_cu = 0;
  std::string name;
  hipStream_t stream = nullptr;
  // per-op scratch, grown on demand
  mcpm::StepState* d_state = nullptr;
  mcpm::StepState* h_state = nullptr;  // pinned
  float2* d_rope = nullptr;            // one (cos, sin) row
  float2* h_rope = nullptr;            // pinned
  int rope_cap = 0;
  float* d_attn_part = nullptr;
  size_t attn_part_cap = 0;
  float2* d_argmax_part = nullptr;
  int argmax_cap = 0;
  void* d_sample = nullptr;  // device sampler scratch
  size_t sample_cap = 0;
  // per-op kernel timing (mcpm_set_op_timing): an event pair per timed launch
  bool op_timing = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> op_events;
  size_t op_used = 0;
};

struct mcpm_tensor {
  mcpm::DevTensor t;
};

namespace mcpm {
// Uploads a native tensor image; used by the C ABI and by the engine.
int upload_tensor(mcpm_ctx* ctx, const void* host_blocks, size_t bytes, int type, int64_t cols, int64_t rows,
                  DevTensor& out);
void free_tensor(DevTensor& t);
int ensure_attn_scratch(mcpm_ctx* ctx, size_t floats);
int ensure_argmax_scratch(mcpm_ctx* ctx, int n);
// mcpm_noalloc.hip: the device address of its fixed scratch array on the
// current device, looked up once per device (called by mcpm_init).
int noalloc_setup(int device);
// (cos, sin) of pos * theta_i, theta_i = 1/base^(2i/head_dim), i < head_dim/2
// (src/ops/ops.cpp:503-508), evaluated with the C library's powf/cosf/sinf.
void rope_row(int pos, int head_dim, float base, float2* out);
}  // namespace mcpm

namespace mcpm {
// Sampler::sample (src/sampler.cpp:8-73) for a given uniform draw r.
int sample_token(const float* logits, int n, float temperature, float top_p, float r);
}  // namespace mcpm
