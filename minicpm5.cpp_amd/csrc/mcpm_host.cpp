// mcpm_host.cpp -- context, device memory, weight upload and the per-op C ABI.
#include "mcpm_host.h"

#include <cmath>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace mcpm {

thread_local LaunchTiming g_launch_timing;

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return MCPM_ERR_HIP;
}

// ------------------------------------------------------------ plane layout

void set_planes(DevTensor& t) {
  const uint8_t* b = static_cast<const uint8_t*>(t.base);
  const size_t nblk = static_cast<size_t>(t.rows) * t.nb;
  t.p0 = b;
  t.p1 = t.p2 = t.p3 = nullptr;
  if (t.type == MCPM_TYPE_Q4_K) {
    t.p1 = b + nblk * 128;
  } else if (t.type == MCPM_TYPE_Q6_K) {
    t.p1 = b + nblk * 128;
    t.p2 = t.p1 + nblk * 64;
    t.p3 = t.p2 + nblk * 16;
  } else if (t.type == MCPM_TYPE_Q8_0) {
    t.p1 = b + nblk * 32;
  }
}

// Native row-major blocks <-> chunked planes (see DevTensor).  One routine
// serves both directions: `to_dev` copies native -> image, else image -> native.
static void repack_planes(int type, int64_t rows, int64_t cols, uint8_t* nat, uint8_t* img, bool to_dev) {
  const int64_t nb = cols / type_block_elems(type);
  const size_t R = static_cast<size_t>(rows), nblk = static_cast<size_t>(rows * nb);
  auto mv = [&](uint8_t* native_bytes, uint8_t* image_bytes, size_t n) {
    if (to_dev) std::memcpy(image_bytes, native_bytes, n);
    else std::memcpy(native_bytes, image_bytes, n);
  };
  auto chunk = [&](uint8_t* plane, int nc, int64_t b, int c, int64_t r) {
    return plane + ((static_cast<size_t>(b) * nc + c) * R + static_cast<size_t>(r)) * 16;
  };
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const size_t di = static_cast<size_t>(b) * R + static_cast<size_t>(r);
      if (type == MCPM_TYPE_Q4_K) {
        uint8_t* s = nat + (static_cast<size_t>(r * nb + b)) * sizeof(BlockQ4K);
        for (int c = 0; c < 8; ++c) mv(s + offsetof(BlockQ4K, qs) + 16 * c, chunk(img, 8, b, c, r), 16);
        mv(s, img + nblk * 128 + di * 16, 16);
      } else if (type == MCPM_TYPE_Q6_K) {
        uint8_t* s = nat + (static_cast<size_t>(r * nb + b)) * sizeof(BlockQ6K);
        for (int c = 0; c < 8; ++c) mv(s + offsetof(BlockQ6K, ql) + 16 * c, chunk(img, 8, b, c, r), 16);
        for (int c = 0; c < 4; ++c) mv(s + offsetof(BlockQ6K, qh) + 16 * c, chunk(img + nblk * 128, 4, b, c, r), 16);
        mv(s + offsetof(BlockQ6K, scales), img + nblk * 192 + di * 16, 16);
        mv(s + offsetof(BlockQ6K, d), img + nblk * 208 + di * 2, 2);
      } else if (type == MCPM_TYPE_Q8_0) {
        uint8_t* s = nat + (static_cast<size_t>(r * nb + b)) * sizeof(BlockQ8_0);
        mv(s + offsetof(BlockQ8_0, qs), img + di * 32, 32);
        mv(s + offsetof(BlockQ8_0, d), img + nblk * 32 + di * 2, 2);
      }
    }
  }
}

void repack_to_device_image(int type, int64_t rows, int64_t cols, const uint8_t* nat, uint8_t* img) {
  if (type == MCPM_TYPE_F32) {
    std::memcpy(img, nat, static_cast<size_t>(rows * cols * 4));
    return;
  }
  repack_planes(type, rows, cols, const_cast<uint8_t*>(nat), img, true);
}

void repack_from_device_image(int type, int64_t rows, int64_t cols, const uint8_t* img, uint8_t* nat) {
  if (type == MCPM_TYPE_F32) {
    std::memcpy(nat, img, static_cast<size_t>(rows * cols * 4));
    return;
  }
  repack_planes(type, rows, cols, nat, const_cast<uint8_t*>(img), false);
}

int upload_tensor(mcpm_ctx* ctx, const void* host, size_t bytes, int type, int64_t cols, int64_t rows,
                  DevTensor& out) {
  const int be = type_block_elems(type);
  if (!host || be == 0) return fail(MCPM_ERR_UNSUPPORTED, "tensor upload: unsupported type " + std::to_string(type));
  if (cols <= 0 || rows <= 0 || cols % be) return fail(MCPM_ERR_ARG, "tensor upload: bad dims");
  const size_t need = type_row_bytes(type, cols) * static_cast<size_t>(rows);
  if (bytes != need) return fail(MCPM_ERR_ARG, "tensor upload: size " + std::to_string(bytes) + " != " + std::to_string(need));
  std::vector<uint8_t> img(need);
  repack_to_device_image(type, rows, cols, static_cast<const uint8_t*>(host), img.data());
  DevTensor t;
  t.type = type;
  t.rows = rows;
  t.cols = cols;
  t.nb = static_cast<int>(cols / be);
  t.bytes = need;
  MCPM_HIP(hipMalloc(&t.base, need));
  hipError_t e = hipMemcpyAsync(t.base, img.data(), need, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(t.base);
    return hip_fail(e, "tensor upload copy");
  }
  set_planes(t);
  out = t;
  return MCPM_OK;
}

void free_tensor(DevTensor& t) {
  if (t.base && t.owned) (void)hipFree(t.base);
  t.base = nullptr;
}

int ensure_attn_scratch(mcpm_ctx* ctx, size_t floats) {
  if (floats <= ctx->attn_part_cap) return MCPM_OK;
  if (ctx->d_attn_part) (void)hipFree(ctx->d_attn_part);
  ctx->d_attn_part = nullptr;
  MCPM_HIP(hipMalloc(&ctx->d_attn_part, floats * sizeof(float)));
  ctx->attn_part_cap = floats;
  return MCPM_OK;
}

int ensure_argmax_scratch(mcpm_ctx* ctx, int n) {
  if (n <= ctx->argmax_cap) return MCPM_OK;
  if (ctx->d_argmax_part) (void)hipFree(ctx->d_argmax_part);
  ctx->d_argmax_part = nullptr;
  MCPM_HIP(hipMalloc(&ctx->d_argmax_part, n * sizeof(float2)));
  ctx->argmax_cap = n;
  return MCPM_OK;
}

void rope_row(int pos, int head_dim, float base, float2* out) {
  for (int i = 0; i < head_dim; i += 2) {
    const float theta = 1.0f / powf(base, static_cast<float>(i) / static_cast<float>(head_dim));
    const float a = static_cast<float>(pos) * theta;
    out[i / 2] = make_float2(cosf(a), sinf(a));
  }
}

}  // namespace mcpm

using namespace mcpm;

namespace {

bool is_q8k_type(const mcpm_tensor* w) {
  return w && (w->t.type == MCPM_TYPE_Q4_K || w->t.type == MCPM_TYPE_Q6_K);
}

int set_state(mcpm_ctx* ctx, int token, int pos) {
  ctx->h_state->token = token;
  ctx->h_state->pos = pos;
  ctx->h_state->step = 0;
  ctx->h_state->n_out = 0;
  MCPM_HIP(hipMemcpyAsync(ctx->d_state, ctx->h_state, sizeof(StepState), hipMemcpyHostToDevice, ctx->stream));
  MCPM_HIP(hipStreamSynchronize(ctx->stream));
  return MCPM_OK;
}

GemvArgs single_region(const mcpm_tensor* w, float* out, int rows, int cols) {
  GemvArgs a{};
  a.reg[0] = GemvRegion{view_of(w->t), out, 0, rows};
  a.nreg = 1;
  a.total_rows = rows;
  a.nb = cols / QK_K;
  return a;
}

int check_q8k_gemv(const mcpm_tensor* w, int type, int rows, int cols, const char* fn) {
  if (!w) return fail(MCPM_ERR_ARG, std::string(fn) + ": null tensor");
  if (type >= 0 && w->t.type != type) return fail(MCPM_ERR_UNSUPPORTED, std::string(fn) + ": wrong tensor type");
  if (cols != w->t.cols || rows <= 0 || rows > w->t.rows || cols % QK_K || cols / QK_K > MAX_NB)
    return fail(MCPM_ERR_ARG, std::string(fn) + ": bad shape");
  return MCPM_OK;
}

// The single-kernel GEMV entries launch through here: with per-op timing on,
// the kernel records an event pair at its start and end (hipExtLaunchKernel).
template <class F>
hipError_t op_launch(mcpm_ctx* c, F&& launch) {
  if (!c->op_timing) return launch();
  if (c->op_used == c->op_events.size()) {
    std::pair<hipEvent_t, hipEvent_t> p{nullptr, nullptr};
    hipError_t err = hipEventCreate(&p.first);
    if (err == hipSuccess) err = hipEventCreate(&p.second);
    if (err != hipSuccess) {
      if (p.first) (void)hipEventDestroy(p.first);
      return err;
    }
    c->op_events.push_back(p);
  }
  const auto& p = c->op_events[c->op_used++];
  g_launch_timing = LaunchTiming{p.first, p.second};
  const hipError_t err = launch();
  g_launch_timing = LaunchTiming{};
  if (err != hipSuccess) --c->op_used;  // no kernel, no events to read
  return err;
}

}  // namespace

extern "C" {

const char* mcpm_last_error(void) { return g_last_error.c_str(); }

int mcpm_init(int device, mcpm_ctx** out) {
  if (!out) return fail(MCPM_ERR_ARG, "mcpm_init: null out");
  int n = 0;
  MCPM_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(MCPM_ERR_ARG, "mcpm_init: no such device");
  MCPM_HIP(hipSetDevice(device));
  auto* c = new mcpm_ctx();
  c->device = device;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipGetDeviceProperties");
  }
  c->n_cu = prop.multiProcessorCount;
  c->name = prop.gcnArchName;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->d_state, sizeof(StepState));
  if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->h_state), sizeof(StepState), hipHostMallocDefault);
  if (e == hipSuccess) e = hipMalloc(&c->d_rope, 512 * sizeof(float2));
  if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->h_rope), 512 * sizeof(float2), hipHostMallocDefault);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    mcpm_destroy(c);
    return hip_fail(e, "mcpm_init");
  }
  if (const int rc = noalloc_setup(device)) {
    mcpm_destroy(c);
    return rc;
  }
  c->rope_cap = 512;
  *out = c;
  return MCPM_OK;
}

void mcpm_destroy(mcpm_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  if (c->d_state) (void)hipFree(c->d_state);
  if (c->h_state) (void)hipHostFree(c->h_state);
  if (c->d_rope) (void)hipFree(c->d_rope);
  if (c->h_rope) (void)hipHostFree(c->h_rope);
  if (c->d_attn_part) (void)hipFree(c->d_attn_part);
  if (c->d_argmax_part) (void)hipFree(c->d_argmax_part);
  if (c->d_sample) (void)hipFree(c->d_sample);
  for (auto& p : c->op_events) {
    (void)hipEventDestroy(p.first);
    (void)hipEventDestroy(p.second);
  }
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

int mcpm_sync(mcpm_ctx* c) {
  if (!c) return fail(MCPM_ERR_ARG, "mcpm_sync: null ctx");
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_device_info(mcpm_ctx* c, int* n_cu, char* name, size_t name_len) {
  if (!c) return fail(MCPM_ERR_ARG, "mcpm_device_info: null ctx");
  if (n_cu) *n_cu = c->n_cu;
  if (name && name_len) std::snprintf(name, name_len, "%s", c->name.c_str());
  return MCPM_OK;
}

int mcpm_device_alloc(mcpm_ctx* c, size_t bytes, void** p) {
  if (!c || !p) return fail(MCPM_ERR_ARG, "mcpm_device_alloc: null argument");
  MCPM_HIP(hipMalloc(p, bytes ? bytes : 1));
  return MCPM_OK;
}

int mcpm_device_free(mcpm_ctx* c, void* p) {
  if (!c) return fail(MCPM_ERR_ARG, "mcpm_device_free: null ctx");
  if (p) MCPM_HIP(hipFree(p));
  return MCPM_OK;
}

int mcpm_copy_to_device(mcpm_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return fail(MCPM_ERR_ARG, "mcpm_copy_to_device: null argument");
  MCPM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_copy_to_host(mcpm_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return fail(MCPM_ERR_ARG, "mcpm_copy_to_host: null argument");
  MCPM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_copy_device(mcpm_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return fail(MCPM_ERR_ARG, "mcpm_copy_device: null argument");
  MCPM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_stream_read(mcpm_ctx* c, const void* src, size_t bytes, int grid, uint32_t* out) {
  if (!c || !src || !out) return fail(MCPM_ERR_ARG, "mcpm_stream_read: null argument");
  if (bytes == 0 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(MCPM_ERR_ARG, "mcpm_stream_read: bytes must be a positive multiple of 16 and src 16-byte aligned");
  if (grid < 1 || grid > 65536) return fail(MCPM_ERR_ARG, "mcpm_stream_read: grid must be 1 .. 65536");
  MCPM_HIP(op_launch(c, [&] { return launch_stream_read(src, bytes, grid, out, c->stream); }));
  return MCPM_OK;
}

int mcpm_fill_device(mcpm_ctx* c, void* dst, int v, size_t bytes) {
  if (!c || (!dst && bytes)) return fail(MCPM_ERR_ARG, "mcpm_fill_device: null argument");
  MCPM_HIP(hipMemsetAsync(dst, v, bytes, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

// ------------------------------------------------------------- tensors ----

int mcpm_tensor_upload(mcpm_ctx* c, const void* host, size_t bytes, int type, int64_t cols, int64_t rows,
                       mcpm_tensor** out) {
  if (!c || !out) return fail(MCPM_ERR_ARG, "mcpm_tensor_upload: null argument");
  auto* t = new mcpm_tensor();
  const int rc = upload_tensor(c, host, bytes, type, cols, rows, t->t);
  if (rc != MCPM_OK) {
    delete t;
    return rc;
  }
  *out = t;
  return MCPM_OK;
}

int mcpm_tensor_download(mcpm_ctx* c, const mcpm_tensor* t, void* host, size_t bytes) {
  if (!c || !t || !host) return fail(MCPM_ERR_ARG, "mcpm_tensor_download: null argument");
  if (bytes != t->t.bytes) return fail(MCPM_ERR_ARG, "mcpm_tensor_download: size mismatch");
  std::vector<uint8_t> img(bytes);
  MCPM_HIP(hipMemcpyAsync(img.data(), t->t.base, bytes, hipMemcpyDeviceToHost, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  repack_from_device_image(t->t.type, t->t.rows, t->t.cols, img.data(), static_cast<uint8_t*>(host));
  return MCPM_OK;
}

int mcpm_tensor_info(const mcpm_tensor* t, int* type, int64_t* cols, int64_t* rows) {
  if (!t) return fail(MCPM_ERR_ARG, "mcpm_tensor_info: null tensor");
  if (type) *type = t->t.type;
  if (cols) *cols = t->t.cols;
  if (rows) *rows = t->t.rows;
  return MCPM_OK;
}

void mcpm_tensor_free(mcpm_tensor* t) {
  if (!t) return;
  free_tensor(t->t);
  delete t;
}

int mcpm_tensor_dequantize_rows(mcpm_ctx* c, const mcpm_tensor* t, int64_t row0, int64_t n_rows, float* out) {
  if (!c || !t || !out) return fail(MCPM_ERR_ARG, "mcpm_tensor_dequantize_rows: null argument");
  if (row0 < 0 || n_rows <= 0 || row0 + n_rows > t->t.rows || n_rows > 65535)
    return fail(MCPM_ERR_ARG, "mcpm_tensor_dequantize_rows: bad row range");
  MCPM_HIP(launch_dequant_rows(view_of(t->t), static_cast<int>(row0), static_cast<int>(n_rows),
                               static_cast<int>(t->t.cols), out, c->stream));
  return MCPM_OK;
}

// -------------------------------------------------------------- per-op ----

int mcpm_set_op_timing(mcpm_ctx* c, int enable) {
  if (!c) return fail(MCPM_ERR_ARG, "mcpm_set_op_timing: null context");
  MCPM_HIP(hipStreamSynchronize(c->stream));
  c->op_timing = enable != 0;
  c->op_used = 0;
  return MCPM_OK;
}

int mcpm_op_time(mcpm_ctx* c, double* total_ms, int64_t* launches) {
  if (!c || !total_ms || !launches) return fail(MCPM_ERR_ARG, "mcpm_op_time: null argument");
  MCPM_HIP(hipStreamSynchronize(c->stream));
  double sum = 0.0;
  for (size_t i = 0; i < c->op_used; ++i) {
    float ms = 0.0f;
    MCPM_HIP(hipEventElapsedTime(&ms, c->op_events[i].first, c->op_events[i].second));
    sum += ms;
  }
  *total_ms = sum;
  *launches = static_cast<int64_t>(c->op_used);
  c->op_used = 0;
  return MCPM_OK;
}

int mcpm_quantize_row_q8_K(mcpm_ctx* c, const float* x, int n, void* y) {
  if (!c || !x || !y || n <= 0 || n % QK_K) return fail(MCPM_ERR_ARG, "mcpm_quantize_row_q8_K: bad argument");
  MCPM_HIP(launch_quantize_q8k(x, nullptr, 0.0f, n, PRO_QUANT_EVEN, static_cast<BlockQ8K*>(y), c->stream));
  return MCPM_OK;
}

int mcpm_gemv_q4_K_q8_K(mcpm_ctx* c, const mcpm_tensor* w, const void* xq, float* out, int rows, int cols) {
  if (!c || !xq || !out) return fail(MCPM_ERR_ARG, "mcpm_gemv_q4_K_q8_K: null argument");
  int rc = check_q8k_gemv(w, MCPM_TYPE_Q4_K, rows, cols, "mcpm_gemv_q4_K_q8_K");
  if (rc) return rc;
  GemvArgs a = single_region(w, out, rows, cols);
  a.xq = static_cast<const BlockQ8K*>(xq);
  MCPM_HIP(op_launch(c, [&] { return launch_gemv(a, PRO_Q8K, EPI_STORE, c->n_cu, c->stream); }));
  return MCPM_OK;
}

int mcpm_gemv_q6_K_q8_K(mcpm_ctx* c, const mcpm_tensor* w, const void* xq, float* out, int rows, int cols) {
  if (!c || !xq || !out) return fail(MCPM_ERR_ARG, "mcpm_gemv_q6_K_q8_K: null argument");
  int rc = check_q8k_gemv(w, MCPM_TYPE_Q6_K, rows, cols, "mcpm_gemv_q6_K_q8_K");
  if (rc) return rc;
  GemvArgs a = single_region(w, out, rows, cols);
  a.xq = static_cast<const BlockQ8K*>(xq);
  MCPM_HIP(op_launch(c, [&] { return launch_gemv(a, PRO_Q8K, EPI_STORE, c->n_cu, c->stream); }));
  return MCPM_OK;
}

int mcpm_gemv_qkv_q8_K(mcpm_ctx* c, const mcpm_tensor* wq, const mcpm_tensor* wk, const mcpm_tensor* wv,
                       const void* xq, float* q, float* k, float* v, int q_rows, int kv_rows, int cols) {
  if (!c || !xq || !q || !k || !v) return fail(MCPM_ERR_ARG, "mcpm_gemv_qkv_q8_K: null argument");
  int rc = check_q8k_gemv(wq, MCPM_TYPE_Q4_K, q_rows, cols, "mcpm_gemv_qkv_q8_K(q)");
  if (!rc) rc = check_q8k_gemv(wk, MCPM_TYPE_Q4_K, kv_rows, cols, "mcpm_gemv_qkv_q8_K(k)");
  if (!rc) rc = check_q8k_gemv(wv, -1, kv_rows, cols, "mcpm_gemv_qkv_q8_K(v)");
  if (rc) return rc;
  if (!is_q8k_type(wv)) {
    // matmul_qkv_q8k's fallback (src/ops/ops.cpp:394-403): zeros.
    MCPM_HIP(launch_fill_f32(q, 0.0f, q_rows, c->stream));
    MCPM_HIP(launch_fill_f32(k, 0.0f, kv_rows, c->stream));
    MCPM_HIP(launch_fill_f32(v, 0.0f, kv_rows, c->stream));
    return fail(MCPM_ERR_UNSUPPORTED, "mcpm_gemv_qkv_q8_K: v type not supported");
  }
  GemvArgs a{};
  a.reg[0] = GemvRegion{view_of(wq->t), q, 0, q_rows};
  a.reg[1] = GemvRegion{view_of(wk->t), k, q_rows, kv_rows};
  a.reg[2] = GemvRegion{view_of(wv->t), v, q_rows + kv_rows, kv_rows};
  a.nreg = 3;
  a.total_rows = q_rows + 2 * kv_rows;
  a.nb = cols / QK_K;
  a.xq = static_cast<const BlockQ8K*>(xq);
  MCPM_HIP(op_launch(c, [&] { return launch_gemv(a, PRO_Q8K, EPI_STORE, c->n_cu, c->stream); }));
  return MCPM_OK;
}

int mcpm_gemv_gate_up_q4_K_q8_K(mcpm_ctx* c, const mcpm_tensor* wg, const mcpm_tensor* wu, const void* xq,
                                float* gate, float* up, int rows, int cols) {
  if (!c || !xq || !gate || !up) return fail(MCPM_ERR_ARG, "mcpm_gemv_gate_up_q4_K_q8_K: null argument");
  int rc = check_q8k_gemv(wg, MCPM_TYPE_Q4_K, rows, cols, "mcpm_gemv_gate_up_q4_K_q8_K(gate)");
  if (!rc) rc = check_q8k_gemv(wu, MCPM_TYPE_Q4_K, rows, cols, "mcpm_gemv_gate_up_q4_K_q8_K(up)");
  if (rc) return rc;
  GemvArgs a{};
  a.reg[0] = GemvRegion{view_of(wg->t), gate, 0, rows};
  a.reg[1] = GemvRegion{view_of(wu->t), up, 0, rows};
  a.nreg = 2;
  a.pair = 1;
  a.total_rows = rows;
  a.nb = cols / QK_K;
  a.xq = static_cast<const BlockQ8K*>(xq);
  MCPM_HIP(op_launch(c, [&] { return launch_gemv(a, PRO_Q8K, EPI_STORE, c->n_cu, c->stream); }));
  return MCPM_OK;
}

static int gemv_f32act_q8k(mcpm_ctx* c, const mcpm_tensor* w, int type, const float* x, float* out, int rows,
                           int cols, const char* fn) {
  if (!c || !x || !out) return fail(MCPM_ERR_ARG, std::string(fn) + ": null argument");
  int rc = check_q8k_gemv(w, type, rows, cols, fn);
  if (rc) return rc;
  GemvArgs a = single_region(w, out, rows, cols);
  a.x = x;
  MCPM_HIP(op_launch(c, [&] { return launch_gemv(a, PRO_QUANT_EVEN, EPI_STORE, c->n_cu, c->stream); }));
  return MCPM_OK;
}

int mcpm_gemv_q4_K(mcpm_ctx* c, const mcpm_tensor* w, const float* x, float* out, int rows, int cols) {
  return gemv_f32act_q8k(c, w, MCPM_TYPE_Q4_K, x, out, rows, cols, "mcpm_gemv_q4_K");
}

int mcpm_gemv_q6_K(mcpm_ctx* c, const mcpm_tensor* w, const float* x, float* out, int rows, int cols) {
  return gemv_f32act_q8k(c, w, MCPM_TYPE_Q6_K, x, out, rows, cols, "mcpm_gemv_q6_K");
}

int mcpm_gemv_q8_0(mcpm_ctx* c, const mcpm_tensor* w, const float* x, float* out, int rows, int cols) {
  if (!c || !w || !x || !out) return fail(MCPM_ERR_ARG, "mcpm_gemv_q8_0: null argument");
  if (w->t.type != MCPM_TYPE_Q8_0) return fail(MCPM_ERR_UNSUPPORTED, "mcpm_gemv_q8_0: wrong tensor type");
  if (cols != w->t.cols || rows <= 0 || rows > w->t.rows) return fail(MCPM_ERR_ARG, "mcpm_gemv_q8_0: bad shape");
  MCPM_HIP(launch_gemv_q8_0(view_of(w->t), x, out, rows, cols, c->stream));
  return MCPM_OK;
}

int mcpm_gemv_f32(mcpm_ctx* c, const mcpm_tensor* w, const float* x, float* out, int rows, int cols) {
  if (!c || !w || !x || !out) return fail(MCPM_ERR_ARG, "mcpm_gemv_f32: null argument");
  if (w->t.type != MCPM_TYPE_F32) return fail(MCPM_ERR_UNSUPPORTED, "mcpm_gemv_f32: wrong tensor type");
  if (cols != w->t.cols || rows <= 0 || rows > w->t.rows) return fail(MCPM_ERR_ARG, "mcpm_gemv_f32: bad shape");
  MCPM_HIP(launch_gemv_f32(reinterpret_cast<const float*>(w->t.p0), x, out, rows, cols, c->stream));
  return MCPM_OK;
}

int mcpm_matmul(mcpm_ctx* c, const mcpm_tensor* w, const float* x, float* out) {
  if (!c || !w || !x || !out) return fail(MCPM_ERR_ARG, "mcpm_matmul: null argument");
  const int rows = static_cast<int>(w->t.rows), cols = static_cast<int>(w->t.cols);
  switch (w->t.type) {
    case MCPM_TYPE_F32: return mcpm_gemv_f32(c, w, x, out, rows, cols);
    case MCPM_TYPE_Q8_0: return mcpm_gemv_q8_0(c, w, x, out, rows, cols);
    case MCPM_TYPE_Q4_K: return mcpm_gemv_q4_K(c, w, x, out, rows, cols);
    case MCPM_TYPE_Q6_K: return mcpm_gemv_q6_K(c, w, x, out, rows, cols);
    default:
      MCPM_HIP(launch_fill_f32(out, 0.001f, rows, c->stream));
      return fail(MCPM_ERR_UNSUPPORTED, "mcpm_matmul: tensor type not implemented");
  }
}

int mcpm_matmul_q8k(mcpm_ctx* c, const mcpm_tensor* w, const void* xq, int num_cols, float* out) {
  if (!c || !w || !xq || !out) return fail(MCPM_ERR_ARG, "mcpm_matmul_q8k: null argument");
  const int rows = static_cast<int>(w->t.rows);
  if (w->t.type == MCPM_TYPE_Q4_K) return mcpm_gemv_q4_K_q8_K(c, w, xq, out, rows, num_cols);
  if (w->t.type == MCPM_TYPE_Q6_K) return mcpm_gemv_q6_K_q8_K(c, w, xq, out, rows, num_cols);
  MCPM_HIP(launch_fill_f32(out, 0.0f, rows, c->stream));
  return fail(MCPM_ERR_UNSUPPORTED, "mcpm_matmul_q8k: tensor type not supported");
}

int mcpm_rmsnorm(mcpm_ctx* c, float* out, const float* x, const float* w, int dim, float eps) {
  if (!c || !out || !x || !w || dim <= 0) return fail(MCPM_ERR_ARG, "mcpm_rmsnorm: bad argument");
  MCPM_HIP(launch_rmsnorm(x, w, eps, dim, out, c->stream));
  return MCPM_OK;
}

int mcpm_rmsnorm_and_quantize_q8k(mcpm_ctx* c, void* out, const float* x, const float* w, int dim, float eps) {
  if (!c || !out || !x || !w || dim <= 0 || dim % QK_K)
    return fail(MCPM_ERR_ARG, "mcpm_rmsnorm_and_quantize_q8k: bad argument");
  MCPM_HIP(launch_quantize_q8k(x, w, eps, dim, PRO_NORM_AWAY, static_cast<BlockQ8K*>(out), c->stream));
  return MCPM_OK;
}

int mcpm_swiglu_and_quantize_q8k(mcpm_ctx* c, void* out, const float* gate, const float* up, int dim) {
  if (!c || !out || !gate || !up || dim < 0) return fail(MCPM_ERR_ARG, "mcpm_swiglu_and_quantize_q8k: bad argument");
  if (dim < QK_K) return MCPM_OK;
  MCPM_HIP(launch_swiglu_quant(gate, up, dim, static_cast<BlockQ8K*>(out), c->stream));
  return MCPM_OK;
}

int mcpm_apply_rope(mcpm_ctx* c, float* vec, int pos, int n_heads, int head_dim, float base) {
  if (!c || !vec || n_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim / 2 > c->rope_cap || pos < 0)
    return fail(MCPM_ERR_ARG, "mcpm_apply_rope: bad argument");
  rope_row(pos, head_dim, base, c->h_rope);
  MCPM_HIP(hipMemcpyAsync(c->d_rope, c->h_rope, sizeof(float2) * (head_dim / 2), hipMemcpyHostToDevice, c->stream));
  MCPM_HIP(launch_rope(vec, c->d_rope, n_heads, head_dim, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_execute_attention(mcpm_ctx* c, float* out, const float* q, const float* k_cur, const float* v_cur,
                           float* k_cache, float* v_cache, int pos, int max_seq_len, int n_heads, int n_kv_heads,
                           int head_dim) {
  if (!c || !out || !q || !k_cur || !v_cur || !k_cache || !v_cache || pos < 0 || n_heads <= 0 ||
      n_kv_heads <= 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 8 || head_dim <= 0 || head_dim > 128 ||
      head_dim % 4 || n_kv_heads > 256)
    return fail(MCPM_ERR_ARG, "mcpm_execute_attention: bad argument");
  if (pos >= max_seq_len) return fail(MCPM_ERR_CONTEXT, "Maximum context exceeded (pos >= max_seq_len).");
  const int max_chunks = (max_seq_len + ATTN_CHUNK - 1) / ATTN_CHUNK;
  int rc = ensure_attn_scratch(c, static_cast<size_t>(n_heads) * max_chunks * (2 + head_dim));
  if (rc) return rc;
  rc = set_state(c, 0, pos);
  if (rc) return rc;
  const int kvd = n_kv_heads * head_dim;
  const int* st = reinterpret_cast<const int*>(c->d_state);
  MCPM_HIP(launch_kv_append(k_cur, v_cur, k_cache, v_cache, st, kvd, c->stream));
  const AttnPart part = attn_part_of(c->d_attn_part, n_heads, max_chunks, head_dim);
  MCPM_HIP(launch_attention(q, k_cache, v_cache, st, n_heads, n_kv_heads, head_dim, max_chunks, part, c->stream));
  MCPM_HIP(launch_attn_combine(part, st, n_heads, head_dim, max_chunks, out, c->stream));
  MCPM_HIP(hipStreamSynchronize(c->stream));
  return MCPM_OK;
}

int mcpm_get_embedding(mcpm_ctx* c, float* out, const mcpm_tensor* e, int token) {
  if (!c || !out || !e) return fail(MCPM_ERR_ARG, "mcpm_get_embedding: null argument");
  const int dim = static_cast<int>(e->t.cols);
  if (e->t.type != MCPM_TYPE_Q4_K && e->t.type != MCPM_TYPE_Q6_K) {
    MCPM_HIP(launch_fill_f32(out, 0.0f, dim, c->stream));
    return fail(MCPM_ERR_UNSUPPORTED, "get_embedding implemented for Q4_K and Q6_K only");
  }
  if (token < 0 || token >= e->t.rows) return fail(MCPM_ERR_ARG, "mcpm_get_embedding: token out of range");
  int rc = set_state(c, token, 0);
  if (rc) return rc;
  MCPM_HIP(launch_embedding(view_of(e->t), reinterpret_cast<const int*>(c->d_state), dim, out, c->stream));
  return MCPM_OK;
}

int mcpm_argmax(mcpm_ctx* c, const float* x, int n, int* out) {
  if (!c || !x || !out || n <= 0) return fail(MCPM_ERR_ARG, "mcpm_argmax: bad argument");
  const int nparts = std::min(1024, (n + 255) / 256);
  int rc = ensure_argmax_scratch(c, nparts);
  if (rc) return rc;
  MCPM_HIP(launch_argmax_partial(x, n, c->d_argmax_part, nparts, c->stream));
  MCPM_HIP(launch_argmax_final(c->d_argmax_part, nparts, out, nullptr, nullptr, c->stream));
  return MCPM_OK;
}

int mcpm_sample_device(mcpm_ctx* c, const float* logits, int n, float temperature, float top_p, float r, int* out) {
  if (!c || !logits || !out || n <= 0 || n > sampler_max_n() || !(r >= 0.0f && r < 1.0f))
    return fail(MCPM_ERR_ARG, "mcpm_sample_device: bad argument");
  const size_t need = sampler_bytes(n);
  if (need > c->sample_cap) {
    if (c->d_sample) (void)hipFree(c->d_sample);
    c->d_sample = nullptr;
    c->sample_cap = 0;
    MCPM_HIP(hipMalloc(&c->d_sample, need));
    // the sampler's bucket masses and gather count start at zero (each call
    // leaves them so)
    MCPM_HIP(hipMemsetAsync(c->d_sample, 0, need, c->stream));
    c->sample_cap = need;
  }
  MCPM_HIP(launch_sample(c->d_sample, c->sample_cap, logits, n, temperature, top_p, r, out, nullptr, nullptr,
                         c->stream));
  return MCPM_OK;
}

}  // extern "C"
