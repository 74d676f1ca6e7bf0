// synth.cpp -- deterministic random-init models and ggml block encoders.
//
// The reference only decodes llama.cpp-made blocks; it has no encoder.  These
// encoders write valid Q4_K / Q6_K / Q8_0 blocks from fp32 rows with a simple
// per-block min/max (Q4_K) or absmax (Q6_K, Q8_0) fit.  Both the device path
// and the CPU oracle consume the same bytes, so the encoder's choices never
// enter a parity comparison.  Built without fast-math, so every machine
// produces identical bytes from the same seed.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "gguf.h"
#include "mcpm_internal.h"

namespace mcpm {

uint16_t fp32_to_fp16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    float v;
    std::memcpy(&v, &ax, 4);
    const uint32_t m = static_cast<uint32_t>(std::rint(v * 16777216.0f));
    return static_cast<uint16_t>(sign | m);
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return static_cast<uint16_t>(sign | h);
}

namespace {

uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001b3ull;
  }
  return h;
}

// Element i of stream (seed, tensor): Box-Muller on two uniforms in (0,1].
inline double uniform01(uint64_t key, uint64_t i) {
  return (static_cast<double>(splitmix64(key + i) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void normals(uint64_t seed, uint64_t tensor, double mean, double stddev, float* out, size_t begin, size_t n) {
  const uint64_t key = splitmix64(seed ^ splitmix64(tensor));
  const double two_pi = 6.283185307179586476925286766559;
  const size_t end = begin + n;
  for (size_t pair = begin / 2; 2 * pair < end; ++pair) {
    const double u1 = uniform01(key, 2 * pair), u2 = uniform01(key, 2 * pair + 1);
    const double rad = std::sqrt(-2.0 * std::log(u1));
    const size_t i0 = 2 * pair, i1 = 2 * pair + 1;
    if (i0 >= begin) out[i0 - begin] = static_cast<float>(mean + stddev * (rad * std::cos(two_pi * u2)));
    if (i1 >= begin && i1 < end) out[i1 - begin] = static_cast<float>(mean + stddev * (rad * std::sin(two_pi * u2)));
  }
}

template <class F>
void parallel_for(int64_t n, F&& f) {
  unsigned nt = std::thread::hardware_concurrency();
  if (const char* e = std::getenv("OMP_NUM_THREADS")) nt = static_cast<unsigned>(std::max(1, std::atoi(e)));
  nt = std::max(1u, std::min<unsigned>(nt, 64u));
  if (n < 64 || nt == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  const int64_t chunk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const int64_t b = t * chunk, e = std::min<int64_t>(n, b + chunk);
    if (b >= e) break;
    th.emplace_back([&f, b, e] { f(b, e); });
  }
  for (auto& t : th) t.join();
}

inline float fp16f(uint16_t h) { return fp16_to_fp32(h); }

void encode_q8_0(const float* x, BlockQ8_0* out) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
  const uint16_t dh = fp32_to_fp16(amax / 127.0f);
  const float d = fp16f(dh);
  out->d = dh;
  for (int i = 0; i < 32; ++i) {
    const float q = d > 0.0f ? std::round(x[i] / d) : 0.0f;
    out->qs[i] = static_cast<int8_t>(std::max(-127.0f, std::min(127.0f, q)));
  }
}

void encode_q4_K(const float* x, BlockQ4K* out) {
  float scale[8], minv[8];
  for (int j = 0; j < 8; ++j) {
    float lo = 0.0f, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      lo = std::min(lo, x[32 * j + i]);
      hi = std::max(hi, x[32 * j + i]);
    }
    hi = std::max(hi, lo);
    scale[j] = (hi - lo) / 15.0f;
    minv[j] = -lo;
  }
  float ms = 0.0f, mm = 0.0f;
  for (int j = 0; j < 8; ++j) {
    ms = std::max(ms, scale[j]);
    mm = std::max(mm, minv[j]);
  }
  const uint16_t dh = fp32_to_fp16(ms / 63.0f), mh = fp32_to_fp16(mm / 63.0f);
  const float d = fp16f(dh), dmin = fp16f(mh);
  uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.0f ? static_cast<uint8_t>(std::max(0.0f, std::min(63.0f, std::round(scale[j] / d)))) : 0;
    mn[j] = dmin > 0.0f ? static_cast<uint8_t>(std::max(0.0f, std::min(63.0f, std::round(minv[j] / dmin)))) : 0;
  }
  out->d = dh;
  out->dmin = mh;
  for (int j = 0; j < 4; ++j) {
    out->scales[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    out->scales[j + 4] = static_cast<uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
    out->scales[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
  }
  std::memset(out->qs, 0, sizeof(out->qs));
  for (int e = 0; e < 256; ++e) {
    const int j = e / 32;
    const float es = d * static_cast<float>(sc[j]), em = dmin * static_cast<float>(mn[j]);
    int q = 0;
    if (es > 0.0f) q = static_cast<int>(std::max(0.0f, std::min(15.0f, std::round((x[e] + em) / es))));
    const int c = e / 64, l = e % 32, hi = (e % 64) >= 32;
    out->qs[32 * c + l] |= static_cast<uint8_t>(hi ? (q << 4) : q);
  }
}

void encode_q6_K(const float* x, BlockQ6K* out) {
  float scale[16];
  float ms = 0.0f;
  for (int j = 0; j < 16; ++j) {
    float amax = 0.0f;
    for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * j + i]));
    scale[j] = amax / 31.0f;
    ms = std::max(ms, scale[j]);
  }
  const uint16_t dh = fp32_to_fp16(ms / 127.0f);
  const float d = fp16f(dh);
  int sc[16];
  for (int j = 0; j < 16; ++j) {
    sc[j] = d > 0.0f ? static_cast<int>(std::max(-128.0f, std::min(127.0f, std::round(scale[j] / d)))) : 0;
    out->scales[j] = static_cast<int8_t>(sc[j]);
  }
  out->d = dh;
  std::memset(out->ql, 0, sizeof(out->ql));
  std::memset(out->qh, 0, sizeof(out->qh));
  for (int e = 0; e < 256; ++e) {
    const float es = d * static_cast<float>(sc[e / 16]);
    int q = 32;
    if (es != 0.0f) q = static_cast<int>(std::max(-32.0f, std::min(31.0f, std::round(x[e] / es)))) + 32;
    const int h = e / 128, r = e % 128, g = r / 32, l = r % 32;
    const int qi = 64 * h + 32 * (g & 1) + l;
    out->ql[qi] |= static_cast<uint8_t>(g < 2 ? (q & 15) : ((q & 15) << 4));
    out->qh[32 * h + l] |= static_cast<uint8_t>(((q >> 4) & 3) << (2 * g));
  }
}

}  // namespace

size_t type_row_bytes(int type, int64_t cols) { return gguf_tensor_bytes(type, {static_cast<uint64_t>(cols), 1}); }

int type_block_elems(int type) {
  switch (type) {
    case MCPM_TYPE_F32: return 1;
    case MCPM_TYPE_Q8_0: return 32;
    case MCPM_TYPE_Q4_K:
    case MCPM_TYPE_Q6_K: return 256;
    default: return 0;
  }
}

static void quantize_rows_impl(int type, const float* src, int64_t rows, int64_t cols, uint8_t* dst) {
  const size_t rb = type_row_bytes(type, cols);
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = src + r * cols;
    uint8_t* o = dst + r * rb;
    if (type == MCPM_TYPE_F32) {
      std::memcpy(o, x, cols * 4);
    } else if (type == MCPM_TYPE_Q8_0) {
      for (int64_t b = 0; b < cols / 32; ++b) encode_q8_0(x + 32 * b, reinterpret_cast<BlockQ8_0*>(o) + b);
    } else if (type == MCPM_TYPE_Q4_K) {
      for (int64_t b = 0; b < cols / 256; ++b) encode_q4_K(x + 256 * b, reinterpret_cast<BlockQ4K*>(o) + b);
    } else if (type == MCPM_TYPE_Q6_K) {
      for (int64_t b = 0; b < cols / 256; ++b) encode_q6_K(x + 256 * b, reinterpret_cast<BlockQ6K*>(o) + b);
    }
  }
}

// A vocabulary of n strings for tokenizer.ggml.tokens, the key the reference's
// tokenizer reads (src/tokenizer.cpp:10-60): a few chat control tokens, the
// 256 byte tokens "<0xHH>", one token per byte in GPT-2's byte-to-unicode
// mapping (printable bytes 33-126, 161-172, 174-255 as themselves, the other
// 68 bytes as code points 256, 257, ... in byte order), so that any text
// tokenizes, then distinct filler strings.  The words carry no meaning: the
// weights are random.
std::vector<std::string> synth_vocabulary(int n) {
  std::vector<std::string> v = {"<unk>", "<s>", "</s>", "<|im_start|>", "<|im_end|>", "<think>", "</think>",
                                "<tool_call>", "</tool_call>", "/think", "/no_think"};
  char buf[16];
  for (int b = 0; b < 256; ++b) {
    std::snprintf(buf, sizeof buf, "<0x%02X>", b);
    v.emplace_back(buf);
  }
  auto utf8 = [](uint32_t cp) {
    std::string s;
    if (cp < 0x80) {
      s += static_cast<char>(cp);
    } else {  // every code point here is below 0x800
      s += static_cast<char>(0xC0 | (cp >> 6));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    }
    return s;
  };
  uint32_t next = 256;
  for (int b = 0; b < 256; ++b) {
    const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174);
    v.push_back(utf8(printable ? static_cast<uint32_t>(b) : next++));
  }
  for (int i = static_cast<int>(v.size()); i < n; ++i) v.push_back("w" + std::to_string(i));
  v.resize(static_cast<size_t>(n));
  return v;
}

}  // namespace mcpm

using namespace mcpm;

extern "C" {

void mcpm_synth_normal(uint64_t seed, uint64_t tensor_id, float mean, float stddev, float* out, size_t n) {
  parallel_for(static_cast<int64_t>((n + 4095) / 4096), [&](int64_t b, int64_t e) {
    for (int64_t c = b; c < e; ++c) {
      const size_t s = static_cast<size_t>(c) * 4096, k = std::min<size_t>(4096, n - s);
      normals(seed, tensor_id, mean, stddev, out + s, s, k);
    }
  });
}

size_t mcpm_type_row_bytes(int ggml_type, int64_t cols) { return type_row_bytes(ggml_type, cols); }

int mcpm_quantize_rows(int ggml_type, const float* src, int64_t rows, int64_t cols, void* dst) {
  const int be = type_block_elems(ggml_type);
  if (!src || !dst || rows < 0 || be == 0 || cols % be != 0) return MCPM_ERR_ARG;
  const size_t rb = type_row_bytes(ggml_type, cols);
  parallel_for(rows, [&](int64_t b, int64_t e) {
    quantize_rows_impl(ggml_type, src + b * cols, e - b, cols, static_cast<uint8_t*>(dst) + b * rb);
  });
  return MCPM_OK;
}

void mcpm_free_host(void* p) { std::free(p); }

int mcpm_synth_gguf(const mcpm_model_config* cfg, uint64_t seed, int mix, const char* path, void** image,
                    size_t* image_bytes) {
  if (!cfg || mix < 0 || mix > 2 || cfg->n_layers <= 0 || cfg->dim % 256 || cfg->ffn <= 0 || cfg->vocab <= 0 ||
      cfg->n_heads <= 0 ||
      cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads || cfg->head_dim <= 0 || cfg->head_dim % 2)
    return fail(MCPM_ERR_ARG, "mcpm_synth_gguf: invalid config");
  const int ffn_pad = (cfg->ffn + 255) / 256 * 256;
  const int qd = cfg->n_heads * cfg->head_dim, kvd = cfg->n_kv_heads * cfg->head_dim;
  if (qd % 256) return fail(MCPM_ERR_ARG, "mcpm_synth_gguf: n_heads*head_dim must be a multiple of 256");
  const uint32_t Q4 = MCPM_TYPE_Q4_K, Q6 = MCPM_TYPE_Q6_K, F32 = MCPM_TYPE_F32;
  const uint64_t D = cfg->dim;

  GgufWriter w;
  w.kv_str("general.architecture", "llama");
  w.kv_str("general.name", "minicpm5-synthetic");
  w.kv_u32("general.alignment", 32);
  w.kv_u32("llama.block_count", cfg->n_layers);
  w.kv_u32("llama.embedding_length", cfg->dim);
  w.kv_u32("llama.feed_forward_length", cfg->ffn);
  w.kv_u32("llama.attention.head_count", cfg->n_heads);
  w.kv_u32("llama.attention.head_count_kv", cfg->n_kv_heads);
  w.kv_u32("llama.attention.key_length", cfg->head_dim);
  w.kv_u32("llama.attention.value_length", cfg->head_dim);
  w.kv_u32("llama.rope.dimension_count", cfg->head_dim);
  w.kv_f32("llama.rope.freq_base", cfg->rope_base);
  w.kv_f32("llama.attention.layer_norm_rms_epsilon", cfg->eps);
  w.kv_u32("llama.vocab_size", cfg->vocab);
  w.kv_u32("general.seed_lo", static_cast<uint32_t>(seed));
  w.kv_u32("general.quant_mix", static_cast<uint32_t>(mix));

  const uint64_t V = static_cast<uint64_t>(cfg->vocab);
  const int n = cfg->n_layers;
  // llama.cpp's use_more_bits rule for mix 1 and 2; mix 0 gives every layer Q6_K v/down.
  auto v_type = [&](int l) {
    const bool more = (l < n / 8) || (l >= 7 * n / 8) || ((l - n / 8) % 3 == 2);
    return (mix == 0 || more) ? Q6 : Q4;
  };
  if (mix == 2) {
    // The reference's own file (include/minicpm_metadata.h:30-32 and the
    // tensor table after it): an untied Q6_K output.weight, a Q4_K
    // token_embd.weight, and per layer the tensors in name order; plus the
    // vocabulary its tokenizer reads.
    w.kv_str("tokenizer.ggml.model", "gpt2");
    w.kv_str_array("tokenizer.ggml.tokens", synth_vocabulary(cfg->vocab));
    w.add_tensor("output.weight", Q6, {D, V});
    w.add_tensor("output_norm.weight", F32, {D});
    w.add_tensor("token_embd.weight", Q4, {D, V});
    for (int l = 0; l < n; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      w.add_tensor(p + "attn_k.weight", Q4, {D, static_cast<uint64_t>(kvd)});
      w.add_tensor(p + "attn_norm.weight", F32, {D});
      w.add_tensor(p + "attn_output.weight", Q4, {static_cast<uint64_t>(qd), D});
      w.add_tensor(p + "attn_q.weight", Q4, {D, static_cast<uint64_t>(qd)});
      w.add_tensor(p + "attn_v.weight", v_type(l), {D, static_cast<uint64_t>(kvd)});
      w.add_tensor(p + "ffn_down.weight", v_type(l), {static_cast<uint64_t>(ffn_pad), D});
      w.add_tensor(p + "ffn_gate.weight", Q4, {D, static_cast<uint64_t>(cfg->ffn)});
      w.add_tensor(p + "ffn_norm.weight", F32, {D});
      w.add_tensor(p + "ffn_up.weight", Q4, {D, static_cast<uint64_t>(cfg->ffn)});
    }
  } else {
    // The LM head is the token embedding (tied), stored Q6_K.
    w.add_tensor("token_embd.weight", Q6, {D, V});
    w.add_tensor("output_norm.weight", F32, {D});
    if (!cfg->tied_embeddings) w.add_tensor("output.weight", Q6, {D, V});
    for (int l = 0; l < n; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      w.add_tensor(p + "attn_norm.weight", F32, {D});
      w.add_tensor(p + "attn_q.weight", Q4, {D, static_cast<uint64_t>(qd)});
      w.add_tensor(p + "attn_k.weight", Q4, {D, static_cast<uint64_t>(kvd)});
      w.add_tensor(p + "attn_v.weight", v_type(l), {D, static_cast<uint64_t>(kvd)});
      w.add_tensor(p + "attn_output.weight", Q4, {static_cast<uint64_t>(qd), D});
      w.add_tensor(p + "ffn_norm.weight", F32, {D});
      w.add_tensor(p + "ffn_gate.weight", Q4, {D, static_cast<uint64_t>(cfg->ffn)});
      w.add_tensor(p + "ffn_up.weight", Q4, {D, static_cast<uint64_t>(cfg->ffn)});
      w.add_tensor(p + "ffn_down.weight", v_type(l), {static_cast<uint64_t>(ffn_pad), D});
    }
  }
  std::vector<size_t> offs;
  if (mix == 2 && cfg->n_layers == 42 && cfg->dim == 2048 && cfg->n_heads == 16 && cfg->n_kv_heads == 2 &&
      cfg->head_dim == 128 && cfg->ffn == 6144 && cfg->vocab == 130560) {
    // At the reference's own geometry the tensor data starts where it starts
    // in the reference's file (output.weight at 5,145,568,
    // include/minicpm_metadata.h:30), so the tensor offsets compiled into the
    // reference (TENSORS_INFO) address this file's tensors: one string
    // key/value pads the header to that length.
    constexpr size_t kRefDataStart = 5145568;
    const std::string key = "general.padding";
    const size_t entry = 8 + key.size() + 4 + 8;  // key length, key, type, string length
    const size_t h = w.layout(offs) - [&] {
      size_t data = 0;
      for (const auto& t : w.tensors()) data += (t.bytes + 31) / 32 * 32;
      return data;
    }();
    if (h + entry > kRefDataStart) return fail(MCPM_ERR_ARG, "mcpm_synth_gguf: header too large to pad");
    w.kv_str(key, std::string(kRefDataStart - h - entry, ' '));
  }
  const size_t total = w.layout(offs);
  uint8_t* img = static_cast<uint8_t*>(std::calloc(total, 1));
  if (!img) return fail(MCPM_ERR_NOMEM, "mcpm_synth_gguf: host allocation failed");
  w.write_header(img);

  const auto& ts = w.tensors();
  for (size_t i = 0; i < ts.size(); ++i) {
    const GgufTensor& t = ts[i];
    const uint64_t tid = fnv1a(t.name);
    const int64_t cols = static_cast<int64_t>(t.dims[0]);
    const int64_t rows = t.dims.size() > 1 ? static_cast<int64_t>(t.dims[1]) : 1;
    const bool is_norm = t.name.find("norm") != std::string::npos;
    const bool is_down = t.name.find("ffn_down") != std::string::npos;
    const size_t rb = type_row_bytes(t.type, cols);
    uint8_t* dst = img + offs[i];
    parallel_for((rows + 15) / 16, [&](int64_t b, int64_t e) {
      std::vector<float> buf(static_cast<size_t>(16 * cols));
      for (int64_t c = b; c < e; ++c) {
        const int64_t r0 = c * 16, nr = std::min<int64_t>(16, rows - r0);
        for (int64_t r = 0; r < nr; ++r) {
          float* row = buf.data() + r * cols;
          // ffn_down: columns >= ffn are padding and hold zeros.
          const int64_t real = is_down ? cfg->ffn : cols;
          normals(seed, tid, is_norm ? 1.0 : 0.0, is_norm ? 0.1 : 0.02, row,
                  static_cast<size_t>((r0 + r) * real), static_cast<size_t>(real));
          for (int64_t k = real; k < cols; ++k) row[k] = 0.0f;
        }
        quantize_rows_impl(static_cast<int>(t.type), buf.data(), nr, cols, dst + r0 * rb);
      }
    });
  }

  if (path) {
    FILE* f = std::fopen(path, "wb");
    if (!f) {
      std::free(img);
      return fail(MCPM_ERR_IO, std::string("mcpm_synth_gguf: cannot open ") + path);
    }
    const size_t wr = std::fwrite(img, 1, total, f);
    std::fclose(f);
    std::free(img);
    if (wr != total) return fail(MCPM_ERR_IO, "mcpm_synth_gguf: short write");
    if (image_bytes) *image_bytes = total;
    if (image) *image = nullptr;
    return MCPM_OK;
  }
  if (!image) {
    std::free(img);
    return fail(MCPM_ERR_ARG, "mcpm_synth_gguf: need a path or an image pointer");
  }
  *image = img;
  if (image_bytes) *image_bytes = total;
  return MCPM_OK;
}

}  // extern "C"
