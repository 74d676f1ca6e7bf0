// gguf.cpp -- GGUF v3 reader and writer (host).
#include "gguf.h"

#include <cstring>

namespace mcpm {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian

struct Reader {
  const uint8_t* p;
  size_t n, off = 0;
  bool ok = true;
  bool take(void* dst, size_t k) {
    if (!ok || off + k > n) return ok = false;
    std::memcpy(dst, p + off, k);
    off += k;
    return true;
  }
  template <class T>
  T get() {
    T v{};
    take(&v, sizeof(T));
    return v;
  }
  bool str(std::string& s) {
    const uint64_t len = get<uint64_t>();
    if (!ok || len > n - off) return ok = false;
    s.assign(reinterpret_cast<const char*>(p + off), len);
    off += len;
    return true;
  }
};

size_t scalar_size(uint32_t t) {
  switch (t) {
    case GGUF_UINT8: case GGUF_INT8: case GGUF_BOOL: return 1;
    case GGUF_UINT16: case GGUF_INT16: return 2;
    case GGUF_UINT32: case GGUF_INT32: case GGUF_FLOAT32: return 4;
    case GGUF_UINT64: case GGUF_INT64: case GGUF_FLOAT64: return 8;
    default: return 0;
  }
}

bool read_scalar(Reader& r, uint32_t t, GgufValue& v) {
  v.type = t;
  switch (t) {
    case GGUF_UINT8: v.inum = r.get<uint8_t>(); break;
    case GGUF_INT8: v.inum = r.get<int8_t>(); break;
    case GGUF_BOOL: v.inum = r.get<uint8_t>(); break;
    case GGUF_UINT16: v.inum = r.get<uint16_t>(); break;
    case GGUF_INT16: v.inum = r.get<int16_t>(); break;
    case GGUF_UINT32: v.inum = r.get<uint32_t>(); break;
    case GGUF_INT32: v.inum = r.get<int32_t>(); break;
    case GGUF_UINT64: v.inum = static_cast<int64_t>(r.get<uint64_t>()); break;
    case GGUF_INT64: v.inum = r.get<int64_t>(); break;
    case GGUF_FLOAT32: v.num = r.get<float>(); v.inum = static_cast<int64_t>(v.num); return r.ok;
    case GGUF_FLOAT64: v.num = r.get<double>(); v.inum = static_cast<int64_t>(v.num); return r.ok;
    default: return false;
  }
  v.num = static_cast<double>(v.inum);
  return r.ok;
}

}  // namespace

size_t gguf_tensor_bytes(uint32_t type, const std::vector<uint64_t>& dims) {
  if (dims.empty()) return 0;
  // every product is checked against 2^62 so no step wraps (0: not a valid size)
  constexpr uint64_t kLimit = uint64_t{1} << 62;
  uint64_t rows = 1;
  for (size_t i = 1; i < dims.size(); ++i) {
    if (dims[i] != 0 && rows > kLimit / dims[i]) return 0;
    rows *= dims[i];
  }
  const uint64_t cols = dims[0];
  uint64_t per_row = 0;  // bytes of one row
  switch (type) {
    case 0: per_row = cols > kLimit / 4 ? 0 : cols * 4; break;
    case 1: per_row = cols > kLimit / 2 ? 0 : cols * 2; break;
    case 8: per_row = cols % 32 ? 0 : cols / 32 * 34; break;
    case 12: per_row = cols % 256 ? 0 : cols / 256 * 144; break;
    case 14: per_row = cols % 256 ? 0 : cols / 256 * 210; break;
    default: return 0;
  }
  if (rows != 0 && per_row > kLimit / rows) return 0;
  return static_cast<size_t>(per_row * rows);
}

const GgufTensor* GgufFile::find(const std::string& name) const {
  for (const auto& t : tensors)
    if (t.name == name) return &t;
  return nullptr;
}

bool GgufFile::get_int(const std::string& key, int64_t& out) const {
  auto it = kv.find(key);
  if (it == kv.end() || it->second.type == GGUF_STRING || it->second.type == GGUF_ARRAY) return false;
  out = it->second.inum;
  return true;
}

bool GgufFile::get_float(const std::string& key, double& out) const {
  auto it = kv.find(key);
  if (it == kv.end() || it->second.type == GGUF_STRING || it->second.type == GGUF_ARRAY) return false;
  out = it->second.num;
  return true;
}

bool GgufFile::get_str(const std::string& key, std::string& out) const {
  auto it = kv.find(key);
  if (it == kv.end() || it->second.type != GGUF_STRING) return false;
  out = it->second.str;
  return true;
}

bool gguf_parse(const uint8_t* data, size_t size, GgufFile& out, std::string& err) {
  Reader r{data, size};
  if (r.get<uint32_t>() != kMagic || !r.ok) {
    err = "not a GGUF file (bad magic)";
    return false;
  }
  out.version = r.get<uint32_t>();
  if (out.version < 2 || out.version > 3) {
    err = "unsupported GGUF version " + std::to_string(out.version);
    return false;
  }
  const uint64_t n_tensors = r.get<uint64_t>();
  const uint64_t n_kv = r.get<uint64_t>();
  if (!r.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) {
    err = "truncated or implausible GGUF header";
    return false;
  }
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key;
    if (!r.str(key)) break;
    GgufValue v;
    v.type = r.get<uint32_t>();
    if (v.type == GGUF_STRING) {
      r.str(v.str);
    } else if (v.type == GGUF_ARRAY) {
      v.arr_type = r.get<uint32_t>();
      v.arr_len = r.get<uint64_t>();
      if (v.arr_type == GGUF_STRING) {
        if (v.arr_len > (size - r.off) / 8) {  // each string takes at least its 8-byte length
          err = "bad array in key " + key;
          return false;
        }
        v.strs.reserve(v.arr_len);
        for (uint64_t k = 0; k < v.arr_len && r.ok; ++k) {
          std::string tmp;
          r.str(tmp);
          v.strs.push_back(std::move(tmp));
        }
      } else {
        const size_t es = scalar_size(v.arr_type);
        if (es == 0 || v.arr_len > (size - r.off) / es) {
          err = "bad array in key " + key;
          return false;
        }
        r.off += es * v.arr_len;
      }
    } else if (!read_scalar(r, v.type, v)) {
      err = "bad value type for key " + key;
      return false;
    }
    if (!r.ok) break;
    out.kv[key] = v;
  }
  if (!r.ok) {
    err = "truncated GGUF key/value section";
    return false;
  }
  auto al = out.kv.find("general.alignment");
  if (al != out.kv.end() && al->second.inum > 0) out.alignment = static_cast<uint64_t>(al->second.inum);
  out.tensors.resize(n_tensors);
  for (auto& t : out.tensors) {
    r.str(t.name);
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok || nd == 0 || nd > 4) {
      err = "bad tensor dims in table";
      return false;
    }
    t.dims.resize(nd);
    for (auto& d : t.dims) d = r.get<uint64_t>();
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (!r.ok) {
      err = "truncated tensor table";
      return false;
    }
  }
  const uint64_t data_start = (r.off + out.alignment - 1) / out.alignment * out.alignment;
  if (data_start > size) {
    err = "truncated GGUF: no data section";
    return false;
  }
  for (auto& t : out.tensors) {
    t.bytes = gguf_tensor_bytes(t.type, t.dims);
    // in this order no sum can wrap: offset and size each checked against
    // what is left of the file
    if (t.offset > size - data_start || t.bytes > size - data_start - t.offset) {
      err = "tensor " + t.name + " extends past the end of the file";
      return false;
    }
    t.data = data + data_start + t.offset;
  }
  return true;
}

// ------------------------------------------------------------------ writer

void GgufWriter::kv_u32(const std::string& k, uint32_t v) {
  GgufValue x;
  x.type = GGUF_UINT32;
  x.inum = v;
  kv_.emplace_back(k, x);
}
void GgufWriter::kv_f32(const std::string& k, float v) {
  GgufValue x;
  x.type = GGUF_FLOAT32;
  x.num = v;
  kv_.emplace_back(k, x);
}
void GgufWriter::kv_str(const std::string& k, const std::string& v) {
  GgufValue x;
  x.type = GGUF_STRING;
  x.str = v;
  kv_.emplace_back(k, x);
}

void GgufWriter::kv_str_array(const std::string& k, const std::vector<std::string>& v) {
  GgufValue x;
  x.type = GGUF_ARRAY;
  x.arr_type = GGUF_STRING;
  x.arr_len = v.size();
  x.strs = v;
  kv_.emplace_back(k, x);
}

void GgufWriter::add_tensor(const std::string& name, uint32_t type, const std::vector<uint64_t>& dims) {
  GgufTensor t;
  t.name = name;
  t.type = type;
  t.dims = dims;
  t.bytes = gguf_tensor_bytes(type, dims);
  tensors_.push_back(t);
}

size_t GgufWriter::layout(std::vector<size_t>& abs) {
  const uint64_t align = 32;
  size_t h = 4 + 4 + 8 + 8;
  for (const auto& kv : kv_) {
    h += 8 + kv.first.size() + 4;
    if (kv.second.type == GGUF_STRING) {
      h += 8 + kv.second.str.size();
    } else if (kv.second.type == GGUF_ARRAY) {
      h += 4 + 8;
      for (const auto& e : kv.second.strs) h += 8 + e.size();
    } else {
      h += scalar_size(kv.second.type);
    }
  }
  for (const auto& t : tensors_) h += 8 + t.name.size() + 4 + 8 * t.dims.size() + 4 + 8;
  header_bytes_ = h;
  const size_t data_start = (h + align - 1) / align * align;
  size_t off = 0;
  abs.clear();
  for (auto& t : tensors_) {
    t.offset = off;
    abs.push_back(data_start + off);
    off += (t.bytes + align - 1) / align * align;
  }
  return data_start + off;
}

void GgufWriter::write_header(uint8_t* image) const {
  size_t o = 0;
  auto put = [&](const void* src, size_t k) {
    std::memcpy(image + o, src, k);
    o += k;
  };
  auto put_str = [&](const std::string& s) {
    const uint64_t len = s.size();
    put(&len, 8);
    put(s.data(), s.size());
  };
  const uint32_t magic = kMagic, version = 3;
  const uint64_t nt = tensors_.size(), nkv = kv_.size();
  put(&magic, 4);
  put(&version, 4);
  put(&nt, 8);
  put(&nkv, 8);
  for (const auto& kv : kv_) {
    put_str(kv.first);
    put(&kv.second.type, 4);
    if (kv.second.type == GGUF_STRING) {
      put_str(kv.second.str);
    } else if (kv.second.type == GGUF_ARRAY) {
      const uint32_t at = GGUF_STRING;
      const uint64_t n = kv.second.strs.size();
      put(&at, 4);
      put(&n, 8);
      for (const auto& e : kv.second.strs) put_str(e);
    } else if (kv.second.type == GGUF_FLOAT32) {
      const float f = static_cast<float>(kv.second.num);
      put(&f, 4);
    } else if (kv.second.type == GGUF_UINT32) {
      const uint32_t u = static_cast<uint32_t>(kv.second.inum);
      put(&u, 4);
    }
  }
  for (const auto& t : tensors_) {
    put_str(t.name);
    const uint32_t nd = static_cast<uint32_t>(t.dims.size());
    put(&nd, 4);
    for (uint64_t d : t.dims) put(&d, 8);
    put(&t.type, 4);
    put(&t.offset, 8);
  }
  while (o % 32) image[o++] = 0;
}

}  // namespace mcpm
