// GGUF reader (host code): the container the reference loads quantized
// models from (weight_loading/gguf.rs:49-151, 551-591), mapped read-only so
// the K-quant decoder can upload a tensor's block bytes straight into its
// device layout instead of dequantizing them first.
//
// Layout (GGUF v2/v3, little-endian): magic "GGUF" (u32 0x46554747), version
// (u32), tensor count (u64), metadata count (u64); metadata entries (string
// key, u32 value type, value; arrays nest); tensor infos (string name, u32
// n_dims, u64 dims[n_dims], u32 ggml type, u64 offset); tensor data from the
// first 32-byte boundary after the infos (the reference always uses the
// default alignment of 32; this reader also honours general.alignment).  dims[0] is the fastest axis: a
// weight of N output rows over K inputs has dims {K, N} and N rows of K/elems
// blocks.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

using namespace syn;

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;
constexpr size_t kGgufAlign = 32;

// ggml tensor types the reference loads (gguf.rs:12-19), plus BF16, and their
// block sizes
size_t ggml_type_bytes(uint32_t type, uint64_t numel, bool *ok) {
  *ok = true;
  switch (type) {
    case SYN_HIP_GGML_F32: return numel * 4;
    case SYN_HIP_GGML_F16: return numel * 2;
    case SYN_HIP_GGML_BF16: return numel * 2;
    case SYN_HIP_GGML_Q4_0: if (numel % 32) break; return numel / 32 * 18;
    case SYN_HIP_GGML_Q4_1: if (numel % 32) break; return numel / 32 * 20;
    case SYN_HIP_GGML_Q8_0: if (numel % 32) break; return numel / 32 * 34;
    case SYN_HIP_GGML_Q4_K: if (numel % 256) break; return numel / 256 * 144;
    case SYN_HIP_GGML_Q6_K: if (numel % 256) break; return numel / 256 * 210;
    default: break;
  }
  *ok = false;
  return 0;
}

struct Reader {  // bounds-checked cursor over the mapping
  const uint8_t *p;
  size_t size, pos = 0;
  bool fail = false;
  bool take(void *dst, size_t n) {
    if (fail || n > size - pos) {
      fail = true;
      return false;
    }
    std::memcpy(dst, p + pos, n);
    pos += n;
    return true;
  }
  uint32_t u32() { uint32_t v = 0; take(&v, 4); return v; }
  uint64_t u64() { uint64_t v = 0; take(&v, 8); return v; }
  std::string str() {
    const uint64_t n = u64();
    if (fail || n > size - pos) {
      fail = true;
      return {};
    }
    std::string s(reinterpret_cast<const char *>(p + pos), n);
    pos += n;
    return s;
  }
  bool skip(uint64_t n) {
    if (fail || n > size - pos) {
      fail = true;
      return false;
    }
    pos += n;
    return true;
  }
};

}  // namespace

struct syn_hip_gguf_s {
  void *map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  struct Tensor {
    std::string name;
    uint32_t type = 0, n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;
  // scalar metadata (integers widened to u64/i64, floats to double, strings)
  struct Meta {
    uint32_t type = 0;
    uint64_t u = 0;
    double f = 0.0;
    std::string s;
  };
  std::unordered_map<std::string, Meta> meta;
  size_t data_start = 0;

  ~syn_hip_gguf_s() {
    if (map) munmap(map, size);
  }

  // metadata value of `vtype` (gguf.rs:561-591); scalars are kept
  bool read_value(Reader &r, uint32_t vtype, Meta *keep, int depth) {
    if (depth > 4) return false;
    switch (vtype) {
      case SYN_HIP_GGUF_UINT8: case SYN_HIP_GGUF_BOOL: { uint8_t v = 0; r.take(&v, 1); if (keep) keep->u = v; break; }
      case SYN_HIP_GGUF_INT8: { int8_t v = 0; r.take(&v, 1); if (keep) keep->u = (uint64_t)(int64_t)v; break; }
      case SYN_HIP_GGUF_UINT16: { uint16_t v = 0; r.take(&v, 2); if (keep) keep->u = v; break; }
      case SYN_HIP_GGUF_INT16: { int16_t v = 0; r.take(&v, 2); if (keep) keep->u = (uint64_t)(int64_t)v; break; }
      case SYN_HIP_GGUF_UINT32: { uint32_t v = 0; r.take(&v, 4); if (keep) keep->u = v; break; }
      case SYN_HIP_GGUF_INT32: { int32_t v = 0; r.take(&v, 4); if (keep) keep->u = (uint64_t)(int64_t)v; break; }
      case SYN_HIP_GGUF_FLOAT32: { float v = 0; r.take(&v, 4); if (keep) keep->f = v; break; }
      case SYN_HIP_GGUF_UINT64: case SYN_HIP_GGUF_INT64: { uint64_t v = r.u64(); if (keep) keep->u = v; break; }
      case SYN_HIP_GGUF_FLOAT64: { double v = 0; r.take(&v, 8); if (keep) keep->f = v; break; }
      case SYN_HIP_GGUF_STRING: { std::string s = r.str(); if (keep) keep->s = std::move(s); break; }
      case SYN_HIP_GGUF_ARRAY: {
        const uint32_t et = r.u32();
        const uint64_t count = r.u64();
        if (r.fail) return false;
        // fixed-size element types are skipped in one step
        const int fixed = et == SYN_HIP_GGUF_UINT8 || et == SYN_HIP_GGUF_INT8 || et == SYN_HIP_GGUF_BOOL ? 1
                        : et == SYN_HIP_GGUF_UINT16 || et == SYN_HIP_GGUF_INT16 ? 2
                        : et == SYN_HIP_GGUF_UINT32 || et == SYN_HIP_GGUF_INT32 || et == SYN_HIP_GGUF_FLOAT32 ? 4
                        : et == SYN_HIP_GGUF_UINT64 || et == SYN_HIP_GGUF_INT64 || et == SYN_HIP_GGUF_FLOAT64 ? 8 : 0;
        if (fixed) {
          if (count > (r.size - r.pos) / (uint64_t)fixed) return false;
          r.skip(count * (uint64_t)fixed);
        } else {
          for (uint64_t i = 0; i < count && !r.fail; i++)
            if (!read_value(r, et, nullptr, depth + 1)) return false;
        }
        break;
      }
      default: return false;
    }
    return !r.fail;
  }

  syn_status_t parse() {
    Reader r{static_cast<const uint8_t *>(map), size};
    if (r.u32() != kGgufMagic || r.fail) {
      set_error("GGUF: bad magic");
      return SYN_ERR_INVALID_ARG;
    }
    version = r.u32();
    if (version < 2 || version > 3) {  // gguf.rs:82-84
      set_error("GGUF: unsupported version " + std::to_string(version));
      return SYN_ERR_INVALID_ARG;
    }
    const uint64_t n_tensors = r.u64(), n_meta = r.u64();
    if (r.fail || n_tensors > size / 24 || n_meta > size / 12) {
      set_error("GGUF: truncated or inconsistent header");
      return SYN_ERR_INVALID_ARG;
    }
    for (uint64_t i = 0; i < n_meta; i++) {
      std::string key = r.str();
      const uint32_t vt = r.u32();
      Meta m;
      m.type = vt;
      if (r.fail || !read_value(r, vt, &m, 0)) {
        set_error("GGUF: malformed metadata entry " + std::to_string(i));
        return SYN_ERR_INVALID_ARG;
      }
      if (vt != SYN_HIP_GGUF_ARRAY) meta[key] = std::move(m);
    }
    tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
      Tensor &t = tensors[i];
      t.name = r.str();
      t.n_dims = r.u32();
      if (r.fail || t.n_dims == 0 || t.n_dims > 4) {
        set_error("GGUF: malformed tensor info " + std::to_string(i));
        return SYN_ERR_INVALID_ARG;
      }
      uint64_t numel = 1;
      for (uint32_t d = 0; d < t.n_dims; d++) {
        t.dims[d] = r.u64();
        if (t.dims[d] == 0 || t.dims[d] > (1ull << 40) || numel > (1ull << 42) / t.dims[d]) {
          set_error("GGUF: tensor '" + t.name + "' has an invalid shape");
          return SYN_ERR_INVALID_ARG;
        }
        numel *= t.dims[d];
      }
      t.type = r.u32();
      t.offset = r.u64();
      if (r.fail) {
        set_error("GGUF: truncated tensor info " + std::to_string(i));
        return SYN_ERR_INVALID_ARG;
      }
      bool ok = false;
      t.nbytes = ggml_type_bytes(t.type, numel, &ok);
      if (!ok) {  // gguf.rs:137-139
        set_error("GGUF: tensor '" + t.name + "' has unsupported GGML type " +
                  std::to_string(t.type) + " or a size that is not whole blocks");
        return SYN_ERR_INVALID_ARG;
      }
      by_name[t.name] = i;
    }
    // llama.cpp writers may set general.alignment; the reference assumes 32,
    // the default, which files without the key use
    size_t align = kGgufAlign;
    auto al = meta.find("general.alignment");
    if (al != meta.end() && al->second.type == SYN_HIP_GGUF_UINT32) {
      align = (size_t)al->second.u;
      if (align == 0 || (align & (align - 1)) || align > 4096) {
        set_error("GGUF: general.alignment " + std::to_string(align) + " is not a power of two");
        return SYN_ERR_INVALID_ARG;
      }
    }
    data_start = round_up(r.pos, align);
    for (const Tensor &t : tensors) {
      if (data_start > size || t.offset > size - data_start || t.nbytes > size - data_start - t.offset) {
        set_error("GGUF: tensor '" + t.name + "' lies outside the file");
        return SYN_ERR_INVALID_ARG;
      }
    }
    return SYN_OK;
  }
};

extern "C" {

syn_status_t syn_hip_gguf_open(const char *path, syn_hip_gguf_t **out) {
  if (!path || !out) return SYN_ERR_NULL_PTR;
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) {
    set_error(std::string("GGUF: cannot open ") + path);
    return SYN_ERR_INVALID_ARG;
  }
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    set_error(std::string("GGUF: file too small: ") + path);
    return SYN_ERR_INVALID_ARG;
  }
  void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) {
    set_error(std::string("GGUF: mmap failed for ") + path);
    return SYN_ERR_INVALID_ARG;
  }
  auto *g = new syn_hip_gguf_s();
  g->map = map;
  g->size = (size_t)st.st_size;
  const syn_status_t s = g->parse();
  if (s != SYN_OK) {
    delete g;
    return s;
  }
  *out = g;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_tensor_count(const syn_hip_gguf_t *g, size_t *n) {
  if (!g || !n) return SYN_ERR_NULL_PTR;
  *n = g->tensors.size();
  return SYN_OK;
}

syn_status_t syn_hip_gguf_find(const syn_hip_gguf_t *g, const char *name, size_t *index) {
  if (!g || !name || !index) return SYN_ERR_NULL_PTR;
  auto it = g->by_name.find(name);
  if (it == g->by_name.end()) {
    set_error(std::string("GGUF: no tensor named ") + name);
    return SYN_ERR_INVALID_ARG;
  }
  *index = it->second;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_tensor_info(const syn_hip_gguf_t *g, size_t index, const char **name,
                                      uint32_t *ggml_type, uint32_t *n_dims, uint64_t *dims4,
                                      uint64_t *nbytes, const void **data) {
  if (!g) return SYN_ERR_NULL_PTR;
  if (index >= g->tensors.size()) return SYN_ERR_INVALID_ARG;
  const auto &t = g->tensors[index];
  if (name) *name = t.name.c_str();
  if (ggml_type) *ggml_type = t.type;
  if (n_dims) *n_dims = t.n_dims;
  if (dims4)
    for (int d = 0; d < 4; d++) dims4[d] = t.dims[d];
  if (nbytes) *nbytes = t.nbytes;
  if (data) *data = static_cast<const uint8_t *>(g->map) + g->data_start + t.offset;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_meta_u64(const syn_hip_gguf_t *g, const char *key, uint64_t *value) {
  if (!g || !key || !value) return SYN_ERR_NULL_PTR;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type == SYN_HIP_GGUF_STRING ||
      it->second.type == SYN_HIP_GGUF_FLOAT32 || it->second.type == SYN_HIP_GGUF_FLOAT64) {
    set_error(std::string("GGUF: no integer metadata ") + key);
    return SYN_ERR_INVALID_ARG;
  }
  *value = it->second.u;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_meta_f64(const syn_hip_gguf_t *g, const char *key, double *value) {
  if (!g || !key || !value) return SYN_ERR_NULL_PTR;
  auto it = g->meta.find(key);
  if (it == g->meta.end() ||
      (it->second.type != SYN_HIP_GGUF_FLOAT32 && it->second.type != SYN_HIP_GGUF_FLOAT64)) {
    set_error(std::string("GGUF: no float metadata ") + key);
    return SYN_ERR_INVALID_ARG;
  }
  *value = it->second.f;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_meta_str(const syn_hip_gguf_t *g, const char *key, const char **value) {
  if (!g || !key || !value) return SYN_ERR_NULL_PTR;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type != SYN_HIP_GGUF_STRING) {
    set_error(std::string("GGUF: no string metadata ") + key);
    return SYN_ERR_INVALID_ARG;
  }
  *value = it->second.s.c_str();
  return SYN_OK;
}

syn_status_t syn_hip_gguf_close(syn_hip_gguf_t *g) {
  delete g;
  return SYN_OK;
}

}  // extern "C"
