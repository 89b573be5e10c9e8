// safetensors reader and the tensor views the model loaders read weights
// through (host code).
//
// safetensors (safetensors.rs:21-302): u64 header length, a JSON object
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__":
// {string: string}}, then the data section the offsets are relative to.  A
// directory opens as the sharded checkpoint its model.safetensors.index.json
// describes (only the tensors its weight_map lists are visible, each from the
// shard it names, safetensors.rs:21-62), or as the one .safetensors file in
// it.  Files are mapped read-only; tensor pointers stay valid until close.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <unordered_map>
#include <vector>

#include "kquant.hpp"
#include "weights.hpp"

using namespace syn;

namespace {

// ------------------------------------------------------------------ JSON
// Enough JSON for safetensors headers and index files: objects, arrays,
// strings (with escapes), numbers, true/false/null.
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  bool is_uint = false;  // a non-negative integer literal, exact in u
  uint64_t u = 0;
  std::string s;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json *get(const std::string &k) const {
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char *p, *end;
  std::string err;
  int depth = 0;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  static void put_utf8(std::string &o, uint32_t c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xC0 | (c >> 6));
      o += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      o += (char)(0xE0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    } else {
      o += (char)(0xF0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 0x3F));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t *v) {
    if (end - p < 4) return fail("short \\u escape");
    *v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p++;
      *v <<= 4;
      if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool str(std::string &o) {
    if (p >= end || *p != '"') return fail("expected a string");
    p++;
    while (p < end && *p != '"') {
      const char c = *p++;
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        o += c;
        continue;
      }
      if (p >= end) return fail("unterminated escape");
      const char e = *p++;
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(&c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            uint32_t c2;
            if (!hex4(&c2)) return false;
            if (c2 < 0xDC00 || c2 >= 0xE000) return fail("bad surrogate pair");
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          }
          put_utf8(o, c1);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    p++;
    return true;
  }
  bool number(Json &v) {
    const char *b = p;
    if (p < end && *p == '-') p++;
    const char *digits = p;
    while (p < end && *p >= '0' && *p <= '9') p++;
    if (p == digits) return fail("bad number");
    bool integer = true;
    if (p < end && *p == '.') {
      integer = false;
      p++;
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      integer = false;
      p++;
      if (p < end && (*p == '+' || *p == '-')) p++;
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    v.kind = Json::NUM;
    v.num = std::strtod(std::string(b, p).c_str(), nullptr);
    if (integer && *b != '-' && p - digits <= 19) {
      uint64_t u = 0;
      for (const char *q = digits; q < p; q++) u = u * 10 + (uint64_t)(*q - '0');
      v.is_uint = true;
      v.u = u;
    }
    return true;
  }
  bool lit(const char *w) {
    const size_t n = std::strlen(w);
    if ((size_t)(end - p) < n || std::memcmp(p, w, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool value(Json &v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    bool ok = true;
    if (*p == '{') {
      v.kind = Json::OBJ;
      p++;
      ws();
      if (p < end && *p == '}') {
        p++;
      } else {
        for (;;) {
          ws();
          std::string k;
          if (!str(k)) return false;
          ws();
          if (p >= end || *p != ':') return fail("expected ':'");
          p++;
          Json x;
          if (!value(x)) return false;
          v.obj.emplace_back(std::move(k), std::move(x));
          ws();
          if (p < end && *p == ',') { p++; continue; }
          if (p < end && *p == '}') { p++; break; }
          return fail("expected ',' or '}'");
        }
      }
    } else if (*p == '[') {
      v.kind = Json::ARR;
      p++;
      ws();
      if (p < end && *p == ']') {
        p++;
      } else {
        for (;;) {
          Json x;
          if (!value(x)) return false;
          v.arr.push_back(std::move(x));
          ws();
          if (p < end && *p == ',') { p++; continue; }
          if (p < end && *p == ']') { p++; break; }
          return fail("expected ',' or ']'");
        }
      }
    } else if (*p == '"') {
      v.kind = Json::STR;
      ok = str(v.s);
    } else if (*p == 't') {
      v.kind = Json::BOOL;
      v.b = true;
      ok = lit("true");
    } else if (*p == 'f') {
      v.kind = Json::BOOL;
      ok = lit("false");
    } else if (*p == 'n') {
      ok = lit("null");
    } else {
      ok = number(v);
    }
    depth--;
    return ok;
  }
  bool parse(Json &v) {
    if (!value(v)) return false;
    ws();
    return p == end || fail("trailing characters");
  }
};

// ------------------------------------------------------------------ files
struct Mapping {
  void *map = nullptr;
  size_t size = 0;
  ~Mapping() {
    if (map) munmap(map, size);
  }
};

syn_status_t map_file(const std::string &path, Mapping &m) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    set_error("safetensors: cannot open " + path);
    return SYN_ERR_INVALID_ARG;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    set_error("safetensors: cannot stat " + path);
    return SYN_ERR_INVALID_ARG;
  }
  m.size = (size_t)st.st_size;
  if (m.size > 0) {
    void *p = mmap(nullptr, m.size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      close(fd);
      set_error("safetensors: mmap failed for " + path);
      return SYN_ERR_INVALID_ARG;
    }
    m.map = p;
  }
  close(fd);
  return SYN_OK;
}

bool read_text(const std::string &path, std::string *out) {
  Mapping m;
  if (map_file(path, m) != SYN_OK) return false;
  out->assign(static_cast<const char *>(m.map), m.size);
  return true;
}

bool is_dir(const std::string &p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

bool exists(const std::string &p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0;
}

int st_dtype_of(const std::string &s, size_t *elem) {
  static const std::pair<const char *, int> kT[] = {
      {"F32", ST_F32}, {"F16", ST_F16}, {"BF16", ST_BF16}, {"I64", ST_I64}, {"I32", ST_I32},
      {"U8", ST_U8}};
  static const size_t kE[] = {4, 2, 2, 8, 4, 1};
  for (const auto &t : kT)
    if (s == t.first) {
      *elem = kE[t.second];
      return t.second;
    }
  return -1;
}

}  // namespace

struct syn_hip_safetensors_s {
  std::vector<std::unique_ptr<Mapping>> files;
  struct Tensor {
    std::string name;
    uint32_t dtype = 0, n_dims = 0;
    uint64_t shape[8] = {};
    const uint8_t *data = nullptr;
    uint64_t nbytes = 0;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;
  std::map<std::string, std::string> meta;

  // parse_safetensors (safetensors.rs:176-302) over one mapped file; `keep`
  // restricts the tensors taken (a shard's names in the index), `found`
  // records which of them the file had
  syn_status_t add_file(const std::string &path, const std::vector<std::string> *keep,
                        std::vector<bool> *found) {
    auto m = std::make_unique<Mapping>();
    SYN_TRY(map_file(path, *m));
    const uint8_t *base = static_cast<const uint8_t *>(m->map);
    if (m->size < 8) {
      set_error("safetensors: " + path + " is too small");
      return SYN_ERR_INVALID_ARG;
    }
    uint64_t hlen;
    std::memcpy(&hlen, base, 8);
    if (hlen > m->size - 8) {
      set_error("safetensors: header size exceeds the length of " + path);
      return SYN_ERR_INVALID_ARG;
    }
    const size_t data_start = 8 + (size_t)hlen, data_len = m->size - data_start;
    JsonParser jp{reinterpret_cast<const char *>(base + 8),
                  reinterpret_cast<const char *>(base + 8 + hlen)};
    Json h;
    if (!jp.parse(h) || h.kind != Json::OBJ) {
      set_error("safetensors: invalid JSON header in " + path + ": " +
                (jp.err.empty() ? "not an object" : jp.err));
      return SYN_ERR_INVALID_ARG;
    }
    for (const auto &kv : h.obj) {
      const std::string &name = kv.first;
      const Json &info = kv.second;
      if (name == "__metadata__") {
        for (const auto &mkv : info.obj)
          if (mkv.second.kind == Json::STR) meta[mkv.first] = mkv.second.s;
        continue;
      }
      size_t want_idx = 0;
      if (keep) {
        auto it = std::find(keep->begin(), keep->end(), name);
        if (it == keep->end()) continue;  // not listed in the index: skipped
        want_idx = (size_t)(it - keep->begin());
      }
      const Json *dt = info.get("dtype"), *sh = info.get("shape"), *of = info.get("data_offsets");
      if (info.kind != Json::OBJ || !dt || dt->kind != Json::STR) {
        set_error("safetensors: missing dtype for " + name);
        return SYN_ERR_INVALID_ARG;
      }
      if (!sh || sh->kind != Json::ARR || sh->arr.size() > 8) {
        set_error("safetensors: missing or invalid shape for " + name);
        return SYN_ERR_INVALID_ARG;
      }
      if (!of || of->kind != Json::ARR || of->arr.size() != 2 || !of->arr[0].is_uint ||
          !of->arr[1].is_uint) {
        set_error("safetensors: missing data_offsets for " + name);
        return SYN_ERR_INVALID_ARG;
      }
      size_t elem = 0;
      const int dtype = st_dtype_of(dt->s, &elem);
      if (dtype < 0) {  // safetensors.rs:291
        set_error("safetensors: unsupported dtype " + dt->s + " for " + name);
        return SYN_ERR_INVALID_ARG;
      }
      Tensor t;
      t.name = name;
      t.dtype = (uint32_t)dtype;
      t.n_dims = (uint32_t)sh->arr.size();
      uint64_t numel = 1;
      for (size_t d = 0; d < sh->arr.size(); d++) {
        const Json &x = sh->arr[d];
        if (!x.is_uint || x.u > (1ull << 40) || (x.u && numel > (1ull << 42) / x.u)) {
          set_error("safetensors: invalid shape for " + name);
          return SYN_ERR_INVALID_ARG;
        }
        t.shape[d] = x.u;
        numel *= x.u;
      }
      const uint64_t b = of->arr[0].u, e = of->arr[1].u;
      if (e < b || e > data_len) {  // safetensors.rs:224-228
        set_error("safetensors: tensor " + name + " data exceeds file bounds");
        return SYN_ERR_INVALID_ARG;
      }
      if (e - b != numel * elem) {
        set_error("safetensors: tensor " + name + " holds " + std::to_string(e - b) +
                  " bytes, its shape and dtype need " + std::to_string(numel * elem));
        return SYN_ERR_SHAPE_MISMATCH;
      }
      t.data = base + data_start + b;
      t.nbytes = e - b;
      if (by_name.count(name)) {
        set_error("safetensors: tensor " + name + " appears twice");
        return SYN_ERR_INVALID_ARG;
      }
      by_name[name] = tensors.size();
      tensors.push_back(t);
      if (found) (*found)[want_idx] = true;
    }
    files.push_back(std::move(m));
    return SYN_OK;
  }

  // load_safetensors_sharded (safetensors.rs:21-62)
  syn_status_t add_index(const std::string &dir) {
    const std::string ipath = dir + "/model.safetensors.index.json";
    std::string text;
    if (!read_text(ipath, &text)) return SYN_ERR_INVALID_ARG;
    JsonParser jp{text.data(), text.data() + text.size()};
    Json idx;
    const Json *wm = nullptr;
    if (!jp.parse(idx) || idx.kind != Json::OBJ || !(wm = idx.get("weight_map")) ||
        wm->kind != Json::OBJ) {
      set_error("safetensors: invalid index JSON " + ipath +
                (jp.err.empty() ? "" : ": " + jp.err));
      return SYN_ERR_INVALID_ARG;
    }
    std::map<std::string, std::vector<std::string>> by_shard;
    for (const auto &kv : wm->obj) {
      if (kv.second.kind != Json::STR || kv.second.s.find('/') != std::string::npos) {
        set_error("safetensors: index entry for " + kv.first + " is not a shard file name");
        return SYN_ERR_INVALID_ARG;
      }
      by_shard[kv.second.s].push_back(kv.first);
    }
    for (const auto &sh : by_shard) {
      std::vector<bool> found(sh.second.size(), false);
      const syn_status_t s = add_file(dir + "/" + sh.first, &sh.second, &found);
      if (s != SYN_OK) {
        set_error("safetensors: failed to load shard '" + sh.first + "': " +
                  syn_hip_last_error());
        return s;
      }
      for (size_t i = 0; i < found.size(); i++)
        if (!found[i]) {
          set_error("safetensors: tensor '" + sh.second[i] + "' listed in index but not found "
                    "in shard '" + sh.first + "'");
          return SYN_ERR_INVALID_ARG;
        }
    }
    return SYN_OK;
  }

  syn_status_t open_path(const std::string &path) {
    if (!is_dir(path)) return add_file(path, nullptr, nullptr);
    if (exists(path + "/model.safetensors.index.json")) return add_index(path);
    // the one .safetensors file of the directory
    std::vector<std::string> found;
    if (DIR *d = opendir(path.c_str())) {
      while (dirent *e = readdir(d)) {
        const std::string n = e->d_name;
        if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) found.push_back(n);
      }
      closedir(d);
    }
    if (found.size() != 1) {
      set_error("safetensors: " + path + " holds " + std::to_string(found.size()) +
                " .safetensors files and no model.safetensors.index.json");
      return SYN_ERR_INVALID_ARG;
    }
    return add_file(path + "/" + found[0], nullptr, nullptr);
  }
};

namespace syn {

// ------------------------------------------------------------------ views
namespace {

class GgufSource : public WeightSource {
 public:
  explicit GgufSource(const syn_hip_gguf_t *g) : g_(g) {}
  bool find(const std::string &name, TensorView *t) const override {
    size_t idx = 0;
    if (syn_hip_gguf_find(g_, name.c_str(), &idx) != SYN_OK) return false;
    uint32_t type = 0, nd = 0;
    uint64_t dims[4], nb = 0;
    const void *d = nullptr;
    syn_hip_gguf_tensor_info(g_, idx, nullptr, &type, &nd, dims, &nb, &d);
    t->name = name;
    t->gguf = true;
    t->type = type;
    t->n_dims = (int)nd;
    for (uint32_t i = 0; i < nd; i++) t->shape[i] = dims[nd - 1 - i];  // slowest first
    t->data = static_cast<const uint8_t *>(d);
    t->nbytes = nb;
    return true;
  }

 private:
  const syn_hip_gguf_t *g_;
};

class SafetensorsSource : public WeightSource {
 public:
  explicit SafetensorsSource(const syn_hip_safetensors_t *st) : st_(st) {}
  bool find(const std::string &name, TensorView *t) const override {
    auto it = st_->by_name.find(name);
    if (it == st_->by_name.end()) return false;
    const auto &x = st_->tensors[it->second];
    t->name = name;
    t->gguf = false;
    t->type = x.dtype;
    t->n_dims = (int)x.n_dims;
    for (uint32_t i = 0; i < x.n_dims; i++) t->shape[i] = x.shape[i];
    t->data = x.data;
    t->nbytes = x.nbytes;
    return true;
  }

 private:
  const syn_hip_safetensors_t *st_;
};

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
float bf16_to_f32(uint16_t b) {  // converter.rs:44-46
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

}  // namespace

std::unique_ptr<WeightSource> gguf_source(const syn_hip_gguf_t *g) {
  return std::make_unique<GgufSource>(g);
}
std::unique_ptr<WeightSource> safetensors_source(const syn_hip_safetensors_t *st) {
  return std::make_unique<SafetensorsSource>(st);
}

syn_status_t tensor_to_f32(const TensorView &t, float *out) {
  const uint64_t n = t.numel();
  const uint8_t *p = t.data;
  if (t.gguf) {
    switch (t.type) {
      case SYN_HIP_GGML_F32: std::memcpy(out, p, n * 4); return SYN_OK;
      case SYN_HIP_GGML_F16:  // gguf.rs:214-219 with converter.rs:12-40
        for (uint64_t i = 0; i < n; i++) out[i] = f16_to_f32_reference(rd16(p + 2 * i));
        return SYN_OK;
      case SYN_HIP_GGML_BF16:
        for (uint64_t i = 0; i < n; i++) out[i] = bf16_to_f32(rd16(p + 2 * i));
        return SYN_OK;
      case SYN_HIP_GGML_Q4_0:  // gguf.rs:294-330: element 2i low nibble, 2i+1 high
        for (uint64_t b = 0; b < n / 32; b++) {
          const uint8_t *q = p + b * 18;
          const float d = f16_to_f32_reference(rd16(q));
          for (int i = 0; i < 16; i++) {
            out[b * 32 + 2 * i] = d * (float)((int)(q[2 + i] & 15) - 8);
            out[b * 32 + 2 * i + 1] = d * (float)((int)(q[2 + i] >> 4) - 8);
          }
        }
        return SYN_OK;
      case SYN_HIP_GGML_Q4_1:  // gguf.rs:332-373: nibble*d + m
        for (uint64_t b = 0; b < n / 32; b++) {
          const uint8_t *q = p + b * 20;
          const float d = f16_to_f32_reference(rd16(q)), m = f16_to_f32_reference(rd16(q + 2));
          for (int i = 0; i < 16; i++) {
            const float lo = (float)(q[4 + i] & 15) * d, hi = (float)(q[4 + i] >> 4) * d;
            out[b * 32 + 2 * i] = lo + m;
            out[b * 32 + 2 * i + 1] = hi + m;
          }
        }
        return SYN_OK;
      case SYN_HIP_GGML_Q8_0: kq_dequant(SYN_HIP_FMT_Q8_0, p, n / 32, out); return SYN_OK;
      case SYN_HIP_GGML_Q4_K: kq_dequant(SYN_HIP_FMT_Q4_K, p, n / 256, out); return SYN_OK;
      case SYN_HIP_GGML_Q6_K: kq_dequant(SYN_HIP_FMT_Q6_K, p, n / 256, out); return SYN_OK;
      default: break;
    }
  } else {
    switch (t.type) {  // safetensors.rs:232-290
      case ST_F32: std::memcpy(out, p, n * 4); return SYN_OK;
      case ST_F16:
        for (uint64_t i = 0; i < n; i++) out[i] = f16_to_f32_reference(rd16(p + 2 * i));
        return SYN_OK;
      case ST_BF16:
        for (uint64_t i = 0; i < n; i++) out[i] = bf16_to_f32(rd16(p + 2 * i));
        return SYN_OK;
      case ST_I64:
        for (uint64_t i = 0; i < n; i++) {
          int64_t v;
          std::memcpy(&v, p + 8 * i, 8);
          out[i] = (float)v;
        }
        return SYN_OK;
      case ST_I32:
        for (uint64_t i = 0; i < n; i++) {
          int32_t v;
          std::memcpy(&v, p + 4 * i, 4);
          out[i] = (float)v;
        }
        return SYN_OK;
      case ST_U8:
        for (uint64_t i = 0; i < n; i++) out[i] = (float)p[i];
        return SYN_OK;
      default: break;
    }
  }
  set_error("tensor " + t.name + " has a type with no f32 conversion");
  return SYN_ERR_INVALID_ARG;
}

}  // namespace syn

namespace {

// expand_q4_tensors' triple (safetensors.rs:80-170) as pack_for_zig bytes:
// <base>.q4_nibbles U8 [rows, bpr, 16], <base>.q4_scales F16 [rows, bpr],
// <base>.q4_orig_cols I64 [1]
syn_status_t q4_triple(const syn_hip_safetensors_t *st, const std::string &base,
                       uint8_t *packed, size_t *rows, size_t *cols) {
  SafetensorsSource src(st);
  TensorView nib, sc, oc;
  if (!src.find(base + ".q4_nibbles", &nib) || !src.find(base + ".q4_scales", &sc) ||
      !src.find(base + ".q4_orig_cols", &oc)) {
    set_error("safetensors: " + base + " lacks one of .q4_nibbles, .q4_scales, .q4_orig_cols");
    return SYN_ERR_INVALID_ARG;
  }
  if (nib.type != ST_U8 || nib.n_dims != 3 || nib.shape[2] != 16) {
    set_error("safetensors: " + base + ".q4_nibbles expected U8 [rows, bpr, 16]");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  const uint64_t r = nib.shape[0], bpr = nib.shape[1];
  if (sc.type != ST_F16 || !sc.is_matrix(r, bpr)) {
    set_error("safetensors: " + base + ".q4_scales expected F16 [" + std::to_string(r) + ", " +
              std::to_string(bpr) + "]");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  if (oc.numel() < 1 || (oc.type != ST_I64 && oc.type != ST_I32)) {
    set_error("safetensors: " + base + ".q4_orig_cols is empty or not an integer");
    return SYN_ERR_INVALID_ARG;
  }
  float c;
  SYN_TRY(tensor_to_f32(oc, &c));  // the reference reads it through its f32 cast
  const uint64_t cc = (uint64_t)c;
  if (c < 1 || cc > bpr * 32) {
    set_error("safetensors: " + base + ": orig_cols " + std::to_string(cc) + " > padded_cols " +
              std::to_string(bpr * 32));
    return SYN_ERR_SHAPE_MISMATCH;
  }
  *rows = (size_t)r;
  *cols = (size_t)cc;
  if (packed)
    for (uint64_t i = 0; i < r * bpr; i++) {
      std::memcpy(packed + i * 18, sc.data + 2 * i, 2);
      std::memcpy(packed + i * 18 + 2, nib.data + 16 * i, 16);
    }
  return SYN_OK;
}

}  // namespace

extern "C" {

syn_status_t syn_hip_safetensors_open(const char *path, syn_hip_safetensors_t **out) {
  if (!path || !out) return SYN_ERR_NULL_PTR;
  *out = nullptr;
  auto st = std::make_unique<syn_hip_safetensors_s>();
  SYN_TRY(st->open_path(path));
  *out = st.release();
  return SYN_OK;
}

syn_status_t syn_hip_safetensors_tensor_count(const syn_hip_safetensors_t *st, size_t *n) {
  if (!st || !n) return SYN_ERR_NULL_PTR;
  *n = st->tensors.size();
  return SYN_OK;
}

syn_status_t syn_hip_safetensors_find(const syn_hip_safetensors_t *st, const char *name,
                                      size_t *index) {
  if (!st || !name || !index) return SYN_ERR_NULL_PTR;
  auto it = st->by_name.find(name);
  if (it == st->by_name.end()) {
    set_error(std::string("safetensors: no tensor named ") + name);
    return SYN_ERR_INVALID_ARG;
  }
  *index = it->second;
  return SYN_OK;
}

syn_status_t syn_hip_safetensors_tensor_info(const syn_hip_safetensors_t *st, size_t index,
                                             const char **name, uint32_t *dtype,
                                             uint32_t *n_dims, uint64_t *shape8,
                                             uint64_t *nbytes, const void **data) {
  if (!st) return SYN_ERR_NULL_PTR;
  if (index >= st->tensors.size()) return SYN_ERR_INVALID_ARG;
  const auto &t = st->tensors[index];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype;
  if (n_dims) *n_dims = t.n_dims;
  if (shape8)
    for (int d = 0; d < 8; d++) shape8[d] = t.shape[d];
  if (nbytes) *nbytes = t.nbytes;
  if (data) *data = t.data;
  return SYN_OK;
}

syn_status_t syn_hip_safetensors_meta(const syn_hip_safetensors_t *st, const char *key,
                                      const char **value) {
  if (!st || !key || !value) return SYN_ERR_NULL_PTR;
  auto it = st->meta.find(key);
  if (it == st->meta.end()) {
    set_error(std::string("safetensors: no metadata ") + key);
    return SYN_ERR_INVALID_ARG;
  }
  *value = it->second.c_str();
  return SYN_OK;
}

syn_status_t syn_hip_safetensors_to_f32(const syn_hip_safetensors_t *st, size_t index,
                                        float *out) {
  if (!st || !out) return SYN_ERR_NULL_PTR;
  if (index >= st->tensors.size()) return SYN_ERR_INVALID_ARG;
  TensorView t;
  SafetensorsSource(st).find(st->tensors[index].name, &t);
  return tensor_to_f32(t, out);
}

syn_status_t syn_hip_safetensors_q4_pack(const syn_hip_safetensors_t *st, const char *base,
                                         uint8_t *packed, size_t *rows, size_t *cols) {
  if (!st || !base || !rows || !cols) return SYN_ERR_NULL_PTR;
  return q4_triple(st, base, packed, rows, cols);
}

syn_status_t syn_hip_safetensors_close(syn_hip_safetensors_t *st) {
  delete st;
  return SYN_OK;
}

syn_status_t syn_hip_gguf_to_f32(const syn_hip_gguf_t *g, size_t index, float *out) {
  if (!g || !out) return SYN_ERR_NULL_PTR;
  const char *name = nullptr;
  if (syn_hip_gguf_tensor_info(g, index, &name, nullptr, nullptr, nullptr, nullptr, nullptr) !=
      SYN_OK)
    return SYN_ERR_INVALID_ARG;
  TensorView t;
  GgufSource(g).find(name, &t);
  return tensor_to_f32(t, out);
}

syn_status_t syn_hip_qlinear_from_gguf(const syn_hip_gguf_t *g, const char *name,
                                       syn_hip_qlinear_t **out) {
  if (!g || !name || !out) return SYN_ERR_NULL_PTR;
  TensorView t;
  if (!GgufSource(g).find(name, &t)) {
    set_error(std::string("GGUF: no tensor named ") + name);
    return SYN_ERR_INVALID_ARG;
  }
  const int fmt = t.type == SYN_HIP_GGML_Q4_0 ? SYN_HIP_FMT_Q4_0
                : t.type == SYN_HIP_GGML_Q8_0 ? SYN_HIP_FMT_Q8_0
                : t.type == SYN_HIP_GGML_Q4_K ? SYN_HIP_FMT_Q4_K
                : t.type == SYN_HIP_GGML_Q6_K ? SYN_HIP_FMT_Q6_K : -1;
  if (fmt < 0 || t.n_dims != 2) {
    set_error(std::string("GGUF: ") + name + " is not a 2-D Q4_0/Q8_0/Q4_K/Q6_K tensor");
    return SYN_ERR_INVALID_ARG;
  }
  // the block bytes as stored: Q4_0 blocks are the pack_for_zig layout the
  // reference's RawQ4Tensor hands to its Q4 GEMV (gguf.rs:49-57, 104-114)
  return syn_hip_qlinear_create(fmt, (size_t)t.shape[0], (size_t)t.shape[1], t.data, nullptr, 0,
                                out);
}

syn_status_t syn_hip_qlinear_from_safetensors_q4(const syn_hip_safetensors_t *st,
                                                 const char *base, syn_hip_qlinear_t **out) {
  if (!st || !base || !out) return SYN_ERR_NULL_PTR;
  size_t rows = 0, cols = 0;
  SYN_TRY(q4_triple(st, base, nullptr, &rows, &cols));
  if (cols % 32) {
    set_error(std::string("safetensors: ") + base + " has " + std::to_string(cols) +
              " columns; the Q4_0 GEMV needs a multiple of 32 (expand it to f32 instead)");
    return SYN_ERR_SHAPE_MISMATCH;
  }
  std::vector<uint8_t> packed(rows * (cols / 32) * 18);
  SYN_TRY(q4_triple(st, base, packed.data(), &rows, &cols));
  return syn_hip_qlinear_create(SYN_HIP_FMT_Q4_0, rows, cols, packed.data(), nullptr, 0, out);
}

}  // extern "C"
