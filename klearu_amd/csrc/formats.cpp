// On-disk formats of the sparse decode path, read on the host straight into
// the device handles:
//   - safetensors model files (crates/klearu-llm/src/weight/safetensors.rs:37-159,
//     loader.rs:30-64, name_map.rs:36-98): header parse, tensor lookup,
//     tensor_to_f32, and the BF16 gate/up/down and q/k/v/o matrices of one
//     decoder layer uploaded into kh_sparse_ffn / kh_sparse_attn.
//   - the SparsityPredictor JSON file (crates/klearu-dejavu/src/predictor/
//     mlp_predictor.rs:10-26, 87-98; serde_json 1.0.149): fields w1 (nested,
//     [hidden][input]), b1, w2 ([output][hidden]), b2, input_dim, hidden_dim,
//     output_dim.
// Numbers are read as serde_json reads an f32: the decimal is rounded to the
// nearest f64, then the f64 to the nearest f32.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"


namespace {

// ---- a pull parser over one JSON text ------------------------------------

struct Json {
  const char* p;
  const char* end;
  std::string err;

  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool expect(char c) {
    if (eat(c)) return true;
    char m[40];
    snprintf(m, sizeof m, "expected '%c'", c);
    return fail(m);
  }
  static void utf8(std::string& s, unsigned cp) {
    if (cp < 0x80) {
      s += char(cp);
    } else if (cp < 0x800) {
      s += char(0xC0 | (cp >> 6));
      s += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += char(0xE0 | (cp >> 12));
      s += char(0x80 | ((cp >> 6) & 0x3F));
      s += char(0x80 | (cp & 0x3F));
    } else {
      s += char(0xF0 | (cp >> 18));
      s += char(0x80 | ((cp >> 12) & 0x3F));
      s += char(0x80 | ((cp >> 6) & 0x3F));
      s += char(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(unsigned* v) {
    if (end - p < 4) return fail("short \\u escape");
    unsigned r = 0;
    for (int i = 0; i < 4; ++i) {
      char c = *p++;
      r <<= 4;
      if (c >= '0' && c <= '9') r |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') r |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= unsigned(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    *v = r;
    return true;
  }
  bool string(std::string* out) {
    if (!expect('"')) return false;
    out->clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        *out += c;
        continue;
      }
      if (p >= end) break;
      char e = *p++;
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          unsigned cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            unsigned lo;
            if (!hex4(&lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(*out, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  // A JSON number token: -?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?
  bool number_token(const char** b, const char** e, bool* integral) {
    ws();
    const char* s = p;
    const char* q = p;
    if (q < end && *q == '-') ++q;
    if (q >= end || *q < '0' || *q > '9') return fail("expected a number");
    if (*q == '0') ++q;
    else
      while (q < end && *q >= '0' && *q <= '9') ++q;
    *integral = true;
    if (q < end && *q == '.') {
      *integral = false;
      ++q;
      if (q >= end || *q < '0' || *q > '9') return fail("bad fraction");
      while (q < end && *q >= '0' && *q <= '9') ++q;
    }
    if (q < end && (*q == 'e' || *q == 'E')) {
      *integral = false;
      ++q;
      if (q < end && (*q == '+' || *q == '-')) ++q;
      if (q >= end || *q < '0' || *q > '9') return fail("bad exponent");
      while (q < end && *q >= '0' && *q <= '9') ++q;
    }
    *b = s;
    *e = q;
    p = q;
    return true;
  }
  // serde's f32 from a JSON number: nearest f64, then nearest f32.  JSON has
  // no '+' prefix; from_chars rejects one too.
  bool f32(float* v) {
    const char *b, *e;
    bool integral;
    if (!number_token(&b, &e, &integral)) return false;
    double d;
    auto r = std::from_chars(b, e, d);
    if (r.ec == std::errc::result_out_of_range) {
      // from_chars leaves d unset outside the f64 range.  serde_json rejects
      // a number too large for an f64 and reads one too small as a signed
      // zero.
      const char* x = b;
      while (x < e && *x != 'e' && *x != 'E') ++x;
      if (!(x + 1 < e && x[1] == '-')) return fail("number out of range");
      d = *b == '-' ? -0.0 : 0.0;
    } else if (r.ec != std::errc() || r.ptr != e) {
      return fail("bad number");
    }
    *v = (float)d;
    return true;
  }
  bool u64(uint64_t* v) {
    const char *b, *e;
    bool integral;
    if (!number_token(&b, &e, &integral)) return false;
    if (!integral || *b == '-') return fail("expected a non-negative integer");
    auto r = std::from_chars(b, e, *v);
    if (r.ec != std::errc() || r.ptr != e) return fail("integer out of range");
    return true;
  }
  bool literal(const char* w) {
    size_t n = strlen(w);
    if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool skip(int depth = 0) {
    if (depth > 256) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    char c = *p;
    if (c == '"') {
      std::string s;
      return string(&s);
    }
    if (c == '{') {
      ++p;
      if (eat('}')) return true;
      do {
        std::string k;
        if (!string(&k) || !expect(':') || !skip(depth + 1)) return false;
      } while (eat(','));
      return expect('}');
    }
    if (c == '[') {
      ++p;
      if (eat(']')) return true;
      do {
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return expect(']');
    }
    if (c == 't') return literal("true");
    if (c == 'f') return literal("false");
    if (c == 'n') return literal("null");
    const char *b, *e;
    bool integral;
    return number_token(&b, &e, &integral);
  }
  // [f, f, ...] appended to out
  bool f32_array(std::vector<float>* out, size_t* count) {
    if (!expect('[')) return false;
    size_t n = 0;
    if (!eat(']')) {
      do {
        float v;
        if (!f32(&v)) return false;
        out->push_back(v);
        ++n;
      } while (eat(','));
      if (!expect(']')) return false;
    }
    *count = n;
    return true;
  }
  // [[f, ...], ...] row-major into out; every row must have the same length
  bool f32_matrix(std::vector<float>* out, size_t* rows, size_t* cols) {
    if (!expect('[')) return false;
    size_t r = 0, c = 0;
    if (!eat(']')) {
      do {
        size_t n;
        if (!f32_array(out, &n)) return false;
        if (r == 0) c = n;
        else if (n != c) return fail("ragged matrix");
        ++r;
      } while (eat(','));
      if (!expect(']')) return false;
    }
    *rows = r;
    *cols = c;
    return true;
  }
  bool done() {
    ws();
    return p == end || fail("trailing characters");
  }
};

// ---- files ----------------------------------------------------------------

struct Mapped {
  void* base = nullptr;
  size_t len = 0;
  ~Mapped() {
    if (base && len) munmap(base, len);
  }
};

int map_file(const std::string& path, Mapped* m) {
  int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    kh::set_error("cannot open %s", path.c_str());
    return KH_ERR_ARG;
  }
  struct stat sb;
  if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
    close(fd);
    kh::set_error("%s is not a regular file", path.c_str());
    return KH_ERR_ARG;
  }
  m->len = (size_t)sb.st_size;
  if (m->len) {
    void* b = mmap(nullptr, m->len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (b == MAP_FAILED) {
      close(fd);
      m->len = 0;
      kh::set_error("mmap of %s failed", path.c_str());
      return KH_ERR_ALLOC;
    }
    m->base = b;
  }
  close(fd);
  return KH_OK;
}

int read_text(const char* path, std::string* s) {
  Mapped m;
  int rc = map_file(path, &m);
  if (rc != KH_OK) return rc;
  s->assign(static_cast<const char*>(m.base), m.len);
  return KH_OK;
}

inline float bf16_to_f32(uint16_t b) {
  uint32_t u = uint32_t(b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// IEEE binary16 -> binary32, exact (half::f16::to_f32).
inline float f16_to_f32(uint16_t h) {
  uint32_t s = uint32_t(h & 0x8000) << 16;
  uint32_t e = (h >> 10) & 0x1F;
  uint32_t m = h & 0x3FF;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {  // subnormal: normalise
      int sh = 0;
      while (!(m & 0x400)) {
        m <<= 1;
        ++sh;
      }
      m &= 0x3FF;
      u = s | (uint32_t(127 - 15 + 1 - sh) << 23) | (m << 13);
    }
  } else if (e == 31) {
    u = s | 0x7F800000u | (m << 13);
  } else {
    u = s | ((e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

// ---- safetensors ------------------------------------------------------------

struct kh_safetensors {
  struct Tensor {
    int dtype;
    std::vector<int64_t> shape;
    const uint8_t* data;  // start of the tensor's bytes inside its file's mapping
    uint64_t start, stop; // data_offsets relative to the file's data section
    size_t avail;         // bytes of the data section at and after `start`
  };
  std::vector<std::unique_ptr<Mapped>> files;
  std::map<std::string, Tensor> tensors;  // sorted by name; a later file shadows an earlier one
};

namespace {

int elem_size(int dt) { return dt == KH_DT_F32 ? 4 : 2; }

// SafeTensorsFile::open (safetensors.rs:37-113) for one file.
int st_open_file(kh_safetensors* st, const std::string& path) {
  auto m = std::make_unique<Mapped>();
  int rc = map_file(path, m.get());
  if (rc != KH_OK) return rc;
  const uint8_t* base = static_cast<const uint8_t*>(m->base);
  if (m->len < 8) {
    kh::set_error("%s: file too small", path.c_str());
    return KH_ERR_ARG;
  }
  uint64_t hl = 0;
  for (int i = 7; i >= 0; --i) hl = (hl << 8) | base[i];
  if (hl > m->len - 8) {
    kh::set_error("%s: invalid header length", path.c_str());
    return KH_ERR_ARG;
  }
  const size_t data0 = 8 + hl;
  Json j{reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(base + 8 + hl), {}};
  std::map<std::string, kh_safetensors::Tensor> found;
  bool ok = j.expect('{');
  if (ok && !j.eat('}')) {
    do {
      std::string name;
      if (!(ok = j.string(&name) && j.expect(':'))) break;
      if (name == "__metadata__") {
        if (!(ok = j.skip())) break;
        continue;
      }
      kh_safetensors::Tensor t{-1, {}, nullptr, 0, 0, 0};
      bool have_off = false, have_shape = false;
      if (!(ok = j.expect('{'))) break;
      if (!j.eat('}')) {
        do {
          std::string key;
          if (!(ok = j.string(&key) && j.expect(':'))) break;
          if (key == "dtype") {
            std::string d;
            if (!(ok = j.string(&d))) break;
            if (d == "F32") t.dtype = KH_DT_F32;
            else if (d == "F16") t.dtype = KH_DT_F16;
            else if (d == "BF16") t.dtype = KH_DT_BF16;
            else {
              kh::set_error("%s: unsupported dtype %s for %s", path.c_str(), d.c_str(), name.c_str());
              return KH_ERR_UNSUPPORTED;
            }
          } else if (key == "shape") {
            have_shape = true;
            if (!(ok = j.expect('['))) break;
            if (!j.eat(']')) {
              do {
                uint64_t v;
                if (!(ok = j.u64(&v))) break;
                if (v > (uint64_t)INT64_MAX) {
                  ok = j.fail("shape entry out of range");
                  break;
                }
                t.shape.push_back((int64_t)v);
              } while (j.eat(','));
              if (!ok || !(ok = j.expect(']'))) break;
            }
          } else if (key == "data_offsets") {
            have_off = true;
            uint64_t a, b;
            if (!(ok = j.expect('[') && j.u64(&a) && j.expect(',') && j.u64(&b) && j.expect(']'))) break;
            t.start = a;
            t.stop = b;
          } else if (!(ok = j.skip())) {
            break;
          }
        } while (j.eat(','));
        if (!ok || !(ok = j.expect('}'))) break;
      }
      if (t.dtype < 0 || !have_shape || !have_off) {
        kh::set_error("%s: tensor %s lacks dtype, shape or data_offsets", path.c_str(), name.c_str());
        return KH_ERR_ARG;
      }
      if (t.stop < t.start) {
        kh::set_error("%s: tensor %s has data_offsets end < start", path.c_str(), name.c_str());
        return KH_ERR_ARG;
      }
      size_t data_len = m->len - data0;
      t.avail = t.start <= data_len ? data_len - (size_t)t.start : 0;
      t.data = t.start <= data_len ? base + data0 + t.start : nullptr;
      found[name] = std::move(t);
    } while (j.eat(','));
    if (ok) ok = j.expect('}');
  }
  if (ok) ok = j.done();
  if (!ok) {
    kh::set_error("%s: bad header: %s at byte %zu", path.c_str(), j.err.c_str(),
                  (size_t)(j.p - reinterpret_cast<const char*>(base)));
    return KH_ERR_ARG;
  }
  for (auto& kv : found) st->tensors[kv.first] = std::move(kv.second);
  st->files.push_back(std::move(m));
  return KH_OK;
}

const kh_safetensors::Tensor* st_find(const kh_safetensors* st, const std::string& name) {
  auto it = st->tensors.find(name);
  return it == st->tensors.end() ? nullptr : &it->second;
}

int64_t numel(const kh_safetensors::Tensor& t) {
  int64_t n = 1;
  for (int64_t d : t.shape) {
    if (d != 0 && n > INT64_MAX / d) return -1;
    n *= d;
  }
  return n;
}

// tensor_data (safetensors.rs:119-133) with its bounds check, plus the check
// that the bytes hold exactly numel elements of the dtype.
int st_bytes(const kh_safetensors::Tensor& t, const char* name, int64_t* n) {
  uint64_t len = t.stop - t.start;
  if (!t.data || len > t.avail) {
    kh::set_error("tensor %s data out of bounds", name);
    return KH_ERR_ARG;
  }
  int64_t ne = numel(t);
  const uint64_t es = (uint64_t)elem_size(t.dtype);
  // ne > len / es first: the product below then cannot wrap
  if (ne < 0 || (uint64_t)ne > len / es || (uint64_t)ne * es != len) {
    kh::set_error("tensor %s: %llu bytes do not hold its shape", name, (unsigned long long)len);
    return KH_ERR_ARG;
  }
  *n = ne;
  return KH_OK;
}

void to_f32(const kh_safetensors::Tensor& t, int64_t n, float* out) {
  const uint8_t* d = t.data;
  if (t.dtype == KH_DT_F32) {
    memcpy(out, d, (size_t)n * 4);
  } else if (t.dtype == KH_DT_BF16) {
    for (int64_t i = 0; i < n; ++i) {
      uint16_t b;
      memcpy(&b, d + 2 * i, 2);
      out[i] = bf16_to_f32(b);
    }
  } else {
    for (int64_t i = 0; i < n; ++i) {
      uint16_t h;
      memcpy(&h, d + 2 * i, 2);
      out[i] = f16_to_f32(h);
    }
  }
}

// BF16 bits of a tensor expected as [rows][cols].  BF16 is taken as is; F32
// and F16 are accepted when every value is a BF16 value (the bits then carry
// exactly the reference's f32 weights), else KH_ERR_UNSUPPORTED.
int st_bf16_matrix(const kh_safetensors* st, const std::string& name, int64_t rows, int64_t cols,
                   std::vector<uint16_t>* out) {
  const auto* t = st_find(st, name);
  if (!t) {
    kh::set_error("missing weight %s", name.c_str());
    return KH_ERR_ARG;
  }
  if (t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != cols) {
    kh::set_error("weight %s: expected shape [%lld, %lld]", name.c_str(), (long long)rows, (long long)cols);
    return KH_ERR_ARG;
  }
  int64_t n;
  int rc = st_bytes(*t, name.c_str(), &n);
  if (rc != KH_OK) return rc;
  out->resize((size_t)n);
  if (t->dtype == KH_DT_BF16) {
    memcpy(out->data(), t->data, (size_t)n * 2);
    return KH_OK;
  }
  std::vector<float> f((size_t)n);
  to_f32(*t, n, f.data());
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &f[i], 4);
    if (u & 0xFFFFu) {
      kh::set_error("weight %s holds values that are not BF16 (element %lld); the sparse kernels "
                    "keep BF16 weights", name.c_str(), (long long)i);
      return KH_ERR_UNSUPPORTED;
    }
    (*out)[i] = uint16_t(u >> 16);
  }
  return KH_OK;
}

// The decoder-layer prefixes name_map.rs:36-49 normalises.
int st_layer_name(const kh_safetensors* st, int layer, const char* suffix, std::string* out) {
  const char* pre[] = {"model.layers.", "model.language_model.layers.", "layers."};
  for (const char* p : pre) {
    std::string n = std::string(p) + std::to_string(layer) + "." + suffix;
    if (st_find(st, n)) {
      *out = n;
      return KH_OK;
    }
  }
  *out = std::string("model.layers.") + std::to_string(layer) + "." + suffix;
  return KH_OK;
}

}  // namespace

extern "C" int kh_safetensors_open(const char* path, kh_safetensors** out) {
  KH_CHECK_ARG(path && out, "null argument");
  *out = nullptr;
  auto st = std::make_unique<kh_safetensors>();
  struct stat sb;
  if (stat(path, &sb) != 0) {
    kh::set_error("cannot open %s", path);
    return KH_ERR_ARG;
  }
  if (S_ISDIR(sb.st_mode)) {
    // load_model (loader.rs:30-49): every *.safetensors file, sorted by path
    std::vector<std::string> names;
    DIR* d = opendir(path);
    if (!d) {
      kh::set_error("cannot read directory %s", path);
      return KH_ERR_ARG;
    }
    while (struct dirent* e = readdir(d)) {
      std::string n = e->d_name;
      const std::string ext = ".safetensors";
      if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0)
        names.push_back(std::string(path) + "/" + n);
    }
    closedir(d);
    if (names.empty()) {
      kh::set_error("no .safetensors files found in %s", path);
      return KH_ERR_ARG;
    }
    std::sort(names.begin(), names.end());
    for (const auto& n : names) {
      int rc = st_open_file(st.get(), n);
      if (rc != KH_OK) return rc;
    }
  } else {
    int rc = st_open_file(st.get(), path);
    if (rc != KH_OK) return rc;
  }
  *out = st.release();
  return KH_OK;
}

extern "C" int kh_safetensors_close(kh_safetensors* st) {
  delete st;
  return KH_OK;
}

extern "C" int kh_safetensors_count(const kh_safetensors* st, int64_t* n) {
  KH_CHECK_ARG(st && n, "null argument");
  *n = (int64_t)st->tensors.size();
  return KH_OK;
}

extern "C" int kh_safetensors_name(const kh_safetensors* st, int64_t i, char* buf, int64_t cap) {
  KH_CHECK_ARG(st && buf && cap > 0, "null argument");
  KH_CHECK_ARG(i >= 0 && i < (int64_t)st->tensors.size(), "tensor index %lld out of range", (long long)i);
  auto it = st->tensors.begin();
  std::advance(it, i);
  if ((int64_t)it->first.size() >= cap) {
    kh::set_error("name of tensor %lld needs %zu bytes", (long long)i, it->first.size() + 1);
    return KH_ERR_CAPACITY;
  }
  memcpy(buf, it->first.c_str(), it->first.size() + 1);
  return KH_OK;
}

extern "C" int kh_safetensors_info(const kh_safetensors* st, const char* name, int* dtype, int* ndim,
                                   int64_t* shape, int max_dims) {
  KH_CHECK_ARG(st && name && dtype && ndim, "null argument");
  const auto* t = st_find(st, name);
  if (!t) {
    kh::set_error("missing weight %s", name);
    return KH_ERR_ARG;
  }
  *dtype = t->dtype;
  *ndim = (int)t->shape.size();
  if (shape)
    for (int i = 0; i < std::min(max_dims, *ndim); ++i) shape[i] = t->shape[i];
  return KH_OK;
}

extern "C" int kh_safetensors_read_f32(const kh_safetensors* st, const char* name, float* out_host,
                                       int64_t n) {
  KH_CHECK_ARG(st && name && out_host, "null argument");
  const auto* t = st_find(st, name);
  if (!t) {
    kh::set_error("missing weight %s", name);
    return KH_ERR_ARG;
  }
  int64_t ne;
  int rc = st_bytes(*t, name, &ne);
  if (rc != KH_OK) return rc;
  KH_CHECK_ARG(n == ne, "tensor %s has %lld elements, not %lld", name, (long long)ne, (long long)n);
  to_f32(*t, ne, out_host);
  return KH_OK;
}

extern "C" int kh_safetensors_read_raw(const kh_safetensors* st, const char* name, void* out_host,
                                       int64_t bytes) {
  KH_CHECK_ARG(st && name && out_host, "null argument");
  const auto* t = st_find(st, name);
  if (!t) {
    kh::set_error("missing weight %s", name);
    return KH_ERR_ARG;
  }
  int64_t ne;
  int rc = st_bytes(*t, name, &ne);
  if (rc != KH_OK) return rc;
  int64_t len = ne * elem_size(t->dtype);
  KH_CHECK_ARG(bytes == len, "tensor %s has %lld bytes, not %lld", name, (long long)len, (long long)bytes);
  memcpy(out_host, t->data, (size_t)len);
  return KH_OK;
}

extern "C" int kh_sparse_ffn_create_from_safetensors(const kh_safetensors* st, int layer, int max_batch,
                                                     kh_sparse_ffn** out) {
  KH_CHECK_ARG(st && out, "null argument");
  KH_CHECK_ARG(layer >= 0, "layer must be non-negative");
  *out = nullptr;
  std::string gn, un, dn;
  st_layer_name(st, layer, "mlp.gate_proj.weight", &gn);
  st_layer_name(st, layer, "mlp.up_proj.weight", &un);
  st_layer_name(st, layer, "mlp.down_proj.weight", &dn);
  const auto* g = st_find(st, gn);
  if (!g || g->shape.size() != 2) {
    kh::set_error("missing or non-2D weight %s", gn.c_str());
    return KH_ERR_ARG;
  }
  KH_CHECK_ARG(g->shape[0] <= INT32_MAX && g->shape[1] <= INT32_MAX, "weight %s too large", gn.c_str());
  const int inter = (int)g->shape[0], hidden = (int)g->shape[1];
  std::vector<uint16_t> wg, wu, wd;
  int rc = st_bf16_matrix(st, gn, inter, hidden, &wg);
  if (rc == KH_OK) rc = st_bf16_matrix(st, un, inter, hidden, &wu);
  if (rc == KH_OK) rc = st_bf16_matrix(st, dn, hidden, inter, &wd);
  if (rc != KH_OK) return rc;
  return kh_sparse_ffn_create(hidden, inter, wg.data(), wu.data(), wd.data(), max_batch, out);
}

extern "C" int kh_sparse_attn_create_from_safetensors(const kh_safetensors* st, int layer, int num_heads,
                                                      int num_kv_heads, int head_dim, int max_seq,
                                                      int max_batch, float rope_theta, int kv_dtype,
                                                      kh_sparse_attn** out) {
  KH_CHECK_ARG(st && out, "null argument");
  KH_CHECK_ARG(layer >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0, "bad dimensions");
  *out = nullptr;
  std::string qn, kn, vn, on;
  st_layer_name(st, layer, "self_attn.q_proj.weight", &qn);
  st_layer_name(st, layer, "self_attn.k_proj.weight", &kn);
  st_layer_name(st, layer, "self_attn.v_proj.weight", &vn);
  st_layer_name(st, layer, "self_attn.o_proj.weight", &on);
  const auto* q = st_find(st, qn);
  if (!q || q->shape.size() != 2) {
    kh::set_error("missing or non-2D weight %s", qn.c_str());
    return KH_ERR_ARG;
  }
  KH_CHECK_ARG(q->shape[1] <= INT32_MAX, "weight %s too large", qn.c_str());
  const int hidden = (int)q->shape[1];
  const int64_t qd = (int64_t)num_heads * head_dim, kvd = (int64_t)num_kv_heads * head_dim;
  std::vector<uint16_t> wq, wk, wv, wo;
  int rc = st_bf16_matrix(st, qn, qd, hidden, &wq);
  if (rc == KH_OK) rc = st_bf16_matrix(st, kn, kvd, hidden, &wk);
  if (rc == KH_OK) rc = st_bf16_matrix(st, vn, kvd, hidden, &wv);
  if (rc == KH_OK) rc = st_bf16_matrix(st, on, hidden, qd, &wo);
  if (rc != KH_OK) return rc;
  return kh_sparse_attn_create(hidden, num_heads, num_kv_heads, head_dim, max_seq, max_batch, rope_theta,
                               kv_dtype, wq.data(), wk.data(), wv.data(), wo.data(), out);
}

// ---- SparsityPredictor JSON -------------------------------------------------

namespace {

struct PredFile {
  std::vector<float> w1, b1, w2, b2;
  size_t in = 0, hid = 0, out = 0;
};

// serde's derived Deserialize for SparsityPredictor: every field required,
// unknown fields ignored, any field order.  The dims must agree with the
// arrays (the reference's zips would silently truncate on a mismatch).
int parse_predictor(const char* path, PredFile* f) {
  std::string text;
  int rc = read_text(path, &text);
  if (rc != KH_OK) return rc;
  Json j{text.data(), text.data() + text.size(), {}};
  size_t r1 = 0, c1 = 0, r2 = 0, c2 = 0, nb1 = 0, nb2 = 0;
  uint64_t din = 0, dh = 0, dout = 0;
  unsigned seen = 0;
  bool ok = j.expect('{');
  if (ok && !j.eat('}')) {
    do {
      std::string key;
      if (!(ok = j.string(&key) && j.expect(':'))) break;
      if (key == "w1") ok = j.f32_matrix(&f->w1, &r1, &c1), seen |= 1;
      else if (key == "b1") ok = j.f32_array(&f->b1, &nb1), seen |= 2;
      else if (key == "w2") ok = j.f32_matrix(&f->w2, &r2, &c2), seen |= 4;
      else if (key == "b2") ok = j.f32_array(&f->b2, &nb2), seen |= 8;
      else if (key == "input_dim") ok = j.u64(&din), seen |= 16;
      else if (key == "hidden_dim") ok = j.u64(&dh), seen |= 32;
      else if (key == "output_dim") ok = j.u64(&dout), seen |= 64;
      else ok = j.skip();
    } while (ok && j.eat(','));
    if (ok) ok = j.expect('}');
  }
  if (ok) ok = j.done();
  if (!ok) {
    kh::set_error("%s: bad predictor JSON: %s at byte %zu", path, j.err.c_str(), (size_t)(j.p - text.data()));
    return KH_ERR_ARG;
  }
  if (seen != 127) {
    kh::set_error("%s: predictor JSON lacks a field of w1,b1,w2,b2,input_dim,hidden_dim,output_dim", path);
    return KH_ERR_ARG;
  }
  if (r1 != dh || c1 != din || nb1 != dh || r2 != dout || c2 != dh || nb2 != dout || !din || !dh || !dout ||
      din > INT32_MAX || dh > INT32_MAX || dout > INT32_MAX) {
    kh::set_error("%s: predictor arrays disagree with input_dim %llu, hidden_dim %llu, output_dim %llu", path,
                  (unsigned long long)din, (unsigned long long)dh, (unsigned long long)dout);
    return KH_ERR_ARG;
  }
  f->in = din;
  f->hid = dh;
  f->out = dout;
  return KH_OK;
}

// The shortest decimal that reads back as v, laid out as serde_json writes an
// f32 (ryu): with digits d1..dn and 10^(kk-1) <= |v| < 10^kk, positional when
// -6 < kk <= 13 ("16777216.0", "0.1", "0.000001"), else scientific ("1e-7",
// "1.5e13", "-3.4028235e38").
void put_f32(std::string& s, float v) {
  char b[48];
  auto r = std::to_chars(b, b + sizeof b, v, std::chars_format::scientific);
  std::string t(b, r.ptr);  // "-d.ddde+XX"
  bool neg = t[0] == '-';
  if (neg) t.erase(0, 1);
  size_t e = t.find('e');
  std::string digits;
  for (size_t i = 0; i < e; ++i)
    if (t[i] != '.') digits += t[i];
  int exp10 = std::stoi(t.substr(e + 1));  // value = d1.d2..dn * 10^exp10
  if (neg) s += '-';
  if (digits == "0") {
    s += "0.0";
    return;
  }
  const int n = (int)digits.size();
  const int kk = exp10 + 1;
  if (kk > 0 && kk <= 13) {
    if (n <= kk) {
      s += digits;
      s.append((size_t)(kk - n), '0');
      s += ".0";
    } else {
      s += digits.substr(0, kk);
      s += '.';
      s += digits.substr(kk);
    }
  } else if (kk > -6 && kk <= 0) {
    s += "0.";
    s.append((size_t)(-kk), '0');
    s += digits;
  } else {
    s += digits[0];
    if (n > 1) {
      s += '.';
      s += digits.substr(1);
    }
    s += 'e';
    s += std::to_string(kk - 1);
  }
}

void put_array(std::string& s, const float* a, size_t n) {
  s += '[';
  for (size_t i = 0; i < n; ++i) {
    if (i) s += ',';
    put_f32(s, a[i]);
  }
  s += ']';
}

void put_matrix(std::string& s, const float* a, size_t rows, size_t cols) {
  s += '[';
  for (size_t r = 0; r < rows; ++r) {
    if (r) s += ',';
    put_array(s, a + r * cols, cols);
  }
  s += ']';
}

}  // namespace

extern "C" int kh_predictor_read_json(const char* path, int* input_dim, int* hidden_dim, int* output_dim,
                                      float* w1_host, float* b1_host, float* w2_host, float* b2_host) {
  KH_CHECK_ARG(path && input_dim && hidden_dim && output_dim, "null argument");
  PredFile f;
  int rc = parse_predictor(path, &f);
  if (rc != KH_OK) return rc;
  *input_dim = (int)f.in;
  *hidden_dim = (int)f.hid;
  *output_dim = (int)f.out;
  if (w1_host) memcpy(w1_host, f.w1.data(), f.w1.size() * 4);
  if (b1_host) memcpy(b1_host, f.b1.data(), f.b1.size() * 4);
  if (w2_host) memcpy(w2_host, f.w2.data(), f.w2.size() * 4);
  if (b2_host) memcpy(b2_host, f.b2.data(), f.b2.size() * 4);
  return KH_OK;
}

extern "C" int kh_predictor_load(const char* path, kh_predictor** out) {
  KH_CHECK_ARG(path && out, "null argument");
  *out = nullptr;
  PredFile f;
  int rc = parse_predictor(path, &f);
  if (rc != KH_OK) return rc;
  return kh_predictor_create((int)f.in, (int)f.hid, (int)f.out, f.w1.data(), f.b1.data(), f.w2.data(),
                             f.b2.data(), out);
}

extern "C" int kh_predictor_write_json(const char* path, int input_dim, int hidden_dim, int output_dim,
                                       const float* w1_host, const float* b1_host, const float* w2_host,
                                       const float* b2_host) {
  KH_CHECK_ARG(path && w1_host && b1_host && w2_host && b2_host, "null argument");
  KH_CHECK_ARG(input_dim > 0 && hidden_dim > 0 && output_dim > 0, "dims must be positive");
  const size_t din = input_dim, dh = hidden_dim, dout = output_dim;
  for (const auto& a : {std::make_pair(w1_host, din * dh), std::make_pair(b1_host, dh),
                        std::make_pair(w2_host, dh * dout), std::make_pair(b2_host, dout)})
    for (size_t i = 0; i < a.second; ++i)
      KH_CHECK_ARG(std::isfinite(a.first[i]), "non-finite weight: serde_json would write null");
  std::string s;
  s.reserve((din * dh + dh * dout) * 12 + 256);
  s += "{\"w1\":";
  put_matrix(s, w1_host, dh, din);
  s += ",\"b1\":";
  put_array(s, b1_host, dh);
  s += ",\"w2\":";
  put_matrix(s, w2_host, dout, dh);
  s += ",\"b2\":";
  put_array(s, b2_host, dout);
  s += ",\"input_dim\":" + std::to_string(din) + ",\"hidden_dim\":" + std::to_string(dh) +
       ",\"output_dim\":" + std::to_string(dout) + "}";
  FILE* fp = fopen(path, "wb");
  if (!fp) {
    kh::set_error("cannot write %s", path);
    return KH_ERR_ARG;
  }
  size_t w = fwrite(s.data(), 1, s.size(), fp);
  int cl = fclose(fp);
  if (w != s.size() || cl != 0) {
    kh::set_error("short write to %s", path);
    return KH_ERR_ARG;
  }
  return KH_OK;
}

extern "C" int kh_predictor_save(const kh_predictor* p, const char* path) {
  KH_CHECK_ARG(p && path, "null argument");
  int din, dh, dout;
  int rc = kh_predictor_dims(p, &din, &dh, &dout);
  if (rc != KH_OK) return rc;
  std::vector<float> w1((size_t)din * dh), b1(dh), w2((size_t)dh * dout), b2(dout);
  rc = kh_predictor_weights(p, w1.data(), b1.data(), w2.data(), b2.data());
  if (rc != KH_OK) return rc;
  return kh_predictor_write_json(path, din, dh, dout, w1.data(), b1.data(), w2.data(), b2.data());
}
