// libsvm.cpp -- LibSvmDataset (crates/klearu-core/src/data/libsvm.rs:31-183):
// the extreme-classification text format read on the host into CSR arrays
// that the training and inference entry points take as device CSR.
//
// Line format: `l1,l2,... idx:val idx:val ...`; blank lines and lines whose
// first non-blank character is '#' are skipped, and a token starting with '#'
// ends a line's features.  Indices are shifted down by one when no index 0
// appears anywhere and the smallest index is 1; indices at or past
// feature_dim are clamped to feature_dim - 1; each example's pairs are sorted
// by index (stable) and repeated indices summed in that order
// (SparseVector::from_pairs, tensor/sparse.rs:36-57).
//
// Numbers parse as Rust's FromStr does: u32 = optional '+', ASCII digits, no
// overflow; f32 = optional sign, then decimal digits with an optional point
// and exponent, or inf / infinity / nan in any case, rounded once to the
// nearest f32 (std::from_chars<float> rounds correctly).  Whitespace is the
// ASCII set Rust's char::is_whitespace contains; bytes >= 0x80 are treated as
// ordinary characters (the reference would also accept Unicode spaces).
#include <algorithm>
#include <charconv>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

using namespace kh;

struct kh_libsvm {
  int64_t feature_dim = 0, num_labels = 0;
  std::vector<int64_t> off{0};     // [n+1]
  std::vector<uint32_t> idx;       // [nnz]
  std::vector<float> val;          // [nnz]
  std::vector<int64_t> loff{0};    // [n+1]
  std::vector<uint32_t> labels;
};

namespace {

bool is_ws(char c) { return c == ' ' || (c >= '\t' && c <= '\r'); }

// u32::from_str
bool parse_u32(const char* b, const char* e, uint32_t* out) {
  if (b < e && *b == '+') ++b;
  if (b == e) return false;
  for (const char* p = b; p < e; ++p)
    if (*p < '0' || *p > '9') return false;
  uint64_t v = 0;
  for (const char* p = b; p < e; ++p) {
    v = v * 10 + static_cast<uint64_t>(*p - '0');
    if (v > 0xffffffffull) return false;
  }
  *out = static_cast<uint32_t>(v);
  return true;
}

// f32::from_str
bool parse_f32(const char* b, const char* e, float* out) {
  if (b == e) return false;
  bool neg = false;
  if (*b == '+' || *b == '-') {
    neg = *b == '-';
    ++b;
  }
  if (b == e || *b == '+' || *b == '-') return false;
  std::string lower;
  for (const char* p = b; p < e; ++p) lower.push_back(static_cast<char>(std::tolower(static_cast<unsigned char>(*p))));
  float v;
  if (lower == "inf" || lower == "infinity") {
    v = __builtin_inff();
  } else if (lower == "nan") {
    v = __builtin_nanf("");
  } else {
    // decimal only: digits, at most one point, an optional exponent
    bool digit = false;
    const char* p = b;
    while (p < e && *p >= '0' && *p <= '9') ++p, digit = true;
    if (p < e && *p == '.') {
      ++p;
      while (p < e && *p >= '0' && *p <= '9') ++p, digit = true;
    }
    if (!digit) return false;
    if (p < e && (*p == 'e' || *p == 'E')) {
      ++p;
      if (p < e && (*p == '+' || *p == '-')) ++p;
      const char* q = p;
      while (p < e && *p >= '0' && *p <= '9') ++p;
      if (p == q) return false;
    }
    if (p != e) return false;
    auto r = std::from_chars(b, e, v, std::chars_format::general);
    if (r.ec == std::errc::result_out_of_range) {
      // from_chars leaves v unset when the float result under- or overflows:
      // take the double and round it to float; beyond double's range the
      // exponent's sign decides between inf and zero
      double d = 0.0;
      if (std::from_chars(b, e, d, std::chars_format::general).ec == std::errc()) {
        v = static_cast<float>(d);
      } else {
        const char* ep = std::find_if(b, e, [](char c) { return c == 'e' || c == 'E'; });
        v = (ep == e || ep[1] != '-') ? __builtin_inff() : 0.0f;
      }
    } else if (r.ec != std::errc() || r.ptr != e) {
      return false;
    }
  }
  *out = neg ? -v : v;
  return true;
}

struct Raw {
  std::vector<uint32_t> labels;
  std::vector<std::pair<uint32_t, float>> feats;
};

int parse_all(const char* data, size_t len, int64_t feature_dim, int64_t num_labels,
              kh_libsvm** out) {
  KH_CHECK_ARG(feature_dim > 0 && feature_dim <= 0x100000000ll, "feature_dim must be in [1, 2^32]");
  KH_CHECK_ARG(num_labels >= 0, "num_labels must be non-negative");
  std::vector<Raw> raw;
  bool has_zero = false, any = false;
  uint32_t min_idx = 0;
  size_t pos = 0;
  int64_t line_no = 0;
  while (pos < len) {
    size_t end = pos;
    while (end < len && data[end] != '\n') ++end;
    const char* b = data + pos;
    const char* e = data + end;
    pos = end + 1;
    ++line_no;
    while (b < e && is_ws(*b)) ++b;
    while (e > b && is_ws(e[-1])) --e;
    if (b == e || *b == '#') continue;
    Raw r;
    // first token: labels
    const char* t = b;
    while (t < e && !is_ws(*t)) ++t;
    for (const char* s = b;;) {
      const char* c = std::find(s, t, ',');
      uint32_t lab;
      if (!parse_u32(s, c, &lab)) {
        set_error("line %lld: invalid label '%.*s'", (long long)line_no, (int)(c - s), s);
        return KH_ERR_ARG;
      }
      r.labels.push_back(lab);
      if (c == t) break;
      s = c + 1;
    }
    // features
    const char* p = t;
    for (;;) {
      while (p < e && is_ws(*p)) ++p;
      if (p == e || *p == '#') break;
      const char* q = p;
      while (q < e && !is_ws(*q)) ++q;
      const char* colon = std::find(p, q, ':');
      if (colon == q) {
        set_error("line %lld: expected 'index:value', got '%.*s'", (long long)line_no, (int)(q - p), p);
        return KH_ERR_ARG;
      }
      uint32_t ix;
      float v;
      if (!parse_u32(p, colon, &ix)) {
        set_error("line %lld: invalid feature index '%.*s'", (long long)line_no, (int)(colon - p), p);
        return KH_ERR_ARG;
      }
      if (!parse_f32(colon + 1, q, &v)) {
        set_error("line %lld: invalid feature value '%.*s'", (long long)line_no, (int)(q - colon - 1),
                  colon + 1);
        return KH_ERR_ARG;
      }
      if (ix == 0) has_zero = true;
      min_idx = any ? std::min(min_idx, ix) : ix;
      any = true;
      r.feats.emplace_back(ix, v);
      p = q;
    }
    raw.push_back(std::move(r));
  }
  const uint32_t offset = (!has_zero && any && min_idx == 1) ? 1u : 0u;
  auto* ds = new kh_libsvm();
  ds->feature_dim = feature_dim;
  ds->num_labels = num_labels;
  for (Raw& r : raw) {
    for (auto& f : r.feats) {
      const uint32_t a = f.first - offset;
      f.first = static_cast<int64_t>(a) >= feature_dim ? static_cast<uint32_t>(feature_dim - 1) : a;
    }
    std::stable_sort(r.feats.begin(), r.feats.end(),
                     [](const auto& x, const auto& y) { return x.first < y.first; });
    for (const auto& f : r.feats) {
      if (!ds->idx.empty() && static_cast<int64_t>(ds->idx.size()) > ds->off.back() &&
          ds->idx.back() == f.first) {
        ds->val.back() = ds->val.back() + f.second;  // from_pairs: repeated index accumulates
        continue;
      }
      ds->idx.push_back(f.first);
      ds->val.push_back(f.second);
    }
    ds->off.push_back(static_cast<int64_t>(ds->idx.size()));
    ds->labels.insert(ds->labels.end(), r.labels.begin(), r.labels.end());
    ds->loff.push_back(static_cast<int64_t>(ds->labels.size()));
  }
  *out = ds;
  return KH_OK;
}

}  // namespace

extern "C" int kh_libsvm_parse(const char* data, int64_t len, int64_t feature_dim, int64_t num_labels,
                               kh_libsvm** out) {
  KH_CHECK_ARG(out != nullptr && (data != nullptr || len == 0) && len >= 0, "null argument");
  *out = nullptr;
  return parse_all(data, static_cast<size_t>(len), feature_dim, num_labels, out);
}

extern "C" int kh_libsvm_load(const char* path, int64_t feature_dim, int64_t num_labels,
                              kh_libsvm** out) {
  KH_CHECK_ARG(path != nullptr && out != nullptr, "null argument");
  *out = nullptr;
  FILE* f = std::fopen(path, "rb");
  KH_CHECK_ARG(f != nullptr, "cannot open %s", path);
  std::vector<char> buf;
  char tmp[1 << 16];
  size_t n;
  while ((n = std::fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + n);
  const bool err = std::ferror(f) != 0;
  std::fclose(f);
  KH_CHECK_ARG(!err, "read error on %s", path);
  return parse_all(buf.data(), buf.size(), feature_dim, num_labels, out);
}

extern "C" int kh_libsvm_free(kh_libsvm* ds) {
  delete ds;
  return KH_OK;
}

extern "C" int kh_libsvm_dims(const kh_libsvm* ds, int64_t* n, int64_t* nnz, int64_t* n_labels,
                              int64_t* feature_dim, int64_t* num_labels) {
  KH_CHECK_ARG(ds != nullptr, "null dataset");
  if (n) *n = static_cast<int64_t>(ds->off.size()) - 1;
  if (nnz) *nnz = static_cast<int64_t>(ds->idx.size());
  if (n_labels) *n_labels = static_cast<int64_t>(ds->labels.size());
  if (feature_dim) *feature_dim = ds->feature_dim;
  if (num_labels) *num_labels = ds->num_labels;
  return KH_OK;
}

extern "C" int kh_libsvm_copy(const kh_libsvm* ds, int64_t* off, uint32_t* idx, float* val,
                              int64_t* label_off, uint32_t* labels) {
  KH_CHECK_ARG(ds != nullptr, "null dataset");
  if (off) std::memcpy(off, ds->off.data(), sizeof(int64_t) * ds->off.size());
  if (idx && !ds->idx.empty()) std::memcpy(idx, ds->idx.data(), sizeof(uint32_t) * ds->idx.size());
  if (val && !ds->val.empty()) std::memcpy(val, ds->val.data(), sizeof(float) * ds->val.size());
  if (label_off) std::memcpy(label_off, ds->loff.data(), sizeof(int64_t) * ds->loff.size());
  if (labels && !ds->labels.empty())
    std::memcpy(labels, ds->labels.data(), sizeof(uint32_t) * ds->labels.size());
  return KH_OK;
}

extern "C" int kh_libsvm_upload(const kh_libsvm* ds, int64_t row0, int64_t rows, int64_t* off_dev,
                                uint32_t* idx_dev, float* val_dev, void* stream) {
  KH_CHECK_ARG(ds != nullptr, "null dataset");
  const int64_t n = static_cast<int64_t>(ds->off.size()) - 1;
  KH_CHECK_ARG(row0 >= 0 && rows >= 0 && row0 + rows <= n, "rows [%lld, %lld) not in [0, %lld)",
               (long long)row0, (long long)(row0 + rows), (long long)n);
  KH_CHECK_ARG(off_dev != nullptr, "null offsets");
  const int64_t a = ds->off[row0], b = ds->off[row0 + rows];
  std::vector<int64_t> o(rows + 1);
  for (int64_t i = 0; i <= rows; ++i) o[i] = ds->off[row0 + i] - a;
  hipStream_t st = as_stream(stream);
  KH_HIP(hipMemcpyAsync(off_dev, o.data(), sizeof(int64_t) * (rows + 1), hipMemcpyHostToDevice, st));
  if (b > a) {
    KH_CHECK_ARG(idx_dev && val_dev, "null CSR arrays");
    KH_HIP(hipMemcpyAsync(idx_dev, ds->idx.data() + a, sizeof(uint32_t) * (b - a), hipMemcpyHostToDevice, st));
    KH_HIP(hipMemcpyAsync(val_dev, ds->val.data() + a, sizeof(float) * (b - a), hipMemcpyHostToDevice, st));
  }
  KH_HIP(hipStreamSynchronize(st));  // the host staging vector goes out of scope
  return KH_OK;
}
