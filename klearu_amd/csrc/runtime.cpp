// runtime.cpp -- error reporting and device allocation for the C ABI.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.hpp"

namespace kh {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void* dev_alloc(size_t bytes) {
  void* p = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

Scratch::~Scratch() {
  dev_free(p);
  for (void* r : retired) dev_free(r);
}

void* Scratch::get(size_t bytes, bool zero) {
  if (bytes <= cap && p) return p;
  const size_t want = cap ? std::max(bytes, cap + cap / 2) : bytes;
  void* q = dev_alloc(want);
  if (!q) return nullptr;
  if (zero && hipMemset(q, 0, want) != hipSuccess) {
    set_error("hipMemset of a new workspace failed");
    dev_free(q);
    return nullptr;
  }
  if (p) retired.push_back(p);
  p = q;
  cap = want;
  return p;
}

WsSet* StreamWs::get(hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  for (auto& e : sets_)
    if (e.first == s) return e.second.get();
  sets_.emplace_back(s, std::make_unique<WsSet>());
  return sets_.back().second.get();
}

}  // namespace kh

extern "C" const char* kh_last_error(void) { return kh::g_last_error.c_str(); }

extern "C" int kh_version(void) { return 1; }
