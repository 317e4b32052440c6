// runtime.cpp -- error reporting and device allocation for the C ABI.
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

Scratch::~Scratch() { dev_free(p); }

void* Scratch::get(size_t bytes) {
  if (bytes <= cap) return p;
  dev_free(p);
  p = dev_alloc(bytes);
  cap = p ? bytes : 0;
  return p;
}

}  // namespace kh

extern "C" const char* kh_last_error(void) { return kh::g_last_error.c_str(); }

extern "C" int kh_version(void) { return 1; }
