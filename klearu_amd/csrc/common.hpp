// common.hpp -- shared helpers for libklearu_hip.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/klearu_hip.h"

namespace kh {

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define KH_CHECK_ARG(cond, ...)        \
  do {                                 \
    if (!(cond)) {                     \
      ::kh::set_error(__VA_ARGS__);    \
      return KH_ERR_ARG;               \
    }                                  \
  } while (0)

#define KH_HIP(call)                                                                \
  do {                                                                              \
    hipError_t e_ = (call);                                                         \
    if (e_ != hipSuccess) {                                                         \
      ::kh::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                      __LINE__);                                                    \
      return KH_ERR_HIP;                                                            \
    }                                                                               \
  } while (0)

// Checks the launch that was just enqueued.
#define KH_LAUNCHED()                                                              \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess) {                                                        \
      ::kh::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(e_),   \
                      __FILE__, __LINE__);                                         \
      return KH_ERR_HIP;                                                           \
    }                                                                              \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Device allocation that records the failure; returns nullptr on error.
void* dev_alloc(size_t bytes);
void dev_free(void* p);

// Grow-only device buffer owned by a handle.  A buffer that is replaced by a
// larger one stays allocated until the owner is destroyed, so a HIP graph
// captured before the growth never points at freed memory.
struct Scratch {
  void* p = nullptr;
  size_t cap = 0;
  std::vector<void*> retired;
  Scratch() = default;
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  ~Scratch();
  // At least `bytes` (grown by half again when it grows); zero-filled on
  // allocation when `zero` (the fill is synchronous).
  void* get(size_t bytes, bool zero = false);
};

// Device scratch of a handle, one set of kWsSlots buffers per stream.  Calls
// on one stream are ordered by it and share a set; calls on different streams
// get different sets, so a handle's non-mutating calls (the reference's
// `&self` methods, which are Send + Sync) may run concurrently on distinct
// streams and host threads.  Sets live until the handle is destroyed.
constexpr int kWsSlots = 8;
struct WsSet {
  std::mutex mu;  // host threads sharing a stream
  Scratch slot[kWsSlots];
  void* get(int s, size_t bytes, bool zero = false) {
    std::lock_guard<std::mutex> g(mu);
    return slot[s].get(bytes, zero);
  }
};
class StreamWs {
 public:
  WsSet* get(hipStream_t s);
 private:
  std::mutex mu_;
  std::vector<std::pair<hipStream_t, std::unique_ptr<WsSet>>> sets_;
};

// ---------------------------------------------------------------- device helpers
constexpr int kWave = 64;
constexpr int kMaxDynLds = 152 * 1024;  // dynamic LDS ceiling (160 KB per CU minus static use)

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Streaming 16-byte load / store (nontemporal hint): for weight rows that are
// read exactly once per call and for per-block partial rows that another
// kernel reads back.  Measured on the batch-1 FFN gather: 10.2 -> 9.3 us for
// 40.6 MB of rows, against plain loads.
typedef unsigned kh_u32x4 __attribute__((ext_vector_type(4)));
typedef float kh_f32x4_st __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const kh_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const kh_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(float4* p, float4 v) {
  const kh_f32x4_st t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<kh_f32x4_st*>(p));
}

// Round to nearest even; NaN keeps its top bits and is forced quiet.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// ---------------------------------------------------------------- DPP lane moves
// Cross-lane moves through the DPP operand modifier (GFX9 encodings): a VALU
// operand read from another lane, with no LDS round trip (ds_bpermute, behind
// __shfl*, costs an LDS latency per step).  Every lane of the wave must be
// active where these are used.
constexpr int kDppQuadSwap1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowMirror = 0x140;     // lane i <- 15 - i within a row of 16
constexpr int kDppRowHalfMirror = 0x141; // lane i <- 7 - i within each half row
constexpr int kDppRowBcast15 = 0x142;    // lane 15 of row r -> row r + 1
constexpr int kDppRowBcast31 = 0x143;    // lane 31 -> rows 2 and 3

// Value of lane (permutation CTRL); rows outside ROWS, and lanes whose source
// lies outside their row, read 0.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(dpp<CTRL, ROWS>(__float_as_int(v)));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sum over each aligned group of G lanes (G = 2, 4, 8 or 16); every lane of
// the group gets the same value (a butterfly: each step adds a lane pairing).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  v += dppf<kDppQuadSwap1>(v);
  if (G >= 4) v += dppf<kDppQuadSwap2>(v);
  if (G >= 8) v += dppf<kDppRowHalfMirror>(v);
  if (G >= 16) v += dppf<kDppRowMirror>(v);
  return v;
}

// Sum over the 64 lanes of a wave (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dppf<kDppQuadSwap1>(v));
  v = fmaxf(v, dppf<kDppQuadSwap2>(v));
  v = fmaxf(v, dppf<kDppRowHalfMirror>(v));
  v = fmaxf(v, dppf<kDppRowMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp<kDppQuadSwap1>((int)v));
  v = max(v, (uint32_t)dpp<kDppQuadSwap2>((int)v));
  v = max(v, (uint32_t)dpp<kDppRowHalfMirror>((int)v));
  v = max(v, (uint32_t)dpp<kDppRowMirror>((int)v));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return ~wave_max_u32(~v);
}
// Inclusive prefix sum over the lanes of a wave (Hillis-Steele within rows
// of 16, then the row totals carried across rows).
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += dpp<kDppRowShr1>(x);
  x += dpp<kDppRowShr2>(x);
  x += dpp<kDppRowShr4>(x);
  x += dpp<kDppRowShr8>(x);
  x += dpp<kDppRowBcast15, 0xa>(x);
  x += dpp<kDppRowBcast31, 0xc>(x);
  return x;
}

// expf exactly as glibc computes it on x86-64 (the libm behind Rust's
// f32::exp): the published ARM optimized-routines algorithm with a 32-entry
// table of 2^(i/32) and a cubic in double precision, with the FMAs of glibc's
// FMA build (range reduction fused into both of its uses).  Checked equal to
// glibc expf for every non-NaN f32 input.
__device__ __constant__ const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
template <typename Tab>
__device__ __forceinline__ float expf_glibc_t(float x, const Tab& tab) {
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return __int_as_float(0x7f800000);
  if (x < -0x1.9fe368p6f) return 0.0f;
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  const double kShift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = static_cast<double>(x);
  double kd = fma(kInvLn2N, xd, kShift);
  const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd = kd - kShift;
  const double r = fma(kInvLn2N, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __longlong_as_double(static_cast<long long>(t));
  const double z = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_t(x, kExp2Tab); }

// 1 / (1 + exp(-z)) with IEEE f32 add and divide; `tab` may be an LDS copy of
// kExp2Tab when many lanes evaluate different arguments.
template <typename Tab>
__device__ __forceinline__ float sigmoid_ref_t(float z, const Tab& tab) {
  float e = expf_glibc_t(-z, tab);
  float d = __fadd_rn(1.0f, e);
  return __fdiv_rn(1.0f, d);
}
// 1 / (1 + exp(-z)) with IEEE f32 add and divide.
__device__ __forceinline__ float sigmoid_ref(float z) {
  float e = expf_glibc(-z);
  float d = __fadd_rn(1.0f, e);
  return __fdiv_rn(1.0f, d);
}
// z / (1 + exp(-z)) with the 2^(i/32) table at `tab` (an LDS copy of
// kExp2Tab: a lookup from constant memory whose index depends on the value
// just computed costs a full memory round trip on the kernel's critical path).
template <typename Tab>
__device__ __forceinline__ float silu_ref_t(float z, const Tab& tab) {
  float e = expf_glibc_t(-z, tab);
  float d = __fadd_rn(1.0f, e);
  return __fdiv_rn(z, d);
}
// z / (1 + exp(-z)).
__device__ __forceinline__ float silu_ref(float z) {
  float e = expf_glibc(-z);
  float d = __fadd_rn(1.0f, e);
  return __fdiv_rn(z, d);
}

// Order-preserving key of an f32 (larger float -> larger key); -0.0 maps to
// the key of +0.0 so that they compare equal, as partial_cmp does.
__device__ __forceinline__ uint32_t f32_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum of v over the block (blockDim.x a multiple of 64, at
// most 1024).  wsum: shared scratch of blockDim.x/64 ints; *total (shared)
// receives the block total.  Contains two __syncthreads.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  const int nw = blockDim.x >> 6;
  int before = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    const int t = wsum[i];
    before += i < w ? t : 0;
    tot += t;
  }
  if (threadIdx.x == 0) *total = tot;
  __syncthreads();
  return before + x - v;
}

// Same for unsigned 32-bit sums (wrapping arithmetic), e.g. two packed 16-bit counts.
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
  x += (uint32_t)dpp<kDppRowShr1>((int)x);
  x += (uint32_t)dpp<kDppRowShr2>((int)x);
  x += (uint32_t)dpp<kDppRowShr4>((int)x);
  x += (uint32_t)dpp<kDppRowShr8>((int)x);
  x += (uint32_t)dpp<kDppRowBcast15, 0xa>((int)x);
  x += (uint32_t)dpp<kDppRowBcast31, 0xc>((int)x);
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i) before += wsum[i];
  __syncthreads();
  return before + x - v;
}

// RmsNorm applied inside a consumer kernel.  The first kernel that reads the
// un-normalised row (the predictor's layer 1) computes the reference's exact
// scale 1/sqrt(sum_sq/n + eps) and writes it to inv[row]; the kernels after
// it read inv.  w == nullptr means the input is used as is.
struct NormIn {
  const float* w = nullptr;
  float* inv = nullptr;
  float eps = 0.0f;
};

// Cross-file helpers of the fused Deja Vu MLP block (predictor.hip).
int predictor_in_dim(const kh_predictor* p);
int predictor_out_dim(const kh_predictor* p);
int predictor_topk_normed(const kh_predictor* p, const float* hidden, int k, int32_t* ids,
                          const NormIn& nrm, hipStream_t st);
// Layers 1 and 2 of one row into the per-stream score buffer, with layer 2's
// per-block key bounds, for a consumer kernel that selects the top k itself
// (rows of more than 64 outputs whose bounds fit; KH_ERR_UNSUPPORTED otherwise,
// before anything is launched).
struct PredScores {
  const float* scores = nullptr;  // [out_dim]
  const uint32_t* mm = nullptr;   // [nmm] (min key, max key) pairs
  int n = 0, nmm = 0;
};
int predictor_scores_normed(const kh_predictor* p, const float* hidden, const NormIn& nrm,
                            hipStream_t st, PredScores* out);
// Layer 1 of a single-row call launched by another file's kernel (its weights,
// and the per-stream buffer that layer 2 reads), then layers 2 and the top k
// in ascending order from that buffer.
struct PredL1View {
  const void* w1b = nullptr;   // [ceil(in/8)][hid][8], BF16 bits when bf16
  const float* b1 = nullptr;
  const void* w2b = nullptr;   // [ceil(hid/8)][out][8], BF16 bits when bf16
  const float* b2 = nullptr;
  int in_dim = 0, hid = 0, out_dim = 0;
  bool bf16 = false;
  float* hbuf = nullptr;       // [hid] layer-1 outputs of one row
};
int predictor_l1_view(const kh_predictor* p, hipStream_t st, PredL1View* v, int64_t batch = 1);
int predictor_l2_topk_from_h(const kh_predictor* p, int k, int32_t* ids, hipStream_t st);
int predictor_select_marks(const kh_predictor* p, const float* x, int64_t batch, int k, int32_t* ids,
                           hipStream_t st, uint8_t** marks);
int predictor_l1_normed(const kh_predictor* p, const float* hidden, int64_t batch, const NormIn& nrm,
                        float* xn, hipStream_t st, PredL1View* v);

// Workgroup barrier that waits only for LDS traffic.  __syncthreads() on gfx9
// also waits for every outstanding vector-memory load (vmcnt counts loads and
// stores together), which would drain global prefetches issued before it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Block-cooperative copy of n4 float4s from global memory to LDS with four
// loads in flight per thread before any store (a plain strided loop would
// wait one memory round trip per iteration).  Loads and stores are clamped,
// not conditional: a conditional store lets the compiler sink each load into
// its branch, one round trip per load.  Past the end a thread rewrites the
// last float4 with the value it loaded from there.
__device__ __forceinline__ void stage_f4(float4* __restrict__ dst, const float4* __restrict__ src,
                                         int n4) {
  constexpr int U = 4;
  for (int base = threadIdx.x; base < n4; base += blockDim.x * U) {
    float4 v[U];
#pragma unroll
    for (int q = 0; q < U; ++q) v[q] = src[min(base + q * (int)blockDim.x, n4 - 1)];
#pragma unroll
    for (int q = 0; q < U; ++q) dst[min(base + q * (int)blockDim.x, n4 - 1)] = v[q];
  }
}

inline int ceil_div(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

// A row index from a caller's list, kept inside [0, n): an index outside it
// (the reference panics, crates/klearu-accel/src/memory/mod.rs:87-92) reads
// row 0 instead and, when err is set, is recorded there for the handle's
// status call.
__device__ __forceinline__ int checked_row(int id, int n, int* err) {
  if (static_cast<unsigned>(id) < static_cast<unsigned>(n)) return id;
  if (err) atomicOr(err, 1);
  return 0;
}

// p[0..n) = v.  A kernel rather than hipMemsetAsync, so that callers may
// capture it in a HIP graph.  (A template, so that each translation unit
// including this header keeps its own copy.)
template <int Unused = 0>
__global__ void fill_f32_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace kh
