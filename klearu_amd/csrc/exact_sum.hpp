// exact_sum.hpp -- the reference's sequential f32 sums, computed by one block.
//
// Rust's `let mut s = s0; for v in terms { s += v; }` rounds after every add,
// so the result is one particular f32 that only the same order reproduces
// (e.g. RmsNorm's sum of squares, crates/klearu-llm/src/model/rms_norm.rs:48-51).
// A dependent chain of 4096 adds costs about 10 us on one lane.  The block here
// returns the same bits with most of the chain run in parallel:
//
//  1. The terms are cut into chunks of kEsChunk.  A guess of the running sum at
//     the start of chunk c is formed from the chunk sums (f32, any order) with
//     the prefix in f64, rounded to f32.  It is only a guess.
//  2. Every chunk c >= 1 is run sequentially from kEsWin consecutive f32 start
//     values centred on its guess, one lane per start value; chunk 0 runs from
//     s0 itself.  Lane l of the wave owning chunk c ends with f_c(start_l), f_c
//     being the sequential pass over the chunk's terms.  The 16 terms of a group
//     sit in the 16 lanes of every row and each add reads its term through a DPP
//     row broadcast, so a step is one VALU instruction and no LDS traffic.
//  3. One wave composes: s = f_0(s0); for each further chunk, if s is one of its
//     start values, the lane that started there already holds f_c(s); otherwise
//     the chunk is run sequentially from s.
// The result is always the sequential sum; the guesses only decide how much of
// it ran in parallel.  For a monotone running sum (sums of squares) the window
// misses about once in 600 chunks at n = 4096.
//
// Start values are enumerated with an integer key that orders every f32 except
// -0.0 (which shares +0.0's key): a running sum equal to -0.0, or not finite,
// always takes the sequential path.
#pragma once

#include <utility>

#include "common.hpp"

namespace kh {

constexpr int kEsChunk = 128;  // terms per chunk
constexpr int kEsWin = 64;     // start values per chunk (the lanes of one wave)

// Order-preserving integer key of an f32 (consecutive floats -> consecutive keys).
__device__ __forceinline__ int es_key(float f) {
  const int i = __float_as_int(f);
  return i < 0 ? static_cast<int>(0x80000000u - static_cast<uint32_t>(i)) : i;
}
__device__ __forceinline__ float es_from_key(int k) {
  const int i = k < 0 ? static_cast<int>(0x80000000u - static_cast<uint32_t>(k)) : k;
  return __int_as_float(i);
}

// s + (lane K of this lane's row of 16) as one v_add_f32 with a DPP
// row_newbcast operand (the compiler emits the broadcast as a separate move).
template <int K>
__device__ __forceinline__ void es_add_bcast(float& s, float tv) {
  float r;
  asm("v_add_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "=v"(r)
      : "v"(tv), "v"(s), "i"(K));
  s = r;
}
template <int... K>
__device__ __forceinline__ void es_add16(float& s, float tv, std::integer_sequence<int, K...>) {
  (es_add_bcast<K>(s, tv), ...);
}

// Sequential pass over t[j0, j1) from s, in every lane of the wave (each lane
// gets the same value).  Full 16-term groups use the row broadcast; the tail
// reads LDS with a wave-uniform address.
__device__ __forceinline__ float es_run(const float* __restrict__ t, int j0, int j1, float s) {
  const int lane = threadIdx.x & 63;
  int j = j0;
  for (; j + 16 <= j1; j += 16) {
    const float tv = t[j + (lane & 15)];
    es_add16(s, tv, std::make_integer_sequence<int, 16>{});
  }
  for (; j < j1; ++j) s = __fadd_rn(s, t[j]);
  return s;
}

template <int MAXC>
struct EsLds {
  float E[MAXC][kEsWin];  // E[c][l] = f_c(start of lane l)
  float D[MAXC];          // chunk sums (guesses only)
  int gk[MAXC];           // key of the guessed start of chunk c
  float res;
};

// Sequential f32 sum s0 + t[0] + t[1] + ... + t[n-1] (left to right, rounding
// after each add) of terms in LDS.  Every thread of the block (NW waves,
// blockDim.x == 64 * NW) must call it; n <= kEsChunk * MAXC.  Returns the sum
// in every thread.  Contains barriers that wait for LDS traffic only, so
// global loads a wave has in flight stay in flight.
template <int NW, int MAXC>
__device__ __forceinline__ float exact_seq_sum(const float* __restrict__ t, int n, float s0,
                                              EsLds<MAXC>& es) {
  static_assert(NW >= 1 && MAXC <= 64, "one composing wave holds every chunk");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (n <= 0) return s0;
  const int C = (n + kEsChunk - 1) / kEsChunk;
  // 1. chunk sums in f32 (any order: guesses only)
  for (int c = wave; c < C; c += NW) {
    const int j = c * kEsChunk + lane;
    const float a = (j < n ? t[j] : 0.0f) + (j + 64 < n ? t[j + 64] : 0.0f);
    const float d = wave_sum(a);
    if (lane == 0) es.D[c] = d;
  }
  lds_barrier();
  if (wave == 0) {
    // exclusive prefix in f64 over lanes c < C, then the f32 guess
    const double d = lane < C ? static_cast<double>(es.D[lane]) : 0.0;
    double inc = d;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(inc, off, 64);
      if (lane >= off) inc += o;
    }
    double ex = __shfl_up(inc, 1, 64);
    if (lane == 0) ex = 0.0;
    if (lane < C) es.gk[lane] = es_key(static_cast<float>(static_cast<double>(s0) + ex));
  }
  lds_barrier();
  // 2. every chunk from kEsWin start values.  Waves that share a SIMD with
  // another wave of the block (round-robin placement: waves w and w + 4) take
  // half the chunks of a wave alone on its SIMD.
  {
    int wt[NW];
    int tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int shared = (w + 4 < NW) || (w >= 4) ? 1 : 2;
      wt[w] = (NW <= 4) ? 2 : shared;
      tot += wt[w];
    }
    int before = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) before += w < wave ? wt[w] : 0;
    const int c0 = (C * before) / tot, c1 = (C * (before + wt[wave])) / tot;
    for (int c = c0; c < c1; ++c) {
      const float st = c == 0 ? s0 : es_from_key(es.gk[c] + lane - kEsWin / 2);
      const int j0 = c * kEsChunk;
      es.E[c][lane] = es_run(t, j0, min(n, j0 + kEsChunk), st);
    }
  }
  lds_barrier();
  // 3. composition (wave 0)
  if (wave == 0) {
    float er[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) er[c] = es.E[c][lane];
    const int gkv = es.gk[min(lane, MAXC - 1)];
    int s = __builtin_amdgcn_readlane(__float_as_int(er[0]), 0);
#pragma unroll
    for (int c = 1; c < MAXC; ++c) {
      if (c < C) {
        const uint32_t sb = static_cast<uint32_t>(s);
        const int idx = es_key(__int_as_float(s)) - __builtin_amdgcn_readlane(gkv, c) + kEsWin / 2;
        const bool hit = (sb & 0x7f800000u) != 0x7f800000u && sb != 0x80000000u && idx >= 0 &&
                         idx < kEsWin;
        if (hit) {
          s = __builtin_amdgcn_readlane(__float_as_int(er[c]), idx);
        } else {
          const int j0 = c * kEsChunk;
          const float v = es_run(t, j0, min(n, j0 + kEsChunk), __int_as_float(s));
          s = __builtin_amdgcn_readfirstlane(__float_as_int(v));
        }
      }
    }
    if (lane == 0) es.res = __int_as_float(s);
  }
  lds_barrier();
  return es.res;
}

// RmsNorm's scale 1/sqrt(sum_sq/n + eps) from the sequential sum of squares,
// each operation correctly rounded as Rust rounds it (model/rms_norm.rs:52-53).
// HIP's f32 `/` and sqrtf are correctly rounded by default
// (-fhip-fp32-correctly-rounded-divide-sqrt); __fsqrt_rn is not: without
// OCML_BASIC_ROUNDED_OPERATIONS it is the approximate hardware square root.
__device__ __forceinline__ float rms_inv_exact(float sum_sq, int n, float eps) {
  const float rms = sqrtf(__fadd_rn(sum_sq / static_cast<float>(n), eps));
  return 1.0f / rms;
}

}  // namespace kh
