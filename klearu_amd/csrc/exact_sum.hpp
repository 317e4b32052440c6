// exact_sum.hpp -- the reference's sequential f32 sums, computed by one block.
//
// Rust's `let mut s = s0; for v in terms { s += v; }` rounds after every add,
// so the result is one particular f32 that only the same order reproduces
// (e.g. RmsNorm's sum of squares, crates/klearu-llm/src/model/rms_norm.rs:48-51).
// A dependent chain of 4096 adds costs about 10 us on one lane.  The block here
// returns the same bits with most of the chain run in parallel:
//
//  1. The terms are cut into chunks of M.  A guess of the running sum at the
//     start of chunk c is s0 plus the chunk sums before it (f32, any order).
//     It is only a guess.
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
// misses about once in 600 chunks at n = 4096 (CPU model of this scheme).
//
// Start values are enumerated with an integer key that orders every f32 except
// -0.0 (which shares +0.0's key): a running sum equal to -0.0, or not finite,
// always takes the sequential path.
#pragma once

#include <utility>

#include "common.hpp"

namespace kh {

constexpr int kEsWin = 64;      // start values per chunk (the lanes of one wave)
constexpr int kEsMaxChunks = 64;

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

// Chunk c's window entry of lane l ends at e = E[c][l]: the lane of chunk c + 1
// that started from e, or -1 when e is outside that window, not finite, or
// -0.0.  Past the last chunk (c + 1 >= C) the path stays on its lane.
__device__ __forceinline__ int es_next(float e, int gk_next, int c, int C) {
  const int lane = threadIdx.x & 63;
  const uint32_t eb = __float_as_uint(e);
  const int q = es_key(e) - gk_next + kEsWin / 2;
  const bool ok = (eb & 0x7f800000u) != 0x7f800000u && eb != 0x80000000u &&
                  static_cast<uint32_t>(q) < static_cast<uint32_t>(kEsWin);
  return c + 1 >= C ? lane : (ok ? q : -1);
}

// P full chunks of M terms starting at chunk c0 (cnt <= P of them real; the
// others repeat the last one and are not stored), each from the start value
// `st[i]` of this lane, run as P interleaved chains: a dependent DPP add costs
// about 10 cycles, P independent ones about 5 per wave (measured), so the
// chains of a wave hide each other's latency.  Stores E and nx (es_next;
// gkv holds the guessed start key of chunk `lane`) of every real chunk.
template <int P, int M>
__device__ __forceinline__ void es_windows(const float* __restrict__ t, int c0, int cnt, int C,
                                           const float (&st)[P], int gkv, float* __restrict__ E,
                                           int* __restrict__ NX) {
  const int lane = threadIdx.x & 63;
  float s[P];
  int base[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    s[i] = st[i];
    base[i] = (c0 + min(i, cnt - 1)) * M + (lane & 15);
  }
  float tv[P];
#pragma unroll
  for (int i = 0; i < P; ++i) tv[i] = t[base[i]];
#pragma unroll
  for (int g = 0; g < M / 16; ++g) {
    // the next group's terms are requested before this group's adds
    float tn[P];
    const int gn = 16 * min(g + 1, M / 16 - 1);
#pragma unroll
    for (int i = 0; i < P; ++i) tn[i] = t[base[i] + gn];
#define KH_ES_STEP(K)                                          \
  _Pragma("unroll") for (int i = 0; i < P; ++i) es_add_bcast<K>(s[i], tv[i]);
    KH_ES_STEP(0) KH_ES_STEP(1) KH_ES_STEP(2) KH_ES_STEP(3)
    KH_ES_STEP(4) KH_ES_STEP(5) KH_ES_STEP(6) KH_ES_STEP(7)
    KH_ES_STEP(8) KH_ES_STEP(9) KH_ES_STEP(10) KH_ES_STEP(11)
    KH_ES_STEP(12) KH_ES_STEP(13) KH_ES_STEP(14) KH_ES_STEP(15)
#undef KH_ES_STEP
#pragma unroll
    for (int i = 0; i < P; ++i) tv[i] = tn[i];
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int c = c0 + i;
    if (i < cnt) {
      E[c * kEsWin + lane] = s[i];
      NX[c * kEsWin + lane] = es_next(s[i], __builtin_amdgcn_readlane(gkv, min(c + 1, kEsWin - 1)), c, C);
    }
  }
}

// Inclusive prefix sum of f32 over the lanes of a wave (any rounding: the
// result only feeds guesses).
__device__ __forceinline__ float es_wave_scan(float x) {
  x += dppf<kDppRowShr1>(x);
  x += dppf<kDppRowShr2>(x);
  x += dppf<kDppRowShr4>(x);
  x += dppf<kDppRowShr8>(x);
  x += dppf<kDppRowBcast15, 0xa>(x);
  x += dppf<kDppRowBcast31, 0xc>(x);
  return x;
}

template <int MAXC = kEsMaxChunks>
struct EsLds {
  float E[MAXC * kEsWin];  // E[c*64 + l] = f_c(start value of lane l)
  int nx[MAXC * kEsWin];   // lane of chunk c + 1 that started from E[c*64 + l], or -1
  float D[MAXC];           // chunk sums (guesses only)
  int gk[MAXC];            // key of the guessed start of chunk c
  float res;
};

// Sequential f32 sum s0 + t[0] + t[1] + ... + t[n-1] (left to right, rounding
// after each add) of terms in LDS, with chunks of M terms (M = 64 or 128,
// n <= 64 M).  Every thread of the block (NW waves, blockDim.x == 64 * NW)
// must call it.  Returns the sum in every thread.  Its barriers wait for LDS
// traffic only, so global loads a wave has in flight stay in flight.
template <int NW, int M>
__device__ __forceinline__ float exact_seq_sum(const float* __restrict__ t, int n, float s0,
                                              EsLds<>& es) {
  static_assert(M == 64 || M == 128, "chunk of 64 or 128 terms");
  constexpr int kMaxP = 16;
  constexpr int kLpc = M / 8;  // lanes per chunk in the chunk sums (8 terms each)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n <= 0) return s0;
  const int C = (n + M - 1) / M;  // chunks (the last may be partial)
  const int Cf = n / M;           // full chunks
  // 1. chunk sums (any order: guesses only).  A wave takes 512 terms at a
  // time, 8 per lane, and adds them over the M/8 lanes of each chunk.
  for (int r = wave; r * 512 < n; r += NW) {
    const int j0 = r * 512 + 8 * lane;
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a += j0 + e < n ? t[j0 + e] : 0.0f;
    a = group_sum<kLpc>(a);
    const int c = (r * 512) / M + lane / kLpc;
    if (lane % kLpc == 0 && c < C) es.D[c] = a;
  }
  lds_barrier();
  // 2. guesses (every wave, for itself): exclusive prefix of the chunk sums;
  // wave 0 also stores them for the composition
  const float dl = lane < C ? es.D[lane] : 0.0f;
  const float inc = es_wave_scan(dl);
  float ex = __shfl_up(inc, 1, 64);
  if (lane == 0) ex = 0.0f;
  const int gkv = es_key(s0 + ex);  // key of the guessed start of chunk `lane`
  if (wave == 0 && lane < C) es.gk[lane] = gkv;
  // 3. this wave's chunks from kEsWin start values each.  Waves that share a
  // SIMD with another wave of the block (round-robin placement: waves w and
  // w + 4) take half as many chunks as a wave alone on its SIMD.
  int tot = 0, before = 0, mine = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int wt = (NW <= 4 || NW >= 8) ? 1 : ((w + 4 < NW) || (w >= 4) ? 1 : 2);
    before += w < wave ? wt : 0;
    mine = w == wave ? wt : mine;
    tot += wt;
  }
  const int c0 = (C * before) / tot, c1 = (C * (before + mine)) / tot;
  {
    const int cf1 = min(c1, Cf);  // full chunks of this wave
    for (int cb = c0; cb < cf1; cb += kMaxP) {
      const int cnt = min(kMaxP, cf1 - cb);
      float st[kMaxP];
#pragma unroll
      for (int i = 0; i < kMaxP; ++i) {
        const int c = min(cb + i, cf1 - 1);
        st[i] = c == 0 ? s0 : es_from_key(__builtin_amdgcn_readlane(gkv, c) + lane - kEsWin / 2);
      }
      if (cnt > 8) {
        es_windows<kMaxP, M>(t, cb, cnt, C, st, gkv, es.E, es.nx);
      } else {
        float s8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) s8[i] = st[i];
        es_windows<8, M>(t, cb, cnt, C, s8, gkv, es.E, es.nx);
      }
    }
    if (Cf < C && c0 <= Cf && Cf < c1) {
      // the partial last chunk
      const float st = Cf == 0 ? s0 : es_from_key(__builtin_amdgcn_readlane(gkv, Cf) + lane - kEsWin / 2);
      const float e = es_run(t, Cf * M, n, st);
      es.E[Cf * kEsWin + lane] = e;
      es.nx[Cf * kEsWin + lane] = es_next(e, 0, Cf, C);
    }
  }
  lds_barrier();
  // 4. composition (wave 0): the path starts at chunk 0 (every lane of which
  // started from s0) and steps p <- nx[c] of lane p.  A miss anywhere on the
  // path shows as a negative p (collected by OR); the sum is then redone on
  // the slow path.
  if (wave == 0) {
    int nx[kEsMaxChunks];
#pragma unroll
    for (int c = 0; c + 1 < kEsMaxChunks; ++c) nx[c] = es.nx[c * kEsWin + lane];
    int p = 0, any = 0;
#pragma unroll
    for (int c = 0; c + 1 < kEsMaxChunks; ++c) {
      if (c + 1 < C) {
        p = __builtin_amdgcn_readlane(nx[c], p & (kEsWin - 1));
        any |= p;
      }
    }
    int s;
    if (any >= 0) {
      s = __float_as_int(es.E[(C - 1) * kEsWin + p]);
    } else {
      // slow path: chunk by chunk, lookups from LDS or sequential chunks
      s = __float_as_int(es.E[0]);
      for (int c = 1; c < C; ++c) {
        const uint32_t sb = static_cast<uint32_t>(s);
        const int idx = es_key(__int_as_float(s)) - es.gk[c] + kEsWin / 2;
        const bool ok = (sb & 0x7f800000u) != 0x7f800000u && sb != 0x80000000u &&
                        static_cast<uint32_t>(idx) < static_cast<uint32_t>(kEsWin);
        if (ok) {
          s = __float_as_int(es.E[c * kEsWin + idx]);
        } else {
          const float v = es_run(t, c * M, min(n, c * M + M), __int_as_float(s));
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
