// exact_sum.hpp -- the reference's sequential f32 sums, computed by one block.
//
// Rust's `let mut s = s0; for v in terms { s += v; }` rounds after every add,
// so the result is one particular f32 that only the same order reproduces
// (e.g. RmsNorm's sum of squares, crates/klearu-llm/src/model/rms_norm.rs:48-51).
// A dependent chain of 4096 adds costs about 7.5 us on one lane (4.3 cycles a
// step).  The block here returns the same bits with most of the chain run in
// parallel:
//
//  1. The terms are cut into CH chunks of M.  A guess of the running sum at the
//     start of chunk c is s0 plus the chunk sums before it (f32, any order).
//     It is only a guess.
//  2. Every chunk c >= 1 is run sequentially from W consecutive f32 start
//     values ("slots") centred on its guess; chunk 0 runs from s0 itself.
//     Lane l of every wave works on chunk l % CH; its slots are spread over
//     the waves, the 64 / CH lanes of a chunk and P chains per lane, and all
//     of a lane's chains add the same term, read once from LDS.  f_c(slot k)
//     is stored, and so is the slot of chunk c + 1 it equals (or -1).
//  3. The path from chunk 0 follows those slot links: each wave follows every
//     slot through a segment of chunks at once (lane gathers), then one wave
//     chains the segments.  If the path leaves a window anywhere, that chunk
//     is run sequentially from the exact running sum (the slow path).
// The result is always the sequential sum; the guesses only decide how much of
// it ran in parallel.  For a monotone running sum (sums of squares) the window
// misses about once in 600 chunks at n = 4096 (CPU model of this scheme).
//
// Slots are enumerated with an integer key that orders every f32 except -0.0
// (which shares +0.0's key): a running sum equal to -0.0, or not finite,
// always takes the slow path.  Terms past n are stored as -0.0, which leaves
// every sum unchanged (x + -0.0 == x for every x).
#pragma once

#include "common.hpp"

namespace kh {

constexpr int kEsW = 64;  // slots per chunk (window width, at most 64)

// Order-preserving integer key of an f32 (consecutive floats -> consecutive keys).
__device__ __forceinline__ int es_key(float f) {
  const int i = __float_as_int(f);
  return i < 0 ? static_cast<int>(0x80000000u - static_cast<uint32_t>(i)) : i;
}
__device__ __forceinline__ float es_from_key(int k) {
  const int i = k < 0 ? static_cast<int>(0x80000000u - static_cast<uint32_t>(k)) : k;
  return __int_as_float(i);
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

// LDS of one exact sum: CH chunks of M terms (M a multiple of 4).
template <int CH, int M>
struct EsLds {
  static constexpr int kS = M + 4;   // padded row: 16-byte aligned, conflict-light
  static constexpr int kNS = CH + 4;
  __align__(16) float TP[CH * kS];  // TP[c*kS + j] = t[c*M + j] (the caller fills it; es_slot)
  float E[CH * kEsW];     // E[c*64 + k] = f_c(slot k)
  int NXT[kEsW * kNS];    // NXT[k*kNS + c]: slot of chunk c + 1 equal to E[c*64 + k], or -1
  int SM[16 * kEsW];      // SM[g*64 + k]: slot at the end of segment g from slot k, or -1
  int gk[CH];             // key of the guessed start of chunk c
  float res;
};

// Index in EsLds::TP of term i.
template <int CH, int M>
__device__ __forceinline__ int es_slot(int i) {
  return (i / M) * EsLds<CH, M>::kS + (i % M);
}

// Sequential f32 sum s0 + t[0] + t[1] + ... + t[n-1] (left to right, rounding
// after each add) of the terms the caller stored in es.TP (es_slot; -0.0 for
// n <= i < CH*M), n <= CH*M.  Every thread of the block (NW waves, blockDim.x ==
// 64 * NW) must call it after a barrier that publishes TP.  Returns the sum in
// every thread.  Its barriers wait for LDS traffic only, so global loads a
// wave has in flight stay in flight.
template <int NW, int CH, int M>
__device__ __forceinline__ float exact_seq_sum(int n, float s0, EsLds<CH, M>& es) {
  using L_ = EsLds<CH, M>;
  constexpr int G = 64 / CH;          // lanes per chunk
  constexpr int P = kEsW / (G * NW);  // chains per lane
  constexpr int W = P * G * NW;       // slots per chunk
  constexpr int S = L_::kS, NS = L_::kNS;
  constexpr int SEG = (CH + NW - 1) / NW;  // chunks per segment (one segment per wave)
  static_assert(64 % CH == 0 && P >= 1 && M % (4 * G) == 0 && NW <= 16, "exact-sum layout");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n <= 0) return s0;
  const int C = (n + M - 1) / M;  // chunks holding terms
  // 1. chunk sums (each of a chunk's G lanes adds M/G terms) and guesses
  if (wave == 0) {
    constexpr int MG = M / G;
    const float4* tp = reinterpret_cast<const float4*>(es.TP + min(lane % CH, C - 1) * S + (lane / CH) * MG);
    float4 v[MG / 4];
#pragma unroll
    for (int j = 0; j < MG / 4; ++j) v[j] = tp[j];
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int j = 0; j < MG / 4; ++j) {
      a0 += v[j].x;
      a1 += v[j].y;
      a2 += v[j].z;
      a3 += v[j].w;
    }
    float d = (a0 + a1) + (a2 + a3);
#pragma unroll
    for (int m = CH; m < 64; m <<= 1) d += __shfl_xor(d, m);
    d = lane < C ? d : 0.0f;
    const float inc = es_wave_scan(d);
    float ex = __shfl_up(inc, 1, 64);
    if (lane == 0) ex = 0.0f;
    if (lane < CH) es.gk[lane] = es_key(s0 + ex);
  }
  lds_barrier();
  // 2. windows
  {
    const int c = min(lane % CH, C - 1), h = lane / CH;
    const int gkc = es.gk[c];
    const int gkn = es.gk[min(c + 1, C - 1)];
    const int k0 = (wave * G + h) * P;
    float s[P];
#pragma unroll
    for (int i = 0; i < P; ++i) s[i] = c == 0 ? s0 : es_from_key(gkc + k0 + i - W / 2);
    const float4* tp = reinterpret_cast<const float4*>(es.TP + c * S);
    constexpr int B = 8;  // float4 of terms read ahead
    float4 tv[B];
#pragma unroll
    for (int j = 0; j < B; ++j) tv[j] = tp[min(j, M / 4 - 1)];
    for (int j0 = 0; j0 < M / 4; j0 += B) {
      float4 tn[B];
#pragma unroll
      for (int j = 0; j < B; ++j) tn[j] = tp[min(j0 + B + j, M / 4 - 1)];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        if (j0 + j < M / 4) {
#pragma unroll
          for (int i = 0; i < P; ++i) s[i] = __fadd_rn(s[i], tv[j].x);
#pragma unroll
          for (int i = 0; i < P; ++i) s[i] = __fadd_rn(s[i], tv[j].y);
#pragma unroll
          for (int i = 0; i < P; ++i) s[i] = __fadd_rn(s[i], tv[j].z);
#pragma unroll
          for (int i = 0; i < P; ++i) s[i] = __fadd_rn(s[i], tv[j].w);
        }
      }
#pragma unroll
      for (int j = 0; j < B; ++j) tv[j] = tn[j];
    }
    if ((lane % CH) < C) {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int k = k0 + i;
        const uint32_t eb = __float_as_uint(s[i]);
        const int q = es_key(s[i]) - gkn + W / 2;
        const bool ok = (eb & 0x7f800000u) != 0x7f800000u && eb != 0x80000000u &&
                        static_cast<uint32_t>(q) < static_cast<uint32_t>(W);
        es.E[c * kEsW + k] = s[i];
        es.NXT[k * NS + c] = c + 1 >= C ? k : (ok ? q : -1);
      }
    }
  }
  lds_barrier();
  // 3a. segment g (wave g) covers the links out of chunks g*SEG .. g*SEG+SEG-1:
  // every slot is followed through it at once
  const int nseg = (C - 1 + SEG - 1) / SEG;
  if (wave < nseg) {
    int nx[SEG];
#pragma unroll
    for (int i = 0; i < SEG; ++i) nx[i] = lane < W ? es.NXT[lane * NS + min(wave * SEG + i, CH - 1)] : -1;
    int cur = lane < W ? lane : -1;
    int bad = cur;
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      if (wave * SEG + i + 1 < C) {
        cur = __builtin_amdgcn_ds_bpermute(cur << 2, nx[i]);
        bad |= cur;
      }
    }
    es.SM[wave * kEsW + lane] = bad < 0 ? -1 : cur;
  }
  lds_barrier();
  // 3b. one wave chains the segments from slot 0 of chunk 0 (all of chunk
  // 0's slots started from s0)
  if (wave == 0) {
    int sm[NW];
#pragma unroll
    for (int g = 0; g < NW; ++g) sm[g] = g < nseg ? es.SM[g * kEsW + lane] : lane;
    int p = 0, bad = 0;
#pragma unroll
    for (int g = 0; g < NW; ++g) {
      p = __builtin_amdgcn_readlane(sm[g], p);
      bad |= p;
    }
    float r;
    if (bad >= 0) {
      r = es.E[(C - 1) * kEsW + p];
    } else {
      // slow path: chunk by chunk, a window lookup or a sequential run
      r = es.E[0];
      for (int c = 1; c < C; ++c) {
        const uint32_t sb = __float_as_uint(r);
        const int idx = es_key(r) - es.gk[c] + W / 2;
        const bool ok = (sb & 0x7f800000u) != 0x7f800000u && sb != 0x80000000u &&
                        static_cast<uint32_t>(idx) < static_cast<uint32_t>(W);
        if (ok) {
          r = es.E[c * kEsW + idx];
        } else {
          const float* tp = es.TP + c * S;
          for (int j = 0; j < M; ++j) r = __fadd_rn(r, tp[j]);
        }
      }
    }
    if (lane == 0) es.res = r;
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
