// topk_select.hpp -- the exact k-th key of a row of scores, for one block of NT
// threads that holds the row's keys in registers (select_top_k's stable
// descending sort, crates/klearu-dejavu/src/predictor/mlp_predictor.rs:128-135:
// the first k of the sort are the keys above the k-th key T plus the
// lowest-index keys equal to T).
//
// Thread t holds the keys of the contiguous index range [i0, i0 + cnt) with
// i0 = t * KPT, so a selection comes out in ascending index order from one
// exclusive scan.  Used by topk_kernel (predictor.hip) and by the FFN kernel
// that selects its own neurons (ffn.hip).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace kh {

constexpr int kTopkCand = 256;  // boundary bins up to this size are ranked directly
constexpr int kTopkDigit = 11;  // radix digit (2048 bins)

template <int NT>
struct TopkLds {
  unsigned hist[1 << kTopkDigit];
  uint64_t cand[kTopkCand];
  int wsum[NT / 64];
  uint32_t uwsum[NT / 64];
  uint32_t wmax[NT / 64], wmin[NT / 64];
  uint32_t s_prefix, s_mask, s_T;
  int s_kk, s_total, s_bincount, s_ncand, s_ties;
};

// The k-th key T of the row and `ties`, the number of keys equal to T that the
// first kk0 of the sort take.  mx / mn: the largest and smallest key of the row
// (every thread).  Before the call, sh.hist must be zero and sh.s_ncand 0,
// published by a barrier.
//   1. the radix passes start below the bits common to every key (scores
//      cluster, so a pass over shared high bits would fill one or two bins);
//   2. one pass over the next kTopkDigit bits: LDS histogram, block scan from
//      the top bin down -> the bin holding the k-th key;
//   3. if that bin holds at most kTopkCand keys, they are gathered and ranked
//      directly by (key desc, index asc); otherwise the passes continue.
// (Equal-width bins over [mn, mx] instead of radix digits spread sigmoid
// scores over more bins but cost an f32 conversion per key, and measured
// slower inside the FFN kernel.)
template <int NT, int KPT>
__device__ __forceinline__ void topk_threshold(const uint32_t (&key)[KPT], int cnt, int i0, int kk0,
                                               uint32_t mx, uint32_t mn, TopkLds<NT>& sh,
                                               uint32_t& T_out, int& ties_out) {
  const uint32_t diff = mx ^ mn;
  int hi = diff ? 31 - __clz(diff) : -1;
  uint32_t mask = hi < 0 ? 0xffffffffu : (hi >= 31 ? 0u : ~((2u << hi) - 1u));
  uint32_t prefix = mx & mask;
  int kk = kk0;
  uint32_t T = prefix;
  int ties = kk0;
  bool first = true;
  while (hi >= 0) {
    const int lo = max(0, hi - (kTopkDigit - 1));
    const int nbins = 2 << (hi - lo);
    const uint32_t binmask = (uint32_t)nbins - 1u;
    if (!first) {
      for (int i = threadIdx.x; i < nbins; i += NT) sh.hist[i] = 0;
      __syncthreads();
    }
    first = false;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      if (j < cnt && (key[j] & mask) == prefix) atomicAdd(&sh.hist[(key[j] >> lo) & binmask], 1u);
    __syncthreads();
    // Thread t owns bins [nbins-(t+1)*per, nbins-t*per), thread 0 the highest;
    // the exclusive scan in thread order counts the keys in higher bins.
    const int per = (nbins + NT - 1) / NT;
    const int top = nbins - (int)threadIdx.x * per;
    const int bot = max(top - per, 0);
    int local = 0;
    for (int j = bot; j < top; ++j) local += (int)sh.hist[j];
    const int above = block_excl_scan(local, sh.wsum, &sh.s_total);
    if (top > 0 && above < kk && kk <= above + local) {
      int cum = above, sel = bot;
      for (int j = top - 1; j >= bot; --j) {
        if (cum + (int)sh.hist[j] >= kk) {
          sel = j;
          break;
        }
        cum += (int)sh.hist[j];
      }
      sh.s_kk = kk - cum;
      sh.s_prefix = prefix | ((uint32_t)sel << lo);
      sh.s_mask = mask | (binmask << lo);
      sh.s_bincount = (int)sh.hist[sel];
    }
    __syncthreads();
    kk = sh.s_kk;
    prefix = sh.s_prefix;
    mask = sh.s_mask;
    hi = lo - 1;
    T = prefix;
    ties = kk;
    if (hi < 0) break;  // every bit resolved: the bin is one key value
    if (sh.s_bincount <= kTopkCand) {
      // Gather the bin's keys: one LDS atomic per wave reserves the wave's
      // slots (a wave scan of the per-thread counts places each key).
      using M = typename std::conditional<(KPT > 32), unsigned long long, uint32_t>::type;
      M cm = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        if (j < cnt) cm |= (M)((key[j] & mask) == prefix) << j;
      const int c = (int)__popcll((unsigned long long)cm);
      const int incl = wave_incl_scan(c);
      const int wtot = __builtin_amdgcn_readlane(incl, 63);
      if (wtot) {
        int base = 0;
        if ((threadIdx.x & 63) == 63) base = atomicAdd(&sh.s_ncand, wtot);
        int at = __builtin_amdgcn_readlane(base, 63) + incl - c;
#pragma unroll
        for (int j = 0; j < KPT; ++j)
          if ((cm >> j) & 1u) sh.cand[at++] = ((uint64_t)key[j] << 32) | (uint32_t)(0xffffffffu - (uint32_t)(i0 + j));
      }
      __syncthreads();
      const int m = sh.s_ncand;
      // Four threads per candidate: thread t ranks candidate t/4 against a
      // quarter of the list; the quarters are added across the lane quad.
      // NT/4 candidates at once, so lists longer than that take more rounds.
      for (int base = 0; base < m; base += NT / 4) {
        const int ci = base + ((int)threadIdx.x >> 2), part = (int)threadIdx.x & 3;
        int rank = 0, gt = 0;
        uint32_t mk = 0u;
        if (ci < m) {
          const uint64_t me = sh.cand[ci];
          mk = (uint32_t)(me >> 32);
          const int q = (m + 3) >> 2;
          const int j1 = min(part * q + q, m);
          for (int j = part * q; j < j1; ++j) {
            const uint64_t o = sh.cand[j];
            rank += o > me;
            gt += (uint32_t)(o >> 32) > mk;
          }
        }
        rank += dpp<kDppQuadSwap1>(rank);
        rank += dpp<kDppQuadSwap2>(rank);
        gt += dpp<kDppQuadSwap1>(gt);
        gt += dpp<kDppQuadSwap2>(gt);
        if (ci < m && part == 0 && rank == kk - 1) {
          sh.s_T = mk;
          sh.s_ties = kk - gt;
        }
      }
      __syncthreads();
      T = sh.s_T;
      ties = sh.s_ties;
      break;
    }
  }
  T_out = T;
  ties_out = ties;
}

// Selection masks of this thread's keys (bit j: key j is among the first kk0
// of the sort) and the rank of its first selected key: the keys above T, then
// keys equal to T in index order until `ties` of them are taken.  One block
// scan of packed counts (keys > T in the low 16 bits, keys == T in the high 16
// bits; rows of fewer than 65536 keys).
template <int NT, int KPT>
__device__ __forceinline__ auto topk_select_mask(const uint32_t (&key)[KPT], int cnt, uint32_t T, int ties,
                                                 TopkLds<NT>& sh, int& pos) {
  using M = typename std::conditional<(KPT > 32), unsigned long long, uint32_t>::type;
  M gtm = 0, eqm = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j)
    if (j < cnt) {
      gtm |= (M)(key[j] > T) << j;
      eqm |= (M)(key[j] == T) << j;
    }
  const int ceq = (int)__popcll((unsigned long long)eqm);
  const uint32_t ex =
      block_excl_scan_u32((uint32_t)__popcll((unsigned long long)gtm) | ((uint32_t)ceq << 16), sh.uwsum);
  const int gt_before = (int)(ex & 0xffffu), eq_before = (int)(ex >> 16);
  const int take = max(0, min(ceq, ties - eq_before));
  M em = eqm;
  for (int t = ceq; t > take; --t) em &= ~((M)1 << (63 - __clzll((unsigned long long)em)));  // drop the highest
  pos = gt_before + min(eq_before, ties);
  return (M)(gtm | em);
}

}  // namespace kh
