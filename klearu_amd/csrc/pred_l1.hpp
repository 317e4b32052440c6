// pred_l1.hpp -- layer 1 of the Deja Vu predictor for rows of at most 4096
// inputs (crates/klearu-dejavu/src/predictor/mlp_predictor.rs:102-113), as
// a block body that kernels of predictor.hip and attention.hip launch, and
// layer 2's per-lane chain (mlp_predictor.rs:114-124) for the same files.
//
// Each hidden unit is a sequential f32 sum that starts at -0.0 and adds the
// rounded product w*x term by term (Rust `.map(|(w, x)| w * x).sum()`), with
// no FMA contraction; one lane owns one sum ("chain").  The weights are stored
// blocked-transposed, [in/8][hid][8], so that 64 lanes read 64 adjacent
// 16-byte blocks.
#pragma once

#include "common.hpp"
#include "exact_sum.hpp"

namespace kh {

// ---------------------------------------------------------------- predictor
// Weight element loaders: BF16 bits (predictors whose weights are BF16 values,
// stored losslessly in half the bytes) or f32.
template <typename W> struct Blk8;
template <> struct Blk8<uint16_t> {
  using V = uint4;  // 8 bf16
  static __device__ __forceinline__ void widen(const V& v, float o[8]) {
    o[0] = bf16_lo(v.x); o[1] = bf16_hi(v.x); o[2] = bf16_lo(v.y); o[3] = bf16_hi(v.y);
    o[4] = bf16_lo(v.z); o[5] = bf16_hi(v.z); o[6] = bf16_lo(v.w); o[7] = bf16_hi(v.w);
  }
  static __device__ __forceinline__ V zero() { return make_uint4(0, 0, 0, 0); }
};
template <> struct Blk8<float> {
  struct V { float4 a, b; };
  static __device__ __forceinline__ void widen(const V& v, float o[8]) {
    o[0] = v.a.x; o[1] = v.a.y; o[2] = v.a.z; o[3] = v.a.w;
    o[4] = v.b.x; o[5] = v.b.y; o[6] = v.b.z; o[7] = v.b.w;
  }
  static __device__ __forceinline__ V zero() { return V{make_float4(0, 0, 0, 0), make_float4(0, 0, 0, 0)}; }
};

constexpr int kL1Chains = 8;
constexpr int kL1Stage = 128;     // steps per stage
constexpr int kL1Prod = 4;        // producer waves
constexpr int kL1Threads = 64 * (1 + kL1Prod);
constexpr int kL1Q = (kL1Stage / 8) * kL1Chains / 64;  // weight loads per producer lane per stage
static_assert(kL1Q * 64 == (kL1Stage / 8) * kL1Chains, "stage tiling");

// Layer 1 for n_in <= kL1LdsIn: the block's products w*x for every step are
// formed into LDS first (kL1Chains * n_in floats; all weight loads of the
// block are in flight at once), then the consumer wave runs its chains over
// them with no further barrier, reading 32 steps ahead of the adds.  Wave 0
// is the consumer, kL1Prod waves the producers; kL1Help more waves only
// stage x and share the RmsNorm sum (two waves per SIMD run its windows).
constexpr int kL1LdsIn = 4096;
constexpr int kL1Help = 3;  // waves that only stage x and share the RmsNorm sum
constexpr int kL1LdsThreads = 64 * (1 + kL1Prod + kL1Help);
constexpr int kL1LdsBytes = (kL1Chains + 1) * kL1LdsIn * 4;  // products + x

// With norm_w set, x is the un-normalised hidden row and the kernel applies
// RmsNorm first (model/rms_norm.rs:43-64): the reference's sequential sum of
// squares (exact_seq_sum over 32 chunks of 128 terms, run by every wave while
// the weight loads are in flight), its scale, then (x * inv) * norm_w.  Block 0
// stores the scale in inv_out[b] for the kernels that consume the same
// normalised row later, and, with xn_out set, the normalised row itself at
// xn_out[b][n_in].  The norm requires n_in % 4 == 0 (host-checked).
constexpr int kL1EsChunks = 32;
constexpr int kL1EsM = kL1LdsIn / kL1EsChunks;  // terms per chunk of the exact sum
using L1Es = EsLds<kL1EsChunks, kL1EsM>;
static_assert(sizeof(L1Es) <= sizeof(float4) * (kL1LdsIn / 4) * kL1Chains,
              "the exact-sum scratch fits in the products region");

// The work of one block of pred_l1_lds_kernel: hidden units [bx*kL1Chains, ...)
// of row b, with the block's LDS at lds4 (kL1LdsBytes).  Every thread of a
// kL1LdsThreads-thread block calls it.
template <typename W>
__device__ __forceinline__ void pred_l1_lds_body(
    const int bx, const int b, const W* __restrict__ Wb, const float* __restrict__ bias,
    const float* __restrict__ x, int n_in, int hid, float* __restrict__ h,
    const float* __restrict__ norm_w, float* __restrict__ inv_out, float eps, float4* lds4,
    float* __restrict__ xn_out = nullptr) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  constexpr int SPP = kL1LdsIn / kL1Stage / kL1Prod;  // stages per producer
  float4(*P)[kL1Chains] = reinterpret_cast<float4(*)[kL1Chains]>(lds4);  // [n_in/4][chain]
  float* xs = reinterpret_cast<float*>(lds4 + (kL1LdsIn / 4) * kL1Chains);
  // until the norm is known the products region holds the exact-sum scratch
  auto& es = *reinterpret_cast<L1Es*>(lds4);
  const int c0 = bx * kL1Chains;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nblk = (n_in + 7) >> 3;
  // Waves are placed on the CU's four SIMDs in turn (wave w on SIMD w % 4), so
  // the producers are waves 1, 2, 3 and 5 and the helpers 4, 6 and 7: the
  // consumer (wave 0) shares its SIMD only with a helper, which is idle while
  // the chain runs.
  static_assert(kL1Prod == 4 && kL1Help == 3, "wave roles");
  const int p = wave <= 3 ? wave - 1 : (wave == 5 ? 3 : -1);
  const float* xr = x + (size_t)b * n_in;
  const int n4 = n_in >> 2;
  // Every wave first requests its share of x (and of the norm weights), then
  // the producers request every weight of the block: the small x loads sit
  // ahead of the weight stream in the CU's queue, so the norm can start after
  // one round trip while the weights are still arriving.
  constexpr int kXs = (kL1LdsIn / 4 + kL1LdsThreads - 1) / kL1LdsThreads;  // float4 of x per thread
  const bool vec = (n_in & 3) == 0;
  float4 xv[kXs], wn[kXs];
  const float bv = wave == 0 ? bias[min(c0 + (lane & (kL1Chains - 1)), hid - 1)] : 0.0f;
  if (vec) {
#pragma unroll
    for (int q = 0; q < kXs; ++q)
      xv[q] = reinterpret_cast<const float4*>(xr)[min((int)threadIdx.x + q * kL1LdsThreads, n4 - 1)];
    if (norm_w) {
#pragma unroll
      for (int q = 0; q < kXs; ++q)
        wn[q] = reinterpret_cast<const float4*>(norm_w)[min((int)threadIdx.x + q * kL1LdsThreads, n4 - 1)];
    }
  }
  V pre[SPP][kL1Q];
  const bool prod = p >= 0;
  if (prod) {
    const V* __restrict__ wv = reinterpret_cast<const V*>(Wb);
#pragma unroll
    for (int i = 0; i < SPP; ++i)
#pragma unroll
      for (int q = 0; q < kL1Q; ++q) {
        const int st = p + kL1Prod * i;
        const int pr = lane + 64 * q;
        const int jb = min(st * (kL1Stage / 8) + pr / kL1Chains, nblk - 1);
        const int ch = min(c0 + pr % kL1Chains, hid - 1);
        pre[i][q] = wv[(size_t)jb * hid + ch];
      }
  }
  if (vec) {
    if (norm_w) {
      // squares as Rust forms them (v * v, rounded) for the sequential sum,
      // -0.0 past the row (four terms never straddle a chunk of 128)
#pragma unroll
      for (int q = 0; q < kXs; ++q) {
        const int i4 = threadIdx.x + q * kL1LdsThreads;
        if (i4 < kL1LdsIn / 4)
          *reinterpret_cast<float4*>(&es.TP[es_slot<kL1EsChunks, kL1EsM>(4 * i4)]) =
              i4 < n4 ? make_float4(__fmul_rn(xv[q].x, xv[q].x), __fmul_rn(xv[q].y, xv[q].y),
                                    __fmul_rn(xv[q].z, xv[q].z), __fmul_rn(xv[q].w, xv[q].w))
                      : make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
      }
    } else {
#pragma unroll
      for (int q = 0; q < kXs; ++q)  // clamped, unconditional (see stage_f4)
        reinterpret_cast<float4*>(xs)[min((int)threadIdx.x + q * kL1LdsThreads, n4 - 1)] = xv[q];
    }
  } else {
    for (int j = threadIdx.x; j < n_in; j += kL1LdsThreads) xs[j] = xr[j];
  }
  lds_barrier();
  if (norm_w) {
    // sum_sq over the row in the reference's order (rms_norm.rs:48-51)
    const float ss = exact_seq_sum<kL1LdsThreads / 64, kL1EsChunks, kL1EsM>(n_in, 0.0f, es);
    const float inv = rms_inv_exact(ss, n_in, eps);
#pragma unroll
    for (int q = 0; q < kXs; ++q) {
      float4 v = xv[q];
      v.x = __fmul_rn(__fmul_rn(v.x, inv), wn[q].x);
      v.y = __fmul_rn(__fmul_rn(v.y, inv), wn[q].y);
      v.z = __fmul_rn(__fmul_rn(v.z, inv), wn[q].z);
      v.w = __fmul_rn(__fmul_rn(v.w, inv), wn[q].w);
      reinterpret_cast<float4*>(xs)[min((int)threadIdx.x + q * kL1LdsThreads, n4 - 1)] = v;  // clamped
      if (xn_out && bx == 0)
        reinterpret_cast<float4*>(xn_out + (size_t)b * n_in)[min((int)threadIdx.x + q * kL1LdsThreads, n4 - 1)] = v;
    }
    if (bx == 0 && threadIdx.x == 0) inv_out[b] = inv;
    lds_barrier();
  }
  // products of stage p + kL1Prod*i; loads arrive in issue order, so each
  // stage waits only for its own weights
  auto make = [&](int i) {
    const int st = p + kL1Prod * i;
#pragma unroll
    for (int q = 0; q < kL1Q; ++q) {
      const int pr = lane + 64 * q;
      const int blk = pr / kL1Chains, ch = pr % kL1Chains;
      const int j0 = (st * (kL1Stage / 8) + blk) * 8;
      float w[8];
      B8::widen(pre[i][q], w);
      // j0 + 7 < kL1LdsIn for every stage: two aligned float4 reads of x
      const float4 xa = reinterpret_cast<const float4*>(xs)[j0 / 4];
      const float4 xb = reinterpret_cast<const float4*>(xs)[j0 / 4 + 1];
      P[j0 / 4][ch] = make_float4(__fmul_rn(w[0], xa.x), __fmul_rn(w[1], xa.y),
                                  __fmul_rn(w[2], xa.z), __fmul_rn(w[3], xa.w));
      P[j0 / 4 + 1][ch] = make_float4(__fmul_rn(w[4], xb.x), __fmul_rn(w[5], xb.y),
                                      __fmul_rn(w[6], xb.z), __fmul_rn(w[7], xb.w));
    }
  };
  // Consumer chain over steps [j0, j1) (j0 a multiple of 4): a window of kWin
  // quads is in flight; every kRefill quads are added, then their registers
  // are refilled with the quads kWin ahead, so the only VALU work per step is
  // the dependent add (LDS addresses are immediate offsets from one base
  // pointer).  Refilling in batches keeps the waits for the LDS counter to one
  // per batch: a read and a wait after every quad cost about 2 cycles per add.
  // Window reads past j1 are never added (they stay inside the block's LDS).
  constexpr int kWin = 32;    // quads in flight (128 steps)
  constexpr int kRefill = 8;  // quads added between refills
  constexpr int kSup = 64;    // quads per unrolled loop body (256 steps)
  static_assert(kSup % kWin == 0 && kWin % kRefill == 0, "window layout");
  static_assert((kL1LdsIn / 4 + kWin) * kL1Chains <= (kL1LdsBytes / 16), "window stays in LDS");
  const int ln = lane < kL1Chains ? lane : kL1Chains - 1;
  float s = -0.0f;
  auto run = [&](int j0, int j1) {
    const float4* bp = &P[j0 >> 2][ln];
    float4 r[kWin];
#pragma unroll
    for (int q = 0; q < kWin; ++q) r[q] = bp[q * kL1Chains];
    const int nsup = (j1 - j0) / (4 * kSup);
    for (int c = 0; c < nsup; ++c) {
#pragma unroll
      for (int q = 0; q < kSup; q += kRefill) {
#pragma unroll
        for (int u = 0; u < kRefill; ++u) {
          s = __fadd_rn(s, r[(q + u) % kWin].x);
          s = __fadd_rn(s, r[(q + u) % kWin].y);
          s = __fadd_rn(s, r[(q + u) % kWin].z);
          s = __fadd_rn(s, r[(q + u) % kWin].w);
        }
#pragma unroll
        for (int u = 0; u < kRefill; ++u) r[(q + u) % kWin] = bp[(q + u + kWin) * kL1Chains];
        // keep the refills here: the scheduler would otherwise sink them to their uses
        __builtin_amdgcn_sched_barrier(0);
      }
      bp += kSup * kL1Chains;
    }
    const float* Pf = reinterpret_cast<const float*>(lds4);
    for (int j = j0 + nsup * 4 * kSup; j < j1; ++j)
      s = __fadd_rn(s, Pf[((j >> 2) * kL1Chains + ln) * 4 + (j & 3)]);
  };
  // The first round of stages (one per producer) is published first, so the
  // chain starts while the producers form the rest.
  constexpr int kSeg = kL1Prod * kL1Stage;
  if (prod) make(0);
  lds_barrier();
  if (prod) {
#pragma unroll
    for (int i = 1; i < SPP; ++i) make(i);
  } else if (wave == 0) {
    run(0, min(n_in, kSeg));
  }
  lds_barrier();
  if (wave > 0) return;
  if (n_in > kSeg) run(kSeg, n_in);
  const int chain = c0 + lane;
  if (lane < kL1Chains && chain < hid) h[(size_t)b * hid + chain] = fmaxf(__fadd_rn(s, bv), 0.0f);
}

// ---------------------------------------------------------------- layer 2
// One output per lane: sigmoid(b + w . h) with the dot product a sequential
// f32 sum in input order (mlp_predictor.rs:114-124).  Layer 2's weights are
// stored blocked-transposed, [ceil(hid/8)][out][8], so the 64 lanes of a wave
// read 64 adjacent 16-byte blocks.  l2_load requests lane o's whole row (the
// caller stages h meanwhile); l2_chain runs the sum over h in LDS (n_hid
// floats plus 4 * kL2Hw of padding, 16-byte aligned).
constexpr int kMaxL2Hid = 256;
constexpr int kAttnSelHid = 128;  // head predictors selected inside the Q projection
constexpr int kL2Hw = 4;  // float4 of the hidden vector read ahead (16 steps)

// MAXH: the largest n_hid the call supports (registers for its row).
template <typename W, int MAXH = kMaxL2Hid>
__device__ __forceinline__ void l2_load(const W* __restrict__ Wb, int n_hid, int n_out, int oc,
                                        typename Blk8<W>::V (&w)[MAXH / 8]) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  const int nblk = (n_hid + 7) >> 3;
  const V* __restrict__ wv = reinterpret_cast<const V*>(Wb);
#pragma unroll
  for (int jb = 0; jb < MAXH / 8; ++jb)
    w[jb] = jb < nblk ? wv[(size_t)jb * n_out + oc] : B8::zero();
}

template <typename W, int MAXH = kMaxL2Hid>
__device__ __forceinline__ float l2_chain(const typename Blk8<W>::V (&w)[MAXH / 8], int n_hid,
                                          const float* hs) {
  using B8 = Blk8<W>;
  const int nblk = (n_hid + 7) >> 3;
  float s = -0.0f;
  if ((n_hid & 7) == 0) {
    // Whole 8-step blocks: no per-step test.  The hidden values come from LDS
    // through a window of kL2Hw float4 read ahead of their use (pinned, or the
    // scheduler sinks each read to its use and the chain waits on LDS).
    const float4* h4 = reinterpret_cast<const float4*>(hs);
    float4 hw[kL2Hw];
#pragma unroll
    for (int q = 0; q < kL2Hw; ++q) hw[q] = h4[q];
#pragma unroll
    for (int jb = 0; jb < MAXH / 8; ++jb) {
      if (jb < nblk) {
        float wf[8];
        B8::widen(w[jb], wf);
        const float4 a = hw[(2 * jb) % kL2Hw], c = hw[(2 * jb + 1) % kL2Hw];
        s = __fadd_rn(s, __fmul_rn(wf[0], a.x));
        s = __fadd_rn(s, __fmul_rn(wf[1], a.y));
        s = __fadd_rn(s, __fmul_rn(wf[2], a.z));
        s = __fadd_rn(s, __fmul_rn(wf[3], a.w));
        s = __fadd_rn(s, __fmul_rn(wf[4], c.x));
        s = __fadd_rn(s, __fmul_rn(wf[5], c.y));
        s = __fadd_rn(s, __fmul_rn(wf[6], c.z));
        s = __fadd_rn(s, __fmul_rn(wf[7], c.w));
        hw[(2 * jb) % kL2Hw] = h4[2 * jb + kL2Hw];
        hw[(2 * jb + 1) % kL2Hw] = h4[2 * jb + 1 + kL2Hw];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
#pragma unroll
    for (int jb = 0; jb < MAXH / 8; ++jb) {
      if (jb < nblk) {
        float wf[8];
        B8::widen(w[jb], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (jb * 8 + e < n_hid) s = __fadd_rn(s, __fmul_rn(wf[e], hs[jb * 8 + e]));
      }
    }
  }
  return s;
}

// Rank of lane o's key among the n_out <= 64 keys of its wave (key desc,
// index asc: select_top_k's stable descending sort, mlp_predictor.rs:128-131).
__device__ __forceinline__ int l2_wave_rank(uint32_t key, int o, int n_out) {
  int rank = 0;
  for (int j = 0; j < n_out; ++j) {
    const uint32_t kj = __builtin_amdgcn_readlane(key, j);
    rank += (kj > key || (kj == key && j < o)) ? 1 : 0;
  }
  return rank;
}

}  // namespace kh
