// predictor.hip -- Deja Vu sparsity predictor and top-k selection (gfx950).
//
// Replaces SparsityPredictor::predict / select_top_k
// (crates/klearu-dejavu/src/predictor/mlp_predictor.rs:102-132) as called by
// PredictorStore::predict_neurons / predict_heads
// (crates/klearu-llm/src/sparse/predictor_store.rs:31-45).
//
// Selections must be bit-exact, so both predictor layers reproduce the
// reference's arithmetic exactly: each output is a sequential f32 sum that
// starts at -0.0 and adds the rounded product w*x term by term (Rust
// `.map(|(w, x)| w * x).sum()`), with no FMA contraction.  One lane owns one
// sum ("chain"); the weights are stored blocked-transposed, [in/8][out][8] f32,
// so that at every step the 64 lanes of a wave read 64 adjacent 32-byte blocks
// and the shared input value is a wave-uniform (scalar) load.
//
// Top-k is a radix select over order-preserving 32-bit keys of the scores
// (passes of up to 11 bits with LDS histograms) that finds the exact k-th key T;
// the selected set is {key > T} plus the lowest-index entries with key == T,
// which is exactly what the reference's stable descending sort keeps.
#include <cstring>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "exact_sum.hpp"
#include "pred_l1.hpp"
#include "topk_select.hpp"

namespace kh {

// Layer 1 (long chains).  A block owns kL1Chains consecutive hidden units.
// Its kL1Prod producer waves request every weight the block needs -- the
// blocked layout [ceil(n_in/8)][hid][8] gives 16-byte loads of one 8-step
// block of one chain -- in the first few hundred cycles, each holding SPP
// stages of kL1Stage steps in registers, so HBM latency is paid once.  Stage
// by stage, the producer that owns the next stage forms the rounded products
// w*x and writes them to a two-stage LDS ring laid out [stage][step/4][chain][4],
// while the consumer wave (lanes < kL1Chains, one chain each) adds the current
// stage in step order with one ds_read_b128 per four steps.  The time is then
// set by the chain itself: one dependent add per step, about 6 cycles on
// gfx950.  Output h[b][i] = max(sum + b1[i], 0).
constexpr int kMaxL1In = 8192;    // x row staged in LDS (16 stages per producer)

template <typename W, int SPP>
__global__ __launch_bounds__(kL1Threads) void pred_l1_kernel(
    const W* __restrict__ Wb, const float* __restrict__ bias, const float* __restrict__ x,
    int n_in, int hid, float* __restrict__ h) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  constexpr int kStages = SPP * kL1Prod;                     // stages the loop runs
  constexpr int kXq = (kStages * kL1Stage / 4 + kL1Threads - 1) / kL1Threads;  // x float4 per thread
  __shared__ __align__(16) float xs[kStages * kL1Stage];
  __shared__ float4 ring[2][kL1Stage / 4][kL1Chains];
  const int b = blockIdx.y;
  const int c0 = blockIdx.x * kL1Chains;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nblk = (n_in + 7) >> 3;                 // 8-step blocks
  const int nst = (n_in + kL1Stage - 1) / kL1Stage;  // stages holding steps
  const int p = wave - 1;                            // producer index (consumer: -1)
  // 1. x loads (first, so that waiting for them leaves the weight loads in flight)
  const float* xr = x + (size_t)b * n_in;
  const bool vec = (n_in & 3) == 0;
  float4 xv[kXq];
#pragma unroll
  for (int q = 0; q < kXq; ++q) {
    const int i = threadIdx.x + q * kL1Threads;
    xv[q] = vec ? reinterpret_cast<const float4*>(xr)[min(i, (n_in >> 2) - 1)] : make_float4(0, 0, 0, 0);
  }
  const float bv = bias[min(c0 + (lane & (kL1Chains - 1)), hid - 1)];
  // 2. every weight of the block: producer p owns stages p, p + kL1Prod, ...
  // Loads are unconditional (clamped): out-of-range blocks and chains are
  // never consumed, and branch-free loads let the compiler count them.
  V pre[SPP][kL1Q];
  if (wave > 0) {
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
  // 3. x to LDS
  if (vec) {
    // clamped, unconditional stores (see stage_f4)
#pragma unroll
    for (int q = 0; q < kXq; ++q)
      reinterpret_cast<float4*>(xs)[min((int)threadIdx.x + q * kL1Threads, (n_in >> 2) - 1)] = xv[q];
  } else {
    for (int j = threadIdx.x; j < n_in; j += kL1Threads) xs[j] = xr[j];
  }
  lds_barrier();
  auto make_stage = [&](int st, const V (&r)[kL1Q]) {
    float4(*dst)[kL1Chains] = ring[st & 1];
#pragma unroll
    for (int q = 0; q < kL1Q; ++q) {
      const int pr = lane + 64 * q;
      const int blk = pr / kL1Chains, ch = pr % kL1Chains;
      const int j0 = (st * (kL1Stage / 8) + blk) * 8;
      float w[8], pv[8];
      B8::widen(r[q], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = __fmul_rn(w[e], xs[min(j0 + e, kStages * kL1Stage - 1)]);
      dst[2 * blk][ch] = make_float4(pv[0], pv[1], pv[2], pv[3]);
      dst[2 * blk + 1][ch] = make_float4(pv[4], pv[5], pv[6], pv[7]);
    }
  };
  // 4. kStages + 1 barriers on every wave: stage st is written before
  // barrier st and read between barriers st and st + 1.
  float s = -0.0f;
  if (wave > 0) {
#pragma unroll
    for (int st = 0; st < kStages; ++st) {
      if (st % kL1Prod == p) make_stage(st, pre[st / kL1Prod]);
      lds_barrier();
    }
    lds_barrier();
  } else {
    const int ln = lane < kL1Chains ? lane : kL1Chains - 1;
    lds_barrier();
    for (int st = 0; st < kStages; ++st) {
      const float4(*src)[kL1Chains] = ring[st & 1];
      const int steps = min(kL1Stage, n_in - st * kL1Stage);
      if (steps == kL1Stage) {
#pragma unroll
        for (int q = 0; q < kL1Stage / 4; ++q) {
          const float4 v = src[q][ln];
          s = __fadd_rn(s, v.x);
          s = __fadd_rn(s, v.y);
          s = __fadd_rn(s, v.z);
          s = __fadd_rn(s, v.w);
        }
      } else if (steps > 0) {
        for (int q = 0; q < kL1Stage / 4; ++q) {
          if (4 * q >= steps) break;
          const float4 v = src[q][ln];
          const float e[4] = {v.x, v.y, v.z, v.w};
          for (int u = 0; u < 4 && 4 * q + u < steps; ++u) s = __fadd_rn(s, e[u]);
        }
      }
      lds_barrier();
    }
  }
  (void)nst;
  const int chain = c0 + lane;
  if (wave == 0 && lane < kL1Chains && chain < hid)
    h[(size_t)b * hid + chain] = fmaxf(__fadd_rn(s, bv), 0.0f);
}

// Layer 1 for n_in <= kL1LdsIn (pred_l1.hpp), one block per kL1Chains hidden
// units of row blockIdx.y.
template <typename W>
__global__ __launch_bounds__(kL1LdsThreads) void pred_l1_lds_kernel(
    const W* __restrict__ Wb, const float* __restrict__ bias, const float* __restrict__ x,
    int n_in, int hid, float* __restrict__ h, const float* __restrict__ norm_w,
    float* __restrict__ inv_out, float eps, float* __restrict__ xn_out = nullptr) {
  extern __shared__ float4 lds4[];
  pred_l1_lds_body<W>(blockIdx.x, blockIdx.y, Wb, bias, x, n_in, hid, h, norm_w, inv_out, eps, lds4, xn_out);
}

// Layer 1 for a batch of rows (BF16 weights, n_in a multiple of
// kLbSlots * kLbStage, at most kL1LdsIn): a block owns kLbOut hidden units for
// kLbRows rows, i.e. 16 chains, one per consumer lane (lanes 16-63 leave).
// pred_l1_lds holds every product of its block in LDS, so one block fits per
// CU and a batch's blocks run in several rounds; here the products pass
// through a ring of kLbSlots stages (64 KB of LDS per block with the rows' x),
// so all blocks of a 16-row batch run at once.  Two rows per block measured
// 19.2 us per 7B batch-16 call against 22.4 with four (the consumer's window
// reads move half the bytes); one row per block breaks the ring's swizzle.
//  * The rows' x go to LDS once (the block's only barrier) and the producers
//    hold every weight of the block in registers from the start.
//  * Producer p forms stages p, p + kLbProd, ... into slot stage % kLbSlots
//    once the consumer has released that slot, then publishes the stage index
//    in ready[slot]; the consumer releases a slot by writing the stage index
//    to freed[slot].  LDS flags, not barriers: no wave waits for another
//    except on the data it needs.  One consumer and three producers, one wave
//    per SIMD, so no producer takes issue slots from the chain.
//  * Quad q of chain c sits at position c ^ (q & 14) of its ring row: the
//    consumer's 16 lanes still read one contiguous row, and a producer's
//    write instruction (8 quads x 8 chains) spreads evenly over the banks
//    instead of hitting one bank group 8 times.  Eight slots of 64 steps give
//    a producer six stages of slack to refill a slot: it takes about three
//    times as long to form a stage as the consumer takes to add one.
//  * The consumer adds each chain's products in step order through a window
//    of two stages of quads: while stage s is added, its registers are
//    refilled with stage s + 2, whose flag was checked first (flags are
//    checked and slots released two stages at a time).  The loop is unrolled by the ring
//    size, so every LDS address is a fixed register plus an immediate offset.
// Each chain is the same sequential sum as pred_l1_lds_kernel's.
constexpr int kLbOut = 8, kLbRows = 2, kLbChains = kLbOut * kLbRows;
static_assert(kLbChains == 16 || kLbChains == 32, "the ring swizzle c ^ (q & 14) stays inside a row");
constexpr int kLbStage = 64, kLbSlots = 8, kLbProd = 3;
constexpr int kLbThreads = 64 * (1 + kLbProd);
constexpr int kLbStages = kL1LdsIn / kLbStage;
constexpr int kLbSpp = (kLbStages + kLbProd - 1) / kLbProd;  // stages per producer (at most)
constexpr int kLbQuads = kLbStage / 4;
constexpr int kLbRingBytes = kLbSlots * kLbQuads * kLbChains * 16;
constexpr int kLbLdsBytes = kLbRingBytes + kLbRows * kL1LdsIn * 4;
constexpr int kLbSpinMax = 1 << 22;  // a flag that never arrives ends the wait (no hang)
// A wait that reaches its spin limit carries on (so the kernel always exits)
// with a slot that may still be in use or hold stale products: the scores of
// that call are not trusted, and the kernel records it in *err (read and
// cleared by kh_predictor_status).
static_assert(kLbRingBytes <= 65536, "ring addressed by immediate offsets");

__device__ __forceinline__ int lb_flag(const int* f) {
  return __hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lb_publish(int* f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ constexpr int lb_swz(int q) { return q & 14; }
// The consumer's side of the flags: relaxed (no wait), ordered by the LDS
// itself (a wave's LDS operations execute in issue order) and by compiler
// barriers, so a flag read can be issued a stage ahead of its use.
__device__ __forceinline__ int lb_peek(const int* f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lb_release(int* f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__global__ __launch_bounds__(kLbThreads) void pred_l1_batch_kernel(
    const uint16_t* __restrict__ Wb, const float* __restrict__ bias, const float* __restrict__ x,
    int n_in, int hid, int batch, float* __restrict__ h, int spin_max, int* __restrict__ err) {
  extern __shared__ float4 lb4[];
  float4* ring = lb4;                                             // [slot][quad][chain]
  float* xs = reinterpret_cast<float*>(lb4 + kLbRingBytes / 16);  // [kLbRows][n_in]
  __shared__ int ready[kLbSlots], freed[kLbSlots];
  const int c0 = blockIdx.x * kLbOut, r0 = blockIdx.y * kLbRows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nst = n_in / kLbStage;
  const int n4 = n_in >> 2;
  // Every x load is requested before the weights and before any store
  // (clamped, unconditional: see stage_f4); rows past the batch re-read the
  // last row, their chains unused.
  constexpr int kXq = (kLbRows * kL1LdsIn / 4 + kLbThreads - 1) / kLbThreads;
  float4 xv[kXq];
#pragma unroll
  for (int q = 0; q < kXq; ++q) {
    const int i = min((int)threadIdx.x + q * kLbThreads, kLbRows * n4 - 1);
    const int r = i / n4;
    xv[q] = reinterpret_cast<const float4*>(x + (size_t)min(r0 + r, batch - 1) * n_in)[i - r * n4];
  }
  if (threadIdx.x < kLbSlots) {
    ready[threadIdx.x] = -1;
    freed[threadIdx.x] = -1;
  }
  // producer p = wave - 1: lane -> (8-step block jl of a stage, output o)
  const int p = wave - 1, jl = lane >> 3, po = lane & 7;
  uint4 wr[kLbSpp];
  if (wave > 0) {
    const uint4* __restrict__ wv = reinterpret_cast<const uint4*>(Wb);
#pragma unroll
    for (int i = 0; i < kLbSpp; ++i) {
      const int st = min(p + kLbProd * i, nst - 1);  // clamped, unused past nst
      wr[i] = wv[(size_t)(st * (kLbStage / 8) + jl) * hid + min(c0 + po, hid - 1)];
    }
  }
#pragma unroll
  for (int q = 0; q < kXq; ++q)
    reinterpret_cast<float4*>(xs)[min((int)threadIdx.x + q * kLbThreads, kLbRows * n4 - 1)] = xv[q];
  lds_barrier();
  bool gave_up = false;
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < kLbSpp; ++i) {
      const int st = p + kLbProd * i;
      if (st >= nst) break;
      const int slot = st % kLbSlots;
      // the consumer must have released this slot's previous stage
      for (int n = 0; st >= kLbSlots && lb_flag(&freed[slot]) < st - kLbSlots; ++n) {
        if (n == spin_max) {
          gave_up = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      const int j0 = st * kLbStage + jl * 8;
      float4* row0 = ring + (slot * kLbQuads + 2 * jl) * kLbChains;  // quads 2 jl, 2 jl + 1
      const int sw = lb_swz(2 * jl);  // the same for both quads
      float w[8];
      Blk8<uint16_t>::widen(wr[i], w);
#pragma unroll
      for (int r = 0; r < kLbRows; ++r) {
        const float4 xa = reinterpret_cast<const float4*>(xs + r * n_in + j0)[0];
        const float4 xb = reinterpret_cast<const float4*>(xs + r * n_in + j0)[1];
        const int c = (r * kLbOut + po) ^ sw;
        row0[c] = make_float4(__fmul_rn(w[0], xa.x), __fmul_rn(w[1], xa.y), __fmul_rn(w[2], xa.z),
                              __fmul_rn(w[3], xa.w));
        row0[kLbChains + c] = make_float4(__fmul_rn(w[4], xb.x), __fmul_rn(w[5], xb.y),
                                          __fmul_rn(w[6], xb.z), __fmul_rn(w[7], xb.w));
      }
      lb_publish(&ready[slot], st);  // every lane stores the same value: no branch
    }
    if (gave_up) *err = 1;
    return;
  }
  // consumer: lane ch reads quad q of slot sl at ring[(sl * kLbQuads + q) * kLbChains + (ch ^ swz(q))].
  // Lanes past the chains leave, so each window read moves 256 bytes of
  // LDS, not 1 KB (the LDS, shared with the producers, sets the pace).
  if (lane >= kLbChains) return;
  const int ch = lane;
  const float4* cb[16];
#pragma unroll
  for (int g = 0; g < 16; g += 2) cb[g] = ring + (ch ^ g);
  float s = -0.0f;
  // window of two stages: rq[16 h + q] holds quad q of the stage in slot
  // parity h; a stage's quads are refilled with those two stages ahead, so a
  // read has 64 adds (about 400 cycles) to arrive
  float4 rq[2 * kLbQuads];
  for (int n = 0;; ++n) {
    const int f0 = lb_flag(&ready[0]), f1 = lb_flag(&ready[1]);
    if (f0 >= 0 && (nst < 2 || f1 >= 1)) break;
    if (n == spin_max) {
      gave_up = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int q = 0; q < 2 * kLbQuads; ++q) rq[q] = cb[lb_swz(q % kLbQuads)][q * kLbChains];
  // One stage: add slot SL's quads, refilling them from slot SL + 2.
  auto body = [&](auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
    constexpr int H = SL % 2, NS = (SL + 2) % kLbSlots;
    constexpr int kRefill = 8;
#pragma unroll
    for (int q = 0; q < kLbQuads; q += kRefill) {
#pragma unroll
      for (int u = 0; u < kRefill; ++u) {
        const float4 v = rq[H * kLbQuads + q + u];
        s = __fadd_rn(s, v.x);
        s = __fadd_rn(s, v.y);
        s = __fadd_rn(s, v.z);
        s = __fadd_rn(s, v.w);
      }
#pragma unroll
      for (int u = 0; u < kRefill; ++u)
        rq[H * kLbQuads + q + u] = cb[lb_swz(q + u)][(NS * kLbQuads + q + u) * kLbChains];
      __builtin_amdgcn_sched_barrier(0);
    }
    // pin the chain here: otherwise the adds may be sunk past the next flag
    // loop, and the window's registers double
    asm volatile("" : "+v"(s));
  };
  // Stages st and st + 1 (slots SL, SL + 1).  Their refills read stages
  // st + 2 and st + 3, whose flags were read during the previous pair (f2,
  // f3), so the check costs no wait unless a producer is behind; the flags
  // the next pair needs are read between this pair's two stages.  The two
  // slots of the previous pair, whose quads have been added, are released
  // together.  Past the last stage the refills read stale slots, never added.
  int f2 = lb_peek(&ready[2]), f3 = lb_peek(&ready[3]);
  auto pair = [&](auto slot_c, int st) {
    constexpr int SL = decltype(slot_c)::value;
    constexpr int S2 = (SL + 2) % kLbSlots, S3 = (SL + 3) % kLbSlots;
    constexpr int S4 = (SL + 4) % kLbSlots, S5 = (SL + 5) % kLbSlots;
    for (int n = 0; !((st + 2 >= nst || f2 >= st + 2) && (st + 3 >= nst || f3 >= st + 3)); ++n) {
      if (n == spin_max) {
        gave_up = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      f2 = lb_flag(&ready[S2]);
      f3 = lb_flag(&ready[S3]);
    }
    asm volatile("" ::: "memory");  // no refill read moves above the check
    // for st == 0 these rewrite the initial -1s
    lb_release(&freed[(SL + kLbSlots - 2) % kLbSlots], st - 2);
    lb_release(&freed[(SL + kLbSlots - 1) % kLbSlots], st - 1);
    body(slot_c);
    f2 = lb_peek(&ready[S4]);
    f3 = lb_peek(&ready[S5]);
    body(std::integral_constant<int, (SL + 1) % kLbSlots>{});
  };
  for (int st = 0; st < nst; st += kLbSlots) {
    pair(std::integral_constant<int, 0>{}, st);
    pair(std::integral_constant<int, 2>{}, st + 2);
    pair(std::integral_constant<int, 4>{}, st + 4);
    pair(std::integral_constant<int, 6>{}, st + 6);
  }
  const int r = ch / kLbOut, o = ch % kLbOut;
  if (r0 + r < batch && c0 + o < hid)
    h[(size_t)(r0 + r) * hid + c0 + o] = fmaxf(__fadd_rn(s, bias[c0 + o]), 0.0f);
  if (gave_up) *err = 1;
}

// Layer 2 (short chains): one lane per output, the whole weight row in
// registers (n_hid <= 256), the hidden vector in LDS.  Scores = sigmoid.
// One wave per block, so the weight stream is spread over as many CUs as
// there are waves.
constexpr int kL2Threads = 64;

// With mm set, each block also writes the (min, max) order-preserving keys of
// its scores to mm[b][block]: the key bounds the top-k kernel starts from
// (one slot per block, so no atomics contend on a single address).
// TOPK (n_out <= 64, one block per row): the block also selects the top k
// scores of its row, as topk_kernel does (key descending, ties by index), and
// writes their indices to ids[b][min(k, n_out)] in `order`.
template <typename W, bool TOPK = false>
__global__ __launch_bounds__(kL2Threads) void pred_l2_kernel(const W* __restrict__ Wb,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ hin, int n_hid,
                                                      int n_out, float* __restrict__ out,
                                                      uint32_t* __restrict__ mm, int k = 0,
                                                      int order = 0,
                                                      int32_t* __restrict__ ids = nullptr) {
  using V = typename Blk8<W>::V;
  __shared__ __align__(16) float hs[kMaxL2Hid + 4 * kL2Hw];
  __shared__ uint64_t tab[32];
  const int b = blockIdx.y;
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  // The hidden vector (one float4 per thread) is requested first, then the
  // bias and the weight row, and only then stored to LDS: waiting for the
  // hidden values leaves the weight loads in flight.
  const bool vec = (n_hid & 3) == 0 && n_hid <= 4 * kL2Threads;
  const float4 hv = vec ? reinterpret_cast<const float4*>(hin + (size_t)b * n_hid)
                              [min((int)threadIdx.x, (n_hid >> 2) - 1)]
                        : make_float4(0, 0, 0, 0);
  const bool ok = o < n_out;
  const int oc = ok ? o : 0;
  const float bv = bias[oc];  // used after the chain
  V w[kMaxL2Hid / 8];
  l2_load<W>(Wb, n_hid, n_out, oc, w);
  if (vec) {
    reinterpret_cast<float4*>(hs)[min((int)threadIdx.x, (n_hid >> 2) - 1)] = hv;  // clamped (see stage_f4)
  } else {
    for (int i = threadIdx.x; i < n_hid; i += blockDim.x) hs[i] = hin[(size_t)b * n_hid + i];
  }
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  const float s = l2_chain<W>(w, n_hid, hs);
  const float score = sigmoid_ref_t(__fadd_rn(s, bv), tab);
  if (ok) out[(size_t)b * n_out + o] = score;
  if (mm) {
    const uint32_t key = f32_key(score);
    const uint32_t kmax = wave_max_u32(ok ? key : 0u);
    const uint32_t kmin = wave_min_u32(ok ? key : 0xffffffffu);
    if (threadIdx.x == 0)
      reinterpret_cast<uint2*>(mm)[(size_t)b * gridDim.x + blockIdx.x] = make_uint2(kmin, kmax);
  }
  if constexpr (TOPK) {
    // select_top_k's stable descending sort (mlp_predictor.rs:128-131) over
    // the row's n_out <= 64 scores: lane o's rank among them
    const int rank = l2_wave_rank(f32_key(score), o, n_out);
    const int kk = min(k, n_out);
    const bool sel = ok && rank < kk;
    const uint64_t bal = __ballot(sel);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
    if (sel) ids[(size_t)b * kk + (order == KH_ORDER_SCORE ? rank : below)] = o;
  }
}

// Layer 2 for several rows (BF16 weights, n_hid <= kMaxL2Hid, n_hid % 8 == 0):
// block (x, y) owns outputs [64 x, 64 x + 64) of rows [kL2Rows y, ...).  The
// outputs' weight rows go to LDS once (one 1 KB direct load per 8-input block,
// [block][output]), the rows' hidden vectors beside them, and wave w runs the
// chains of rows 2w and 2w + 1: each weight read from LDS serves both rows.
// The work is VALU-bound (a separately rounded multiply and add per term), so
// blocks stay small (two waves) and every CU takes a few.  pred_l2_kernel
// instead takes one row per block.  The chains, scores and key bounds are
// pred_l2_kernel's.
constexpr int kL2Rows = 4;
constexpr int kL2RowThreads = 32 * kL2Rows;  // two rows per wave
constexpr int kL2RowHs = kMaxL2Hid + 4;      // LDS row stride of the hidden vectors (floats)

__global__ __launch_bounds__(kL2RowThreads) void pred_l2_rows_kernel(
    const uint16_t* __restrict__ Wb, const float* __restrict__ bias, const float* __restrict__ hin, int n_hid,
    int n_out, int batch, float* __restrict__ out, uint32_t* __restrict__ mm) {
  __shared__ __align__(16) uint4 wl[kMaxL2Hid / 8][64];
  __shared__ __align__(16) float hs[kL2Rows][kL2RowHs];
  __shared__ uint64_t tab[32];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int o = blockIdx.x * 64 + lane;
  const bool ok = o < n_out;
  const int oc = ok ? o : n_out - 1;
  const int rb = blockIdx.y * kL2Rows;
  const int nblk = n_hid >> 3;
  const uint4* __restrict__ wv = reinterpret_cast<const uint4*>(Wb);
  // weight rows: wave w loads 8-input blocks w, w + 8, ... (64 outputs, 1 KB each)
  for (int jb = wave; jb < nblk; jb += kL2RowThreads / 64)
    __builtin_amdgcn_global_load_lds(wv + (size_t)jb * n_out + oc, &wl[jb][0], 16, 0, 0);
  // hidden vectors of the block's rows (rows past the batch repeat the last, unused)
  const int n4 = n_hid >> 2;
  for (int i = t; i < kL2Rows * n4; i += kL2RowThreads) {
    const int r = i / n4, c = i - r * n4;
    reinterpret_cast<float4*>(&hs[r][0])[c] =
        reinterpret_cast<const float4*>(hin + (size_t)min(rb + r, batch - 1) * n_hid)[c];
  }
  if (t < 32) tab[t] = kExp2Tab[t];
  const float bv = bias[oc];
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int r0 = 2 * wave, r1 = 2 * wave + 1;
  const float4* h0 = reinterpret_cast<const float4*>(&hs[r0][0]);
  const float4* h1 = reinterpret_cast<const float4*>(&hs[r1][0]);
  float s0 = -0.0f, s1 = -0.0f;
#pragma unroll 4
  for (int jb = 0; jb < nblk; ++jb) {
    float wf[8];
    Blk8<uint16_t>::widen(wl[jb][lane], wf);
    const float4 a0 = h0[2 * jb], a1 = h0[2 * jb + 1], c0 = h1[2 * jb], c1 = h1[2 * jb + 1];
    s0 = __fadd_rn(s0, __fmul_rn(wf[0], a0.x));
    s1 = __fadd_rn(s1, __fmul_rn(wf[0], c0.x));
    s0 = __fadd_rn(s0, __fmul_rn(wf[1], a0.y));
    s1 = __fadd_rn(s1, __fmul_rn(wf[1], c0.y));
    s0 = __fadd_rn(s0, __fmul_rn(wf[2], a0.z));
    s1 = __fadd_rn(s1, __fmul_rn(wf[2], c0.z));
    s0 = __fadd_rn(s0, __fmul_rn(wf[3], a0.w));
    s1 = __fadd_rn(s1, __fmul_rn(wf[3], c0.w));
    s0 = __fadd_rn(s0, __fmul_rn(wf[4], a1.x));
    s1 = __fadd_rn(s1, __fmul_rn(wf[4], c1.x));
    s0 = __fadd_rn(s0, __fmul_rn(wf[5], a1.y));
    s1 = __fadd_rn(s1, __fmul_rn(wf[5], c1.y));
    s0 = __fadd_rn(s0, __fmul_rn(wf[6], a1.z));
    s1 = __fadd_rn(s1, __fmul_rn(wf[6], c1.z));
    s0 = __fadd_rn(s0, __fmul_rn(wf[7], a1.w));
    s1 = __fadd_rn(s1, __fmul_rn(wf[7], c1.w));
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int b = rb + (u ? r1 : r0);
    const float score = sigmoid_ref_t(__fadd_rn(u ? s1 : s0, bv), tab);
    if (b < batch) {
      if (ok) out[(size_t)b * n_out + o] = score;
      if (mm) {
        const uint32_t key = f32_key(score);
        const uint32_t kmax = wave_max_u32(ok ? key : 0u);
        const uint32_t kmin = wave_min_u32(ok ? key : 0xffffffffu);
        if (lane == 0) reinterpret_cast<uint2*>(mm)[(size_t)b * gridDim.x + blockIdx.x] = make_uint2(kmin, kmax);
      }
    }
  }
}

// Generic layer for shapes outside the fast kernels' limits: one lane per
// output, sequential over the input.  act 0 = max(., 0), 1 = sigmoid.
template <int ACT, typename W>
__global__ __launch_bounds__(64) void chain_layer_kernel(const W* __restrict__ Wb,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ in, int n_in,
                                                         int n_out, float* __restrict__ out) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  const int o = blockIdx.x * 64 + threadIdx.x;
  const int b = blockIdx.y;
  const float* __restrict__ xin = in + (size_t)b * n_in;
  const bool ok = o < n_out;
  const int oc = ok ? o : 0;
  const V* __restrict__ wv = reinterpret_cast<const V*>(Wb);
  float s = -0.0f;
  const int nblk = (n_in + 7) >> 3;
  for (int jb = 0; jb < nblk; ++jb) {
    float wf[8];
    B8::widen(wv[(size_t)jb * n_out + oc], wf);
    for (int e = 0; e < 8 && jb * 8 + e < n_in; ++e)
      s = __fadd_rn(s, __fmul_rn(wf[e], xin[jb * 8 + e]));
  }
  if (!ok) return;
  const float z = __fadd_rn(s, bias[o]);
  out[(size_t)b * n_out + o] = ACT == 0 ? fmaxf(z, 0.0f) : sigmoid_ref(z);
}

// ---------------------------------------------------------------- top-k
constexpr int kTopkThreads = 1024;
constexpr int kTopkRegMax = kTopkThreads * 64 - 1;  // keys per thread in registers: 16, 32 or 64
constexpr int kTopkStage = 32768;    // rows up to this size are loaded through LDS

// Score-order output: bitonic sort (descending) of the selected (key, ~index)
// pairs staged in sortbuf, then the indices.
__device__ void topk_score_order(const uint64_t* __restrict__ src, int kk, int32_t* __restrict__ ob,
                                 uint64_t* __restrict__ sv) {
  int P = 1;
  while (P < kk) P <<= 1;
  for (int i = threadIdx.x; i < P; i += blockDim.x) sv[i] = i < kk ? src[i] : 0ull;
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint64_t a = sv[i], c = sv[j];
          if (desc ? (a < c) : (a > c)) {
            sv[i] = c;
            sv[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < kk; i += blockDim.x)
    ob[i] = (int32_t)(0xffffffffu - (uint32_t)(sv[i] & 0xffffffffu));
}

// One block per row.  Thread t holds the keys of the contiguous index range
// [t*kpt, (t+1)*kpt) in registers, so every pass runs from registers and the
// selected indices come out in ascending order from one exclusive scan: the
// k-th key by topk_threshold (radix passes below the keys' common high bits,
// then a direct ranking of the boundary bin), then the compaction.
template <int kTopkPerThread>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores,
                                                            int n, int k, int order,
                                                            int32_t* __restrict__ out,
                                                            uint64_t* __restrict__ sortbuf,
                                                            const uint32_t* __restrict__ mm,
                                                            int nmm,
                                                            uint8_t* __restrict__ marks) {
  extern __shared__ __align__(16) uint64_t sort_lds[];
  __shared__ TopkLds<kTopkThreads> sh;
  const int b = blockIdx.x;
  const float* sc = scores + (size_t)b * n;
  const int kk0 = min(k, n);
  if (kk0 <= 0) return;
  int32_t* ob = out + (size_t)b * kk0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kpt = (n + kTopkThreads - 1) / kTopkThreads;  // <= kTopkPerThread (host-checked)
  // per-block key bounds written by the producing kernel (nmm slots per row),
  // requested with the scores
  const uint2 mmv = (mm && (int)threadIdx.x < nmm)
                        ? reinterpret_cast<const uint2*>(mm)[(size_t)b * nmm + threadIdx.x]
                        : make_uint2(0xffffffffu, 0u);
  const int i0 = threadIdx.x * kpt;
  const int cnt = max(0, min(kpt, n - i0));
  if (mm) {
    // reduced per wave while the scores are still in flight (requested first,
    // so waiting for them does not wait for the scores)
    const uint32_t a = wave_max_u32(mmv.y), c = wave_min_u32(mmv.x);
    if (lane == 0) {
      sh.wmax[wave] = a;
      sh.wmin[wave] = c;
    }
  }
  // Coalesced loads through LDS (a thread's own contiguous range would make
  // every wave load touch dozens of cache lines), then each thread reads its
  // range; the odd-or-power-of-two strides keep the LDS reads conflict-light.
  uint32_t* sstage = reinterpret_cast<uint32_t*>(sort_lds);
  const bool staged = n <= kTopkStage;
  if (!staged) {
    // too many scores to stage: each thread loads its own range directly
  } else if ((n & 3) == 0 && ((reinterpret_cast<uintptr_t>(sc) & 15) == 0)) {
    const float4* s4 = reinterpret_cast<const float4*>(sc);
    constexpr int kQ = (kTopkPerThread + 3) / 4;
    float4 v[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) v[q] = s4[min((int)threadIdx.x + q * kTopkThreads, (n >> 2) - 1)];
#pragma unroll
    for (int q = 0; q < kQ; ++q)  // clamped, unconditional (see stage_f4)
      reinterpret_cast<float4*>(sstage)[min((int)threadIdx.x + q * kTopkThreads, (n >> 2) - 1)] = v[q];
  } else {
    for (int i = threadIdx.x; i < n; i += kTopkThreads) sstage[i] = __float_as_uint(sc[i]);
  }
  for (int i = threadIdx.x; i < (1 << kTopkDigit); i += kTopkThreads) sh.hist[i] = 0;
  if (threadIdx.x == 0) sh.s_ncand = 0;
  lds_barrier();
  uint32_t key[kTopkPerThread];
#pragma unroll
  for (int j = 0; j < kTopkPerThread; ++j)
    key[j] = f32_key(staged ? __uint_as_float(sstage[min(i0 + j, n - 1)]) : sc[min(i0 + j, n - 1)]);
  if (!mm) {
    uint32_t kmax = 0u, kmin = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < kTopkPerThread; ++j)
      if (j < cnt) {
        kmax = max(kmax, key[j]);
        kmin = min(kmin, key[j]);
      }
    kmax = wave_max_u32(kmax);
    kmin = wave_min_u32(kmin);
    if (lane == 0) {
      sh.wmax[wave] = kmax;
      sh.wmin[wave] = kmin;
    }
    __syncthreads();
  }
  uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < kTopkThreads / 64; ++w) {
    mx = max(mx, sh.wmax[w]);
    mn = min(mn, sh.wmin[w]);
  }
  uint32_t T;
  int ties;
  topk_threshold<kTopkThreads, kTopkPerThread>(key, cnt, i0, kk0, mx, mn, sh, T, ties);
  // compaction in ascending index order: one iteration per selected key
  int pos;
  auto selm = topk_select_mask<kTopkThreads, kTopkPerThread>(key, cnt, T, ties, sh, pos);
  auto lowest = [](unsigned long long m) { return __ffsll(m) - 1; };
  if (order == KH_ORDER_ASCENDING && staged) {
    // ids staged in LDS (the scores there are dead: the keys are in
    // registers), then written with coalesced stores
    int32_t* sids = reinterpret_cast<int32_t*>(sort_lds);
    while (selm) {
      const int j = lowest(selm);
      if (pos < kk0) sids[pos] = i0 + j;
      ++pos;
      selm &= selm - 1;
    }
    lds_barrier();
    for (int i = threadIdx.x; i < kk0; i += kTopkThreads) ob[i] = sids[i];
    // union marks shared by the rows of a batch: every writer stores 1
    if (marks)
      for (int i = threadIdx.x; i < kk0; i += kTopkThreads) marks[sids[i]] = 1;
    return;
  }
  uint64_t* stage = sortbuf + (size_t)b * kk0;
  while (selm) {
    const int j = lowest(selm);
    if (pos < kk0) {
      if (order == KH_ORDER_ASCENDING) ob[pos] = i0 + j;
      else stage[pos] = ((uint64_t)key[j] << 32) | (uint32_t)(0xffffffffu - (uint32_t)(i0 + j));
      if (marks) marks[i0 + j] = 1;
    }
    ++pos;
    selm &= selm - 1;
  }
  if (order == KH_ORDER_ASCENDING) return;
  __threadfence_block();
  __syncthreads();
  topk_score_order(stage, kk0, ob, sort_lds);
}

// ---------------------------------------------------------------- union
// Rows up to this many neurons mark membership with one byte per neuron: the
// marks are plain byte stores (every writer stores 1), where a bitmap needs
// atomic ORs that serialise on the few words a batch of ids shares (26k ids
// of a 7B batch land on 344 words).
constexpr int kUnionFlagMax = 96 * 1024;

__global__ __launch_bounds__(1024) void union_kernel(const int32_t* __restrict__ ids, int batch,
                                                     int k, int n, int32_t* __restrict__ uni,
                                                     int32_t* __restrict__ count) {
  extern __shared__ uint32_t bits[];
  __shared__ int wsum[16];
  __shared__ int s_total;
  const bool bytes = n <= kUnionFlagMax;
  uint8_t* flags = reinterpret_cast<uint8_t*>(bits);
  // words of marks: 4 neurons per word (byte flags) or 32 (bitmap)
  const int nw = bytes ? (n + 3) >> 2 : (n + 31) >> 5;
  for (int i = threadIdx.x; i < nw; i += blockDim.x) bits[i] = 0;
  __syncthreads();
  // ids requested 32 per thread at a time (clamped, unconditional), so the
  // 16 rows of 1652 ids of a 7B batch arrive in one round trip
  constexpr int U = 32;
  const int total = batch * k;
  for (int i0 = 0; i0 < total; i0 += U * (int)blockDim.x) {
    int v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ids[min(i0 + (int)threadIdx.x + u * (int)blockDim.x, total - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + (int)threadIdx.x + u * (int)blockDim.x < total && v[u] >= 0 && v[u] < n) {
        if (bytes) flags[v[u]] = 1;
        else atomicOr(&bits[v[u] >> 5], 1u << (v[u] & 31));
      }
  }
  __syncthreads();
  // Compaction in ascending id order.  Byte flags: thread t owns the words
  // [t*per, t*per + per) (set bytes hold 1, so a word's popcount counts its
  // marks); one block scan.  Bitmap: one word per thread per round.
  if (bytes) {
    const int per = (nw + (int)blockDim.x - 1) / (int)blockDim.x;
    const int w0 = (int)threadIdx.x * per;
    int cnt = 0;
    for (int j = 0; j < per; ++j) cnt += w0 + j < nw ? __popc(bits[w0 + j]) : 0;
    int p = block_excl_scan(cnt, wsum, &s_total);
    for (int j = 0; j < per && w0 + j < nw; ++j) {
      uint32_t m = bits[w0 + j];
      while (m) {
        const int bit = __ffs(m) - 1;  // bit 8*b of byte b
        uni[p++] = 4 * (w0 + j) + (bit >> 3);
        m &= m - 1;
      }
    }
    if (threadIdx.x == 0) *count = s_total;
    return;
  }
  int base = 0;
  for (int w0 = 0; w0 < nw; w0 += blockDim.x) {
    const int w = w0 + threadIdx.x;
    const uint32_t word = w < nw ? bits[w] : 0u;
    const int pc = __popc(word);
    const int pos = block_excl_scan(pc, wsum, &s_total) + base;
    uint32_t m = word;
    int p = pos;
    while (m) {
      const int bit = __ffs(m) - 1;
      uni[p++] = (w << 5) + bit;
      m &= m - 1;
    }
    base += s_total;
  }
  if (threadIdx.x == 0) *count = base;
}

// Union from the byte marks the top-k kernel set (one byte per neuron, 1 if
// some row selected it): ascending ids and the count; the marks are cleared
// for the next call.  One block; thread t owns the mark words [t*per, ...).
__global__ __launch_bounds__(1024) void marks_union_kernel(uint32_t* __restrict__ marks, int n,
                                                           int32_t* __restrict__ uni,
                                                           int32_t* __restrict__ count) {
  __shared__ int wsum[16];
  __shared__ int s_total;
  const int nw = (n + 3) >> 2;
  const int per = (nw + (int)blockDim.x - 1) / (int)blockDim.x;
  const int w0 = (int)threadIdx.x * per;
  constexpr int kMaxPer = 8;  // n <= 32768 (host-checked)
  uint32_t w[kMaxPer];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    w[j] = (j < per && w0 + j < nw) ? marks[w0 + j] : 0u;
    cnt += __popc(w[j]);  // set bytes hold 1
  }
  int p = block_excl_scan(cnt, wsum, &s_total);
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    uint32_t m = w[j];
    while (m) {
      const int bit = __ffs(m) - 1;
      uni[p++] = 4 * (w0 + j) + (bit >> 3);
      m &= m - 1;
    }
    if (j < per && w0 + j < nw && w[j]) marks[w0 + j] = 0u;
  }
  if (threadIdx.x == 0) *count = s_total;
}

}  // namespace kh

using namespace kh;

struct kh_predictor {
  int in_dim = 0, hid = 0, out_dim = 0;
  bool bf16 = false;     // weights stored as BF16 bits (exact) or f32
  void* w1b = nullptr;   // [ceil(in/8)][hid][8]
  float* b1 = nullptr;
  void* w2b = nullptr;   // [ceil(hid/8)][out][8]
  float* b2 = nullptr;
  int* err = nullptr;    // device word: a batched layer-1 wait reached its spin limit
  int spin_max = kLbSpinMax;
  mutable StreamWs ws;   // scratch per stream (PredBufs)
};

namespace {

// Scratch of one predictor call.  hbuf [batch][hid]: layer-1 outputs;
// sbuf [batch][out]: scores; mm [batch][layer-2 blocks][2]: score key bounds
// per block; sortbuf [batch][k]: score-ordered top-k staging (score order
// only); marks [round_up(out, 4)]: union marks, zero between calls (union only).
struct PredBufs {
  float* hbuf = nullptr;
  float* sbuf = nullptr;
  uint32_t* mm = nullptr;
  uint64_t* sortbuf = nullptr;
  uint8_t* marks = nullptr;
};
enum { kWsH, kWsS, kWsMM, kWsSort, kWsMarks };

int l2_blocks(const kh_predictor* p) { return ceil_div(p->out_dim, kL2Threads); }

size_t sort_bytes(int64_t batch, int kk) { return sizeof(uint64_t) * (size_t)batch * (size_t)kk; }

// Buffers of a call with `batch` rows from the handle's workspace for stream
// st (sortbuf for a score-ordered top-k of kk per row when kk > 0; marks when
// asked).
int pred_bufs(const kh_predictor* p, hipStream_t st, int64_t batch, int kk, bool marks,
              PredBufs* b) {
  WsSet* w = p->ws.get(st);
  b->hbuf = static_cast<float*>(w->get(kWsH, sizeof(float) * batch * p->hid));
  b->sbuf = static_cast<float*>(w->get(kWsS, sizeof(float) * batch * p->out_dim));
  b->mm = static_cast<uint32_t*>(w->get(kWsMM, sizeof(uint32_t) * 2 * batch * l2_blocks(p)));
  if (!b->hbuf || !b->sbuf || !b->mm) return KH_ERR_ALLOC;
  if (kk > 0) {
    b->sortbuf = static_cast<uint64_t*>(w->get(kWsSort, sort_bytes(batch, kk)));
    if (!b->sortbuf) return KH_ERR_ALLOC;
  }
  if (marks) {
    // zero-filled once; the union kernel clears what it reads
    b->marks = static_cast<uint8_t*>(w->get(kWsMarks, (size_t)((p->out_dim + 3) & ~3), true));
    if (!b->marks) return KH_ERR_ALLOC;
  }
  return KH_OK;
}

}  // namespace

static bool all_bf16(const float* w, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &w[i], 4);
    if (u & 0xffffu) return false;
  }
  return true;
}

// Blocked transpose of a row-major [n_out][n_in] matrix into [ceil(n_in/8)][n_out][8].
template <typename T>
static std::vector<T> block_transpose(const float* w, int n_out, int n_in) {
  const int nb = (n_in + 7) / 8;
  std::vector<T> o((size_t)nb * n_out * 8, T(0));
  for (int r = 0; r < n_out; ++r)
    for (int j = 0; j < n_in; ++j) {
      const float v = w[(size_t)r * n_in + j];
      T t;
      if constexpr (sizeof(T) == 2) {
        uint32_t u;
        memcpy(&u, &v, 4);
        t = static_cast<T>(u >> 16);
      } else {
        t = v;
      }
      o[((size_t)(j / 8) * n_out + r) * 8 + (j % 8)] = t;
    }
  return o;
}

template <typename T>
static int upload(void** dst, const T* src, size_t n) {
  *dst = dev_alloc(sizeof(T) * (n ? n : 1));
  if (!*dst) return KH_ERR_ALLOC;
  if (n) KH_HIP(hipMemcpy(*dst, src, sizeof(T) * n, hipMemcpyHostToDevice));
  return KH_OK;
}

extern "C" int kh_predictor_create(int input_dim, int hidden_dim, int output_dim,
                                   const float* w1_host, const float* b1_host,
                                   const float* w2_host, const float* b2_host,
                                   kh_predictor** out) {
  KH_CHECK_ARG(out && w1_host && b1_host && w2_host && b2_host, "null argument");
  KH_CHECK_ARG(input_dim > 0 && hidden_dim > 0 && output_dim > 0, "dims must be positive");
  *out = nullptr;
  auto* p = new kh_predictor();
  p->in_dim = input_dim;
  p->hid = hidden_dim;
  p->out_dim = output_dim;
  p->bf16 = all_bf16(w1_host, (size_t)input_dim * hidden_dim) &&
            all_bf16(w2_host, (size_t)hidden_dim * output_dim);
  int rc;
  if (p->bf16) {
    auto w1b = block_transpose<uint16_t>(w1_host, hidden_dim, input_dim);
    auto w2b = block_transpose<uint16_t>(w2_host, output_dim, hidden_dim);
    rc = upload(&p->w1b, w1b.data(), w1b.size());
    if (rc == KH_OK) rc = upload(&p->w2b, w2b.data(), w2b.size());
  } else {
    auto w1b = block_transpose<float>(w1_host, hidden_dim, input_dim);
    auto w2b = block_transpose<float>(w2_host, output_dim, hidden_dim);
    rc = upload(&p->w1b, w1b.data(), w1b.size());
    if (rc == KH_OK) rc = upload(&p->w2b, w2b.data(), w2b.size());
  }
  void* b1 = nullptr;
  void* b2 = nullptr;
  if (rc == KH_OK) rc = upload(&b1, b1_host, hidden_dim);
  if (rc == KH_OK) rc = upload(&b2, b2_host, output_dim);
  p->b1 = static_cast<float*>(b1);
  p->b2 = static_cast<float*>(b2);
  if (rc == KH_OK) {
    const int zero = 0;
    void* e = nullptr;
    rc = upload(&e, &zero, 1);
    p->err = static_cast<int*>(e);
  }
  if (rc != KH_OK) {
    kh_predictor_destroy(p);
    return rc;
  }
  *out = p;
  return KH_OK;
}

extern "C" int kh_predictor_destroy(kh_predictor* p) {
  if (!p) return KH_OK;
  dev_free(p->w1b);
  dev_free(p->b1);
  dev_free(p->w2b);
  dev_free(p->b2);
  dev_free(p->err);
  delete p;
  return KH_OK;
}

extern "C" int kh_predictor_status(const kh_predictor* p) {
  KH_CHECK_ARG(p != nullptr, "null argument");
  KH_HIP(hipDeviceSynchronize());
  int v = 0;
  KH_HIP(hipMemcpy(&v, p->err, sizeof(int), hipMemcpyDeviceToHost));
  if (v == 0) return KH_OK;
  KH_HIP(hipMemset(p->err, 0, sizeof(int)));
  set_error("a batched layer-1 wait reached its spin limit: the scores of that call are not trusted");
  return KH_ERR_HIP;
}

extern "C" int kh_predictor_set_spin_limit(kh_predictor* p, int spins) {
  KH_CHECK_ARG(p != nullptr, "null argument");
  KH_CHECK_ARG(spins >= 1, "spin limit %d must be at least 1", spins);
  p->spin_max = spins;
  return KH_OK;
}

extern "C" int kh_predictor_dims(const kh_predictor* p, int* input_dim, int* hidden_dim, int* output_dim) {
  KH_CHECK_ARG(p && input_dim && hidden_dim && output_dim, "null argument");
  *input_dim = p->in_dim;
  *hidden_dim = p->hid;
  *output_dim = p->out_dim;
  return KH_OK;
}

// Inverse of block_transpose for one stored matrix.
template <typename T>
static int download_blocked(const void* src, int n_out, int n_in, float* w) {
  const int nb = (n_in + 7) / 8;
  std::vector<T> o((size_t)nb * n_out * 8);
  KH_HIP(hipMemcpy(o.data(), src, o.size() * sizeof(T), hipMemcpyDeviceToHost));
  for (int r = 0; r < n_out; ++r)
    for (int j = 0; j < n_in; ++j) {
      const T t = o[((size_t)(j / 8) * n_out + r) * 8 + (j % 8)];
      float v;
      if constexpr (sizeof(T) == 2) {
        const uint32_t u = uint32_t(t) << 16;
        memcpy(&v, &u, 4);
      } else {
        v = t;
      }
      w[(size_t)r * n_in + j] = v;
    }
  return KH_OK;
}

extern "C" int kh_predictor_weights(const kh_predictor* p, float* w1_host, float* b1_host, float* w2_host,
                                    float* b2_host) {
  KH_CHECK_ARG(p && w1_host && b1_host && w2_host && b2_host, "null argument");
  int rc = p->bf16 ? download_blocked<uint16_t>(p->w1b, p->hid, p->in_dim, w1_host)
                   : download_blocked<float>(p->w1b, p->hid, p->in_dim, w1_host);
  if (rc != KH_OK) return rc;
  rc = p->bf16 ? download_blocked<uint16_t>(p->w2b, p->out_dim, p->hid, w2_host)
               : download_blocked<float>(p->w2b, p->out_dim, p->hid, w2_host);
  if (rc != KH_OK) return rc;
  KH_HIP(hipMemcpy(b1_host, p->b1, sizeof(float) * p->hid, hipMemcpyDeviceToHost));
  KH_HIP(hipMemcpy(b2_host, p->b2, sizeof(float) * p->out_dim, hipMemcpyDeviceToHost));
  return KH_OK;
}

// A top-k request that layer 2 may serve itself (done = true when it did).
struct TopkReq {
  int k = 0, order = 0;
  int32_t* ids = nullptr;
  bool done = false;
};

// Compute units of the current device (cached per device).
static int device_cus() {
  static std::mutex mu;
  static std::vector<int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)cus.size() <= dev) cus.resize(dev + 1, 0);
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                   ? n : 256;
  }
  return cus[dev];
}

static int set_kernel_attrs() {
  static std::once_flag once;
  static int rc = KH_OK;
  std::call_once(once, [] {
    auto lds = [](const void* f, int bytes) {
      if (rc == KH_OK && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) !=
                             hipSuccess) {
        set_error("hipFuncSetAttribute failed");
        rc = KH_ERR_HIP;
      }
    };
    lds(reinterpret_cast<const void*>(&pred_l1_lds_kernel<uint16_t>), kL1LdsBytes);
    lds(reinterpret_cast<const void*>(&pred_l1_lds_kernel<float>), kL1LdsBytes);
    lds(reinterpret_cast<const void*>(&pred_l1_batch_kernel), kLbLdsBytes);
    lds(reinterpret_cast<const void*>(&topk_kernel<6>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<8>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<11>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<12>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<16>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<32>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&topk_kernel<64>), 136 * 1024);
    lds(reinterpret_cast<const void*>(&union_kernel), 96 * 1024);
  });
  return rc;
}

// Layers 1 and 2 into scores (b.sbuf or the caller's array).  With mm set,
// layer 2 also writes the per-block score key bounds; with tk set, layer 2
// selects the top k itself when the row fits one wave (tk->done).
template <typename W>
static int l2_typed(const kh_predictor* p, const float* hbuf, int64_t batch, float* scores,
                    hipStream_t st, uint32_t* mm, TopkReq* tk);

template <typename W>
static int predict_typed(const kh_predictor* p, const float* x, int64_t batch, float* scores,
                         float* hbuf, hipStream_t st, const NormIn& nrm, uint32_t* mm,
                         TopkReq* tk) {
  const W* w1 = static_cast<const W*>(p->w1b);
  const W* w2 = static_cast<const W*>(p->w2b);
  const int l1_stages = ceil_div(p->in_dim, kL1Stage);
  if (nrm.w && (p->in_dim % 4 != 0 || !nrm.inv)) {
    set_error("the fused RmsNorm needs an input size that is a multiple of 4 and a scale buffer");
    return KH_ERR_ARG;
  }
  int rc = set_kernel_attrs();
  if (rc != KH_OK) return rc;
  // pred_l1_lds fits one block per CU; the batched kernel pays off once its
  // blocks would need more than one round of the device's CUs.
  if (std::is_same<W, uint16_t>::value && batch > 1 && !nrm.w && p->in_dim <= kL1LdsIn &&
      p->in_dim % (kLbSlots * kLbStage) == 0 &&
      (int64_t)ceil_div(p->hid, kL1Chains) * batch > device_cus())
    hipLaunchKernelGGL(pred_l1_batch_kernel, dim3(ceil_div(p->hid, kLbOut), ceil_div(batch, kLbRows)),
                       dim3(kLbThreads), kLbLdsBytes, st, static_cast<const uint16_t*>(p->w1b), p->b1,
                       x, p->in_dim, p->hid, static_cast<int>(batch), hbuf, p->spin_max, p->err);
  else if (p->in_dim <= kL1LdsIn)
    hipLaunchKernelGGL(pred_l1_lds_kernel<W>, dim3(ceil_div(p->hid, kL1Chains), batch),
                       dim3(kL1LdsThreads), kL1LdsBytes, st, w1, p->b1, x, p->in_dim, p->hid, hbuf,
                       nrm.w, nrm.inv, nrm.eps);
  else if (nrm.w) {
    set_error("the fused RmsNorm supports predictor inputs up to %d", kL1LdsIn);
    return KH_ERR_UNSUPPORTED;
  }
  else if (l1_stages <= 8 * kL1Prod)
    hipLaunchKernelGGL((pred_l1_kernel<W, 8>), dim3(ceil_div(p->hid, kL1Chains), batch),
                       dim3(kL1Threads), 0, st, w1, p->b1, x, p->in_dim, p->hid, hbuf);
  else if (p->in_dim <= kMaxL1In)
    hipLaunchKernelGGL((pred_l1_kernel<W, 16>), dim3(ceil_div(p->hid, kL1Chains), batch),
                       dim3(kL1Threads), 0, st, w1, p->b1, x, p->in_dim, p->hid, hbuf);
  else
    hipLaunchKernelGGL((chain_layer_kernel<0, W>), dim3(ceil_div(p->hid, 64), batch), dim3(64), 0,
                       st, w1, p->b1, x, p->in_dim, p->hid, hbuf);
  KH_LAUNCHED();
  return l2_typed<W>(p, hbuf, batch, scores, st, mm, tk);
}

// Layer 2 from the layer-1 outputs in hbuf (see predict_typed).
template <typename W>
static int l2_typed(const kh_predictor* p, const float* hbuf, int64_t batch, float* scores,
                    hipStream_t st, uint32_t* mm, TopkReq* tk) {
  const W* w2 = static_cast<const W*>(p->w2b);
  if (p->hid <= kMaxL2Hid && tk && p->out_dim <= kL2Threads) {
    hipLaunchKernelGGL((pred_l2_kernel<W, true>), dim3(1, batch), dim3(kL2Threads), 0, st, w2,
                       p->b2, hbuf, p->hid, p->out_dim, scores, nullptr, tk->k, tk->order,
                       tk->ids);
    tk->done = true;
  } else if (std::is_same<W, uint16_t>::value && batch > 1 && p->hid <= kMaxL2Hid && p->hid % 8 == 0)
    hipLaunchKernelGGL(pred_l2_rows_kernel, dim3(l2_blocks(p), ceil_div(batch, kL2Rows)), dim3(kL2RowThreads), 0,
                       st, reinterpret_cast<const uint16_t*>(w2), p->b2, hbuf, p->hid, p->out_dim,
                       static_cast<int>(batch), scores, mm);
  else if (p->hid <= kMaxL2Hid)
    hipLaunchKernelGGL(pred_l2_kernel<W>, dim3(l2_blocks(p), batch), dim3(kL2Threads), 0, st,
                       w2, p->b2, hbuf, p->hid, p->out_dim, scores, mm);
  else
    hipLaunchKernelGGL((chain_layer_kernel<1, W>), dim3(ceil_div(p->out_dim, 64), batch), dim3(64),
                       0, st, w2, p->b2, hbuf, p->hid, p->out_dim, scores);
  KH_LAUNCHED();
  return KH_OK;
}

// The score key bounds are usable by the top-k kernel when layer 2's fast
// kernel writes them and they fit one slot per top-k thread.
static bool bounds_ok(const kh_predictor* p) {
  return p->hid <= kMaxL2Hid && l2_blocks(p) <= kTopkThreads;
}

static int predict_into(const kh_predictor* p, const float* x, int64_t batch, float* scores,
                        const PredBufs& b, hipStream_t st, const NormIn& nrm = NormIn{},
                        bool bounds = false, TopkReq* tk = nullptr) {
  uint32_t* mm = (bounds && bounds_ok(p)) ? b.mm : nullptr;
  return p->bf16 ? predict_typed<uint16_t>(p, x, batch, scores, b.hbuf, st, nrm, mm, tk)
                 : predict_typed<float>(p, x, batch, scores, b.hbuf, st, nrm, mm, tk);
}

extern "C" int kh_predictor_predict(const kh_predictor* p, const float* x_dev, int64_t batch,
                                    float* scores_dev, void* stream) {
  KH_CHECK_ARG(p && x_dev && scores_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 65535, "bad batch");
  if (batch == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  PredBufs b;
  int rc = pred_bufs(p, st, batch, 0, false, &b);
  if (rc != KH_OK) return rc;
  return predict_into(p, x_dev, batch, scores_dev, b, st);
}

// mm: per-block key bounds from layer 2, nmm slots per row (or nullptr: the
// kernel finds the bounds from the scores).  sortbuf: [batch][min(k, n)]
// staging for score order (unused for ascending order).
static int topk_launch(const float* scores, int64_t batch, int n, int k, int order, int32_t* ids,
                       hipStream_t st, uint64_t* sortbuf, const uint32_t* mm = nullptr,
                       int nmm = 0, uint8_t* marks = nullptr) {
  const int kk = std::min(k, n);
  if (kk <= 0 || batch == 0) return KH_OK;
  KH_CHECK_ARG(n <= kTopkRegMax, "top-k supports n <= %d scores per row (got %d)", kTopkRegMax, n);
  static_assert(kTopkRegMax < 65536, "packed compaction counts");
  int rc = set_kernel_attrs();
  if (rc != KH_OK) return rc;
  size_t lds = n <= kTopkStage ? sizeof(uint32_t) * ((n + 3) & ~3) : 0;  // staged scores
  if (order == KH_ORDER_SCORE) {
    KH_CHECK_ARG(kk <= 4096, "score-ordered top-k supports k <= 4096 (got %d)", kk);
    KH_CHECK_ARG(sortbuf != nullptr, "score-ordered top-k needs a staging buffer");
    int P = 1;
    while (P < kk) P <<= 1;
    lds = std::max(lds, sizeof(uint64_t) * P);
  }
  // keys per thread: the smallest instantiation that holds the row
  const dim3 g(static_cast<unsigned>(batch)), t(kTopkThreads);
  if (n <= kTopkThreads * 6)  // 1.1B intermediate size 5632
    hipLaunchKernelGGL(topk_kernel<6>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else if (n <= kTopkThreads * 8)
    hipLaunchKernelGGL(topk_kernel<8>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else if (n <= kTopkThreads * 11)  // 7B intermediate size 11008: no idle twelfth key per thread
    hipLaunchKernelGGL(topk_kernel<11>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else if (n <= kTopkThreads * 12)
    hipLaunchKernelGGL(topk_kernel<12>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else if (n <= kTopkThreads * 16)
    hipLaunchKernelGGL(topk_kernel<16>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else if (n <= kTopkThreads * 32)
    hipLaunchKernelGGL(topk_kernel<32>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  else
    hipLaunchKernelGGL(topk_kernel<64>, g, t, lds, st, scores, n, k, order, ids, sortbuf, mm, nmm, marks);
  KH_LAUNCHED();
  return KH_OK;
}

// select_top_k over buffers b (the handle's workspace, or the static scratch
// of the allocation-free entry point).
static int select_top_k_with(const kh_predictor* p, const float* x, int64_t batch, int k,
                             int order, int32_t* ids, const PredBufs& b, hipStream_t st) {
  TopkReq tk{k, order, ids};
  int rc = predict_into(p, x, batch, b.sbuf, b, st, NormIn{}, true, &tk);
  if (rc != KH_OK || tk.done) return rc;
  return topk_launch(b.sbuf, batch, p->out_dim, k, order, ids, st, b.sortbuf,
                     bounds_ok(p) ? b.mm : nullptr, l2_blocks(p));
}

extern "C" int kh_predictor_select_top_k(const kh_predictor* p, const float* x_dev, int64_t batch,
                                         int k, int order, int32_t* ids_dev, void* stream) {
  KH_CHECK_ARG(p && x_dev && ids_dev, "null argument");
  KH_CHECK_ARG(k >= 0 && batch >= 0 && batch <= 65535, "bad k/batch");
  KH_CHECK_ARG(order == KH_ORDER_SCORE || order == KH_ORDER_ASCENDING, "bad order");
  if (batch == 0 || k == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  const int kk = std::min(k, p->out_dim);
  PredBufs b;
  int rc = pred_bufs(p, st, batch, order == KH_ORDER_SCORE ? kk : 0, false, &b);
  if (rc != KH_OK) return rc;
  return select_top_k_with(p, x_dev, batch, k, order, ids_dev, b, st);
}

// ---------------------------------------------------------------- allocation-free variant
// kh_predictor_select_top_k_noalloc takes every buffer from this array (one
// copy per GPU, held until the process ends) instead of allocating.  Host code
// never uses the array's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, and is what the kernels receive.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device.
int scratch_ptr(uint8_t** out) {
  int dev = 0;
  KH_HIP(hipGetDevice(&dev));
  KH_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return KH_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<uint8_t*>(g_scratch_ptr[dev]);
  return KH_OK;
}

size_t round256(size_t b) { return (b + 255) & ~size_t(255); }
}  // namespace

extern "C" int kh_predictor_select_top_k_noalloc(const kh_predictor* p, const float* x_dev,
                                                 int64_t batch, int k, int order, int32_t* ids_dev,
                                                 void* stream) {
  KH_CHECK_ARG(p && x_dev && ids_dev, "null argument");
  KH_CHECK_ARG(k >= 0 && batch >= 0 && batch <= 65535, "bad k/batch");
  KH_CHECK_ARG(order == KH_ORDER_SCORE || order == KH_ORDER_ASCENDING, "bad order");
  if (batch == 0 || k == 0) return KH_OK;
  const int kk = std::min(k, p->out_dim);
  const size_t hb = round256(sizeof(float) * batch * p->hid);
  const size_t sb = round256(sizeof(float) * batch * p->out_dim);
  const size_t mb = round256(sizeof(uint32_t) * 2 * batch * l2_blocks(p));
  const size_t ob = order == KH_ORDER_SCORE ? round256(sort_bytes(batch, kk)) : 0;
  const size_t need = hb + sb + mb + ob;
  if (need > kNoAllocScratchBytes) {
    set_error("kh_predictor_select_top_k_noalloc: batch %lld needs %zu bytes of scratch, more than "
              "its %zu (use kh_predictor_select_top_k)",
              (long long)batch, need, kNoAllocScratchBytes);
    return KH_ERR_CAPACITY;
  }
  uint8_t* base = nullptr;
  int rc = scratch_ptr(&base);
  if (rc != KH_OK) return rc;
  PredBufs b;
  b.hbuf = reinterpret_cast<float*>(base);
  b.sbuf = reinterpret_cast<float*>(base + hb);
  b.mm = reinterpret_cast<uint32_t*>(base + hb + sb);
  b.sortbuf = ob ? reinterpret_cast<uint64_t*>(base + hb + sb + mb) : nullptr;
  return select_top_k_with(p, x_dev, batch, k, order, ids_dev, b, as_stream(stream));
}

extern "C" int kh_predictor_select_top_k_union(const kh_predictor* p, const float* x_dev,
                                               int64_t batch, int k, int32_t* ids_dev,
                                               int32_t* union_dev, int32_t* count_dev,
                                               void* stream) {
  KH_CHECK_ARG(p && x_dev && ids_dev && union_dev && count_dev, "null argument");
  KH_CHECK_ARG(k >= 0 && batch >= 0 && batch <= 65535, "bad k/batch");
  hipStream_t st = as_stream(stream);
  const int n = p->out_dim;
  if (batch == 0 || k == 0 || n <= 64 || n > 32768) {
    // nothing selected, rows selected inside layer 2, or rows beyond the
    // marks kernel: ids first, then the union from them
    int rc = kh_predictor_select_top_k(p, x_dev, batch, k, KH_ORDER_ASCENDING, ids_dev, stream);
    if (rc != KH_OK) return rc;
    return kh_union_active(ids_dev, batch, std::min(k, n), n, union_dev, count_dev, stream);
  }
  PredBufs b;
  int rc = pred_bufs(p, st, batch, 0, true, &b);
  if (rc != KH_OK) return rc;
  rc = predict_into(p, x_dev, batch, b.sbuf, b, st, NormIn{}, true, nullptr);
  if (rc != KH_OK) return rc;
  rc = topk_launch(b.sbuf, batch, n, k, KH_ORDER_ASCENDING, ids_dev, st, nullptr,
                   bounds_ok(p) ? b.mm : nullptr, l2_blocks(p), b.marks);
  if (rc != KH_OK) return rc;
  hipLaunchKernelGGL(marks_union_kernel, dim3(1), dim3(1024), 0, st,
                     reinterpret_cast<uint32_t*>(b.marks), n, union_dev, count_dev);
  KH_LAUNCHED();
  return KH_OK;
}

// Score-order staging of handle-less top-k calls, one buffer per stream.
static StreamWs& topk_ws() {
  static StreamWs* w = new StreamWs();  // lives until the process ends
  return *w;
}

extern "C" int kh_topk_select(const float* scores_dev, int64_t batch, int n, int k, int order,
                              int32_t* ids_dev, void* stream) {
  KH_CHECK_ARG(scores_dev && ids_dev, "null argument");
  KH_CHECK_ARG(n >= 0 && k >= 0 && batch >= 0 && batch <= 65535, "bad shape");
  KH_CHECK_ARG(order == KH_ORDER_SCORE || order == KH_ORDER_ASCENDING, "bad order");
  hipStream_t st = as_stream(stream);
  uint64_t* sortbuf = nullptr;
  const int kk = std::min(k, n);
  if (order == KH_ORDER_SCORE && kk > 0 && batch > 0) {
    sortbuf = static_cast<uint64_t*>(topk_ws().get(st)->get(0, sort_bytes(batch, kk)));
    if (!sortbuf) return KH_ERR_ALLOC;
  }
  return topk_launch(scores_dev, batch, n, k, order, ids_dev, st, sortbuf);
}

extern "C" int kh_union_active(const int32_t* ids_dev, int64_t batch, int k, int n,
                               int32_t* union_dev, int32_t* count_dev, void* stream) {
  KH_CHECK_ARG(ids_dev && union_dev && count_dev, "null argument");
  KH_CHECK_ARG(n > 0 && n <= 32 * 12288 && k >= 0 && batch >= 0, "bad shape (n <= 393216)");
  KH_CHECK_ARG(batch * (int64_t)k < (int64_t)1 << 31, "batch * k too large");
  const size_t lds = n <= kUnionFlagMax ? sizeof(uint32_t) * ((n + 3) / 4)
                                        : sizeof(uint32_t) * ((n + 31) / 32);
  int rc = set_kernel_attrs();
  if (rc != KH_OK) return rc;
  hipLaunchKernelGGL(union_kernel, dim3(1), dim3(1024), lds, as_stream(stream), ids_dev,
                     static_cast<int>(batch), k, n, union_dev, count_dev);
  KH_LAUNCHED();
  return KH_OK;
}

namespace kh {
int predictor_in_dim(const kh_predictor* p) { return p->in_dim; }
int predictor_out_dim(const kh_predictor* p) { return p->out_dim; }
// Predictor scores of RmsNorm(hidden) (norm applied inside layer 1) and the
// top-k ids in ascending order, batch 1.
int predictor_topk_normed(const kh_predictor* p, const float* hidden, int k, int32_t* ids,
                          const NormIn& nrm, hipStream_t st) {
  PredBufs b;
  int rc = pred_bufs(p, st, 1, 0, false, &b);
  if (rc != KH_OK) return rc;
  TopkReq tk{k, KH_ORDER_ASCENDING, ids};
  rc = predict_into(p, hidden, 1, b.sbuf, b, st, nrm, true, &tk);
  if (rc != KH_OK || tk.done) return rc;
  return topk_launch(b.sbuf, 1, p->out_dim, k, KH_ORDER_ASCENDING, ids, st, nullptr,
                     bounds_ok(p) ? b.mm : nullptr, l2_blocks(p));
}

int predictor_scores_normed(const kh_predictor* p, const float* hidden, const NormIn& nrm,
                            hipStream_t st, PredScores* out) {
  if (!bounds_ok(p) || p->out_dim <= kL2Threads) return KH_ERR_UNSUPPORTED;
  PredBufs b;
  int rc = pred_bufs(p, st, 1, 0, false, &b);
  if (rc != KH_OK) return rc;
  rc = predict_into(p, hidden, 1, b.sbuf, b, st, nrm, true, nullptr);
  if (rc != KH_OK) return rc;
  out->scores = b.sbuf;
  out->mm = b.mm;
  out->n = p->out_dim;
  out->nmm = l2_blocks(p);
  return KH_OK;
}

int predictor_l1_view(const kh_predictor* p, hipStream_t st, PredL1View* v, int64_t batch) {
  PredBufs b;
  int rc = pred_bufs(p, st, batch, 0, false, &b);
  if (rc != KH_OK) return rc;
  rc = set_kernel_attrs();
  if (rc != KH_OK) return rc;
  v->w1b = p->w1b;
  v->b1 = p->b1;
  v->w2b = p->w2b;
  v->b2 = p->b2;
  v->in_dim = p->in_dim;
  v->hid = p->hid;
  v->out_dim = p->out_dim;
  v->bf16 = p->bf16;
  v->hbuf = b.hbuf;
  return KH_OK;
}

// Layer 1 of RmsNorm(hidden[b]) for rows b < batch (the norm inside the
// layer-1 blocks, each row's scale written to nrm.inv[b] and the normalised
// rows to xn[batch][in_dim]) into the per-stream layer-1 buffer that v->hbuf
// then names ([batch][hid]).
int predictor_l1_normed(const kh_predictor* p, const float* hidden, int64_t batch, const NormIn& nrm,
                        float* xn, hipStream_t st, PredL1View* v) {
  if (!nrm.w || !nrm.inv || p->in_dim > kL1LdsIn || p->in_dim % 4 != 0) {
    set_error("the fused RmsNorm needs predictor inputs that are a multiple of 4 and at most %d", kL1LdsIn);
    return KH_ERR_UNSUPPORTED;
  }
  PredBufs b;
  int rc = pred_bufs(p, st, batch, 0, false, &b);
  if (rc != KH_OK) return rc;
  rc = set_kernel_attrs();
  if (rc != KH_OK) return rc;
  const dim3 g(ceil_div(p->hid, kL1Chains), static_cast<unsigned>(batch));
  if (p->bf16)
    hipLaunchKernelGGL(pred_l1_lds_kernel<uint16_t>, g, dim3(kL1LdsThreads), kL1LdsBytes, st,
                       static_cast<const uint16_t*>(p->w1b), p->b1, hidden, p->in_dim, p->hid, b.hbuf, nrm.w,
                       nrm.inv, nrm.eps, xn);
  else
    hipLaunchKernelGGL(pred_l1_lds_kernel<float>, g, dim3(kL1LdsThreads), kL1LdsBytes, st,
                       static_cast<const float*>(p->w1b), p->b1, hidden, p->in_dim, p->hid, b.hbuf, nrm.w,
                       nrm.inv, nrm.eps, xn);
  KH_LAUNCHED();
  v->w1b = p->w1b;
  v->b1 = p->b1;
  v->w2b = p->w2b;
  v->b2 = p->b2;
  v->in_dim = p->in_dim;
  v->hid = p->hid;
  v->out_dim = p->out_dim;
  v->bf16 = p->bf16;
  v->hbuf = b.hbuf;
  return KH_OK;
}

// Scores of rows 0..batch-1 of x (normalised rows) and their top k, ids
// ascending into ids[batch][k], with the selected neurons' byte marks set in
// the per-stream marks buffer *marks (zero between calls: the caller's
// consumer clears them), as kh_predictor_select_top_k_union before its union
// kernel.  Needs 64 < out_dim <= 32768.
int predictor_select_marks(const kh_predictor* p, const float* x, int64_t batch, int k, int32_t* ids,
                           hipStream_t st, uint8_t** marks) {
  const int n = p->out_dim;
  if (n <= 64 || n > 32768) return KH_ERR_UNSUPPORTED;
  PredBufs b;
  int rc = pred_bufs(p, st, batch, 0, true, &b);
  if (rc != KH_OK) return rc;
  rc = predict_into(p, x, batch, b.sbuf, b, st, NormIn{}, true, nullptr);
  if (rc != KH_OK) return rc;
  rc = topk_launch(b.sbuf, batch, n, k, KH_ORDER_ASCENDING, ids, st, nullptr, bounds_ok(p) ? b.mm : nullptr,
                   l2_blocks(p), b.marks);
  if (rc != KH_OK) return rc;
  *marks = b.marks;
  return KH_OK;
}

int predictor_l2_topk_from_h(const kh_predictor* p, int k, int32_t* ids, hipStream_t st) {
  PredBufs b;
  int rc = pred_bufs(p, st, 1, 0, false, &b);
  if (rc != KH_OK) return rc;
  TopkReq tk{k, KH_ORDER_ASCENDING, ids};
  uint32_t* mm = bounds_ok(p) ? b.mm : nullptr;
  rc = p->bf16 ? l2_typed<uint16_t>(p, b.hbuf, 1, b.sbuf, st, mm, &tk)
               : l2_typed<float>(p, b.hbuf, 1, b.sbuf, st, mm, &tk);
  if (rc != KH_OK || tk.done) return rc;
  return topk_launch(b.sbuf, 1, p->out_dim, k, KH_ORDER_ASCENDING, ids, st, nullptr, mm, l2_blocks(p));
}
}  // namespace kh
