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
// (4 passes of 8 bits with LDS histograms) that finds the exact k-th key T;
// the selected set is {key > T} plus the lowest-index entries with key == T,
// which is exactly what the reference's stable descending sort keeps.
#include <cstring>
#include <vector>

#include "common.hpp"

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

// Layer 1 (long chains).  One block = one consumer wave (wave 0, 64 chains =
// 64 hidden units of one input row) + kProd producer waves.  The producers
// prefetch the blocked weights [ceil(n_in/8)][hid][8] kPre stages ahead in
// registers, form the rounded products w*x for a stage of 64 steps and write
// them to a two-stage LDS ring laid out [stage][step/4][chain][4]; the consumer
// adds them in step order with one ds_read_b128 per four steps.  Output
// h[b][i] = max(sum + b1[i], 0).
constexpr int kProd = 4;          // producer waves
constexpr int kStage = 64;        // steps per stage (8 blocks of 8)
constexpr int kPre = 16;          // stages of weights in flight per producer
constexpr int kL1Threads = 64 * (1 + kProd);
constexpr int kMaxL1In = 8192;    // x row staged in LDS

template <typename W>
__global__ __launch_bounds__(kL1Threads) void pred_l1_kernel(
    const W* __restrict__ Wb, const float* __restrict__ bias, const float* __restrict__ x,
    int n_in, int hid, float* __restrict__ h) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  __shared__ __align__(16) float xs[kMaxL1In];
  __shared__ float4 ring[2][kStage / 4][64];
  const int b = blockIdx.y;
  const int c0 = blockIdx.x * 64;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int chain = c0 + lane;
  const bool chain_ok = chain < hid;
  const int nblk = (n_in + 7) >> 3;               // 8-step blocks
  const int nst = (n_in + kStage - 1) / kStage;   // stages
  if ((n_in & 3) == 0)
    stage_f4(reinterpret_cast<float4*>(xs), reinterpret_cast<const float4*>(x + (size_t)b * n_in),
             n_in >> 2);
  else
    for (int j = threadIdx.x; j < n_in; j += blockDim.x) xs[j] = x[(size_t)b * n_in + j];
  const V* __restrict__ wv = reinterpret_cast<const V*>(Wb);
  // producer wave pw owns blocks pw and pw + kProd of every stage
  const int pw = wave - 1;
  V pre[kPre][2];
  // Unconditional (clamped) loads: out-of-range blocks and chains are never
  // consumed, and branch-free loads let the compiler count them precisely
  // (a conditional load makes it wait for every outstanding load).
  const int chain_c = chain_ok ? chain : hid - 1;
  auto load_stage = [&](int st, V (&r)[2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jb = min(st * (kStage / 8) + pw + kProd * q, nblk - 1);
      r[q] = wv[(size_t)jb * hid + chain_c];
    }
  };
  auto make_stage = [&](int st, const V (&r)[2]) {
    float4(*dst)[64] = ring[st & 1];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jl = pw + kProd * q;  // block within the stage
      const int j0 = (st * (kStage / 8) + jl) * 8;
      float w[8], p[8];
      B8::widen(r[q], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __fmul_rn(w[e], xs[min(j0 + e, kMaxL1In - 1)]);
      dst[2 * jl][lane] = make_float4(p[0], p[1], p[2], p[3]);
      dst[2 * jl + 1][lane] = make_float4(p[4], p[5], p[6], p[7]);
    }
  };
  __syncthreads();  // xs ready (nothing else in flight yet)
  if (wave > 0) {
#pragma unroll
    for (int d = 0; d < kPre; ++d) load_stage(d, pre[d]);
    make_stage(0, pre[0]);
    load_stage(kPre, pre[0]);
  }
  lds_barrier();
  // Producers and the consumer run separate loops with the same number of
  // barriers (one per stage, nst rounded up to a multiple of kPre).  The
  // producer body is branch-free -- it also forms (unused) stages past the end
  // -- so the compiler can wait for exactly the stage it needs rather than
  // for every outstanding prefetch.
  const int nst_pad = (nst + kPre - 1) / kPre * kPre;
  float s = -0.0f;
  if (wave > 0) {
    for (int st0 = 0; st0 < nst_pad; st0 += kPre) {
#pragma unroll
      for (int d = 0; d < kPre; ++d) {
        const int st = st0 + d;
        make_stage(st + 1, pre[(d + 1) % kPre]);
        load_stage(st + 1 + kPre, pre[(d + 1) % kPre]);
        lds_barrier();
      }
    }
  } else {
    for (int st0 = 0; st0 < nst_pad; st0 += kPre) {
#pragma unroll
      for (int d = 0; d < kPre; ++d) {
        const int st = st0 + d;
        const float4(*src)[64] = ring[st & 1];
        const int steps = min(kStage, n_in - st * kStage);
        if (steps == kStage) {
#pragma unroll
          for (int q = 0; q < kStage / 4; ++q) {
            const float4 v = src[q][lane];
            s = __fadd_rn(s, v.x);
            s = __fadd_rn(s, v.y);
            s = __fadd_rn(s, v.z);
            s = __fadd_rn(s, v.w);
          }
        } else if (steps > 0) {
          for (int q = 0; q < kStage / 4; ++q) {
            if (4 * q >= steps) break;
            const float4 v = src[q][lane];
            const float e[4] = {v.x, v.y, v.z, v.w};
            for (int u = 0; u < 4 && 4 * q + u < steps; ++u) s = __fadd_rn(s, e[u]);
          }
        }
        lds_barrier();
      }
    }
  }
  if (wave == 0 && chain_ok) h[(size_t)b * hid + chain] = fmaxf(__fadd_rn(s, bias[chain]), 0.0f);
}

// Layer 2 (short chains): one lane per output, the whole weight row in
// registers (n_hid <= 256), the hidden vector in LDS.  Scores = sigmoid.
constexpr int kMaxL2Hid = 256;

template <typename W>
__global__ __launch_bounds__(256) void pred_l2_kernel(const W* __restrict__ Wb,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ hin, int n_hid,
                                                      int n_out, float* __restrict__ out) {
  using B8 = Blk8<W>;
  using V = typename B8::V;
  __shared__ float hs[kMaxL2Hid];
  __shared__ uint64_t tab[32];
  const int b = blockIdx.y;
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  for (int i = threadIdx.x; i < n_hid; i += blockDim.x) hs[i] = hin[(size_t)b * n_hid + i];
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  const bool ok = o < n_out;
  const int oc = ok ? o : 0;
  const int nblk = (n_hid + 7) >> 3;
  const V* __restrict__ wv = reinterpret_cast<const V*>(Wb);
  V w[kMaxL2Hid / 8];
#pragma unroll
  for (int jb = 0; jb < kMaxL2Hid / 8; ++jb)
    w[jb] = jb < nblk ? wv[(size_t)jb * n_out + oc] : B8::zero();
  __syncthreads();
  float s = -0.0f;
#pragma unroll
  for (int jb = 0; jb < kMaxL2Hid / 8; ++jb) {
    if (jb < nblk) {
      float wf[8];
      B8::widen(w[jb], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (jb * 8 + e < n_hid) s = __fadd_rn(s, __fmul_rn(wf[e], hs[jb * 8 + e]));
    }
  }
  if (ok) out[(size_t)b * n_out + o] = sigmoid_ref_t(__fadd_rn(s, bias[o]), tab);
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
constexpr int kTopkLdsKeys = 12288;  // keys kept in LDS when n fits

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores,
                                                            int n, int k, int order,
                                                            int32_t* __restrict__ out,
                                                            uint64_t* __restrict__ sortbuf) {
  extern __shared__ __align__(16) uint32_t lkeys[];
  __shared__ unsigned hist[256];
  __shared__ int wgt[kTopkThreads / 64], weq[kTopkThreads / 64];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int s_kk, s_hi;
  const int b = blockIdx.x;
  const float* sc = scores + (size_t)b * n;
  const bool in_lds = n <= kTopkLdsKeys;
  const int kk0 = min(k, n);
  int32_t* ob = out + (size_t)b * kk0;
  if (kk0 <= 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (in_lds) {
    if ((n & 3) == 0 && ((reinterpret_cast<uintptr_t>(sc) & 15) == 0))
      stage_f4(reinterpret_cast<float4*>(lkeys), reinterpret_cast<const float4*>(sc), n >> 2);
    else
      for (int i = threadIdx.x; i < n; i += blockDim.x) lkeys[i] = __float_as_uint(sc[i]);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) lkeys[i] = f32_key(__uint_as_float(lkeys[i]));
  }
  // Highest bit where the keys differ: bits above it are common to every key,
  // so the radix passes start there (scores cluster, and a pass over shared
  // high bits would put every key in one or two bins).
  uint32_t kmax = 0u, kmin = 0xffffffffu;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const uint32_t key = in_lds ? lkeys[i] : f32_key(sc[i]);
    kmax = max(kmax, key);
    kmin = min(kmin, key);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, 64));
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o, 64));
  }
  if (lane == 0) {
    wgt[wave] = (int)kmax;
    weq[wave] = (int)kmin;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t mx = 0u, mn = 0xffffffffu;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      mx = max(mx, (uint32_t)wgt[w]);
      mn = min(mn, (uint32_t)weq[w]);
    }
    const uint32_t diff = mx ^ mn;
    const int hb = diff ? 31 - __clz(diff) : -1;
    const uint32_t common = hb >= 31 ? 0u : ~((2u << hb) - 1u);
    s_mask = hb < 0 ? 0xffffffffu : common;
    s_prefix = mx & s_mask;
    s_kk = kk0;
    s_hi = hb;
  }
  __syncthreads();
  for (int hi = s_hi; hi >= 0;) {
    const int lo = max(0, hi - 7);
    const int shift = lo;
    const uint32_t binmask = (2u << (hi - lo)) - 1u;
    for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const uint32_t key = in_lds ? lkeys[i] : f32_key(sc[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & binmask], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l owns bins 4l..4l+3; suffix sums from the top bin down
      const int l = threadIdx.x;
      const int h0 = hist[4 * l], h1 = hist[4 * l + 1], h2 = hist[4 * l + 2], h3 = hist[4 * l + 3];
      const int local = h0 + h1 + h2 + h3;
      int suf = local;  // inclusive suffix over lanes >= l
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_down(suf, o, 64);
        if (l + o < 64) suf += y;
      }
      const int above = suf - local;  // count in bins of lanes > l
      const int kk = s_kk;
      if (above < kk && kk <= suf) {
        int cum = above, sel = 4 * l;
        const int hs[4] = {h0, h1, h2, h3};
        for (int q = 3; q >= 0; --q) {
          if (cum + hs[q] >= kk) {
            sel = 4 * l + q;
            break;
          }
          cum += hs[q];
        }
        s_kk = kk - cum;
        s_prefix = prefix | ((uint32_t)sel << shift);
        s_mask = mask | (binmask << shift);
      }
    }
    __syncthreads();
    hi = lo - 1;
  }
  const uint32_t T = s_prefix;
  const int ties = s_kk;  // entries equal to T to keep, lowest index first
  // Compaction in ascending index order: wave w owns the contiguous segment
  // [w*seg, (w+1)*seg); counts first, then ballot prefix sums inside waves.
  const int nw = blockDim.x >> 6;
  const int seg = ((n + nw - 1) / nw + 63) & ~63;
  const int s0 = min(n, wave * seg), s1 = min(n, s0 + seg);
  int cgt = 0, ceq = 0;
  for (int i0 = s0; i0 < s1; i0 += 64) {
    const int i = i0 + lane;
    const uint32_t key = i < s1 ? (in_lds ? lkeys[i] : f32_key(sc[i])) : 0u;
    cgt += __popcll(__ballot(i < s1 && key > T));
    ceq += __popcll(__ballot(i < s1 && key == T));
  }
  if (lane == 0) {
    wgt[wave] = cgt;
    weq[wave] = ceq;
  }
  __syncthreads();
  int gt_before = 0, eq_before = 0;
  for (int w = 0; w < wave; ++w) {
    gt_before += wgt[w];
    eq_before += weq[w];
  }
  int pos_base = gt_before + min(eq_before, ties);
  int eq_run = eq_before;
  for (int i0 = s0; i0 < s1; i0 += 64) {
    const int i = i0 + lane;
    const uint32_t key = i < s1 ? (in_lds ? lkeys[i] : f32_key(sc[i])) : 0u;
    const bool eq = i < s1 && key == T;
    const bool gt = i < s1 && key > T;
    const uint64_t meq = __ballot(eq);
    const int eq_rank = eq_run + (int)__popcll(meq & ((1ull << lane) - 1ull));
    const bool sel = gt || (eq && eq_rank < ties);
    const uint64_t msel = __ballot(sel);
    const int pos = pos_base + (int)__popcll(msel & ((1ull << lane) - 1ull));
    if (sel) {
      if (order == KH_ORDER_ASCENDING) ob[pos] = i;
      else sortbuf[(size_t)b * kk0 + pos] = ((uint64_t)key << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
    }
    pos_base += (int)__popcll(msel);
    eq_run += (int)__popcll(meq);
  }
  if (order == KH_ORDER_ASCENDING) return;
  // Score order: bitonic sort (descending) of the selected (key, ~index) pairs.
  __syncthreads();
  uint64_t* sv = reinterpret_cast<uint64_t*>(lkeys);
  int P = 1;
  while (P < kk0) P <<= 1;
  for (int i = threadIdx.x; i < P; i += blockDim.x)
    sv[i] = i < kk0 ? sortbuf[(size_t)b * kk0 + i] : 0ull;
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
  for (int i = threadIdx.x; i < kk0; i += blockDim.x)
    ob[i] = (int32_t)(0xffffffffu - (uint32_t)(sv[i] & 0xffffffffu));
}

// ---------------------------------------------------------------- union
__global__ __launch_bounds__(1024) void union_kernel(const int32_t* __restrict__ ids, int batch,
                                                     int k, int n, int32_t* __restrict__ uni,
                                                     int32_t* __restrict__ count) {
  extern __shared__ uint32_t bits[];
  __shared__ int wsum[16];
  __shared__ int s_total;
  const int nw = (n + 31) >> 5;
  for (int i = threadIdx.x; i < nw; i += blockDim.x) bits[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < batch * k; i += blockDim.x) {
    const int v = ids[i];
    if (v >= 0 && v < n) atomicOr(&bits[v >> 5], 1u << (v & 31));
  }
  __syncthreads();
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

}  // namespace kh

using namespace kh;

struct kh_predictor {
  int in_dim = 0, hid = 0, out_dim = 0;
  bool bf16 = false;     // weights stored as BF16 bits (exact) or f32
  void* w1b = nullptr;   // [ceil(in/8)][hid][8]
  float* b1 = nullptr;
  void* w2b = nullptr;   // [ceil(hid/8)][out][8]
  float* b2 = nullptr;
  float* hbuf = nullptr;  // [batch_cap][hid]
  float* sbuf = nullptr;  // [batch_cap][out]
  int batch_cap = 0;
};

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
  dev_free(p->hbuf);
  dev_free(p->sbuf);
  delete p;
  return KH_OK;
}

static int ensure_batch(kh_predictor* p, int64_t batch) {
  if (batch <= p->batch_cap) return KH_OK;
  dev_free(p->hbuf);
  dev_free(p->sbuf);
  p->hbuf = static_cast<float*>(dev_alloc(sizeof(float) * batch * p->hid));
  p->sbuf = static_cast<float*>(dev_alloc(sizeof(float) * batch * p->out_dim));
  if (!p->hbuf || !p->sbuf) {
    p->batch_cap = 0;
    return KH_ERR_ALLOC;
  }
  p->batch_cap = static_cast<int>(batch);
  return KH_OK;
}

template <typename W>
static int predict_typed(kh_predictor* p, const float* x, int64_t batch, float* scores,
                         hipStream_t st) {
  const W* w1 = static_cast<const W*>(p->w1b);
  const W* w2 = static_cast<const W*>(p->w2b);
  if (p->in_dim <= kMaxL1In)
    hipLaunchKernelGGL(pred_l1_kernel<W>, dim3(ceil_div(p->hid, 64), batch), dim3(kL1Threads), 0,
                       st, w1, p->b1, x, p->in_dim, p->hid, p->hbuf);
  else
    hipLaunchKernelGGL((chain_layer_kernel<0, W>), dim3(ceil_div(p->hid, 64), batch), dim3(64), 0,
                       st, w1, p->b1, x, p->in_dim, p->hid, p->hbuf);
  KH_LAUNCHED();
  if (p->hid <= kMaxL2Hid)
    hipLaunchKernelGGL(pred_l2_kernel<W>, dim3(ceil_div(p->out_dim, 256), batch), dim3(256), 0, st,
                       w2, p->b2, p->hbuf, p->hid, p->out_dim, scores);
  else
    hipLaunchKernelGGL((chain_layer_kernel<1, W>), dim3(ceil_div(p->out_dim, 64), batch), dim3(64),
                       0, st, w2, p->b2, p->hbuf, p->hid, p->out_dim, scores);
  KH_LAUNCHED();
  return KH_OK;
}

static int predict_into(const kh_predictor* pc, const float* x, int64_t batch, float* scores,
                        hipStream_t st) {
  auto* p = const_cast<kh_predictor*>(pc);
  int rc = ensure_batch(p, batch);
  if (rc != KH_OK) return rc;
  return p->bf16 ? predict_typed<uint16_t>(p, x, batch, scores, st)
                 : predict_typed<float>(p, x, batch, scores, st);
}

extern "C" int kh_predictor_predict(const kh_predictor* p, const float* x_dev, int64_t batch,
                                    float* scores_dev, void* stream) {
  KH_CHECK_ARG(p && x_dev && scores_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 65535, "bad batch");
  if (batch == 0) return KH_OK;
  return predict_into(p, x_dev, batch, scores_dev, as_stream(stream));
}

static int topk_launch(const float* scores, int64_t batch, int n, int k, int order, int32_t* ids,
                       hipStream_t st) {
  const int kk = std::min(k, n);
  if (kk <= 0 || batch == 0) return KH_OK;
  uint64_t* sortbuf = nullptr;
  size_t lds = n <= kTopkLdsKeys ? sizeof(uint32_t) * n : 0;
  if (order == KH_ORDER_SCORE) {
    KH_CHECK_ARG(kk <= 4096, "score-ordered top-k supports k <= 4096 (got %d)", kk);
    int P = 1;
    while (P < kk) P <<= 1;
    lds = std::max(lds, sizeof(uint64_t) * P);
    static thread_local uint64_t* buf = nullptr;
    static thread_local size_t cap = 0;
    const size_t need = sizeof(uint64_t) * batch * kk;
    if (need > cap) {
      dev_free(buf);
      buf = static_cast<uint64_t*>(dev_alloc(need));
      cap = buf ? need : 0;
      if (!buf) return KH_ERR_ALLOC;
    }
    sortbuf = buf;
  }
  hipLaunchKernelGGL(topk_kernel, dim3(batch), dim3(kTopkThreads), lds, st, scores, n, k, order,
                     ids, sortbuf);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_predictor_select_top_k(const kh_predictor* p, const float* x_dev, int64_t batch,
                                         int k, int order, int32_t* ids_dev, void* stream) {
  KH_CHECK_ARG(p && x_dev && ids_dev, "null argument");
  KH_CHECK_ARG(k >= 0 && batch >= 0 && batch <= 65535, "bad k/batch");
  KH_CHECK_ARG(order == KH_ORDER_SCORE || order == KH_ORDER_ASCENDING, "bad order");
  if (batch == 0 || k == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  auto* pm = const_cast<kh_predictor*>(p);
  int rc = ensure_batch(pm, batch);
  if (rc != KH_OK) return rc;
  rc = predict_into(p, x_dev, batch, pm->sbuf, st);
  if (rc != KH_OK) return rc;
  return topk_launch(pm->sbuf, batch, p->out_dim, k, order, ids_dev, st);
}

extern "C" int kh_topk_select(const float* scores_dev, int64_t batch, int n, int k, int order,
                              int32_t* ids_dev, void* stream) {
  KH_CHECK_ARG(scores_dev && ids_dev, "null argument");
  KH_CHECK_ARG(n >= 0 && k >= 0 && batch >= 0 && batch <= 65535, "bad shape");
  KH_CHECK_ARG(order == KH_ORDER_SCORE || order == KH_ORDER_ASCENDING, "bad order");
  return topk_launch(scores_dev, batch, n, k, order, ids_dev, as_stream(stream));
}

extern "C" int kh_union_active(const int32_t* ids_dev, int64_t batch, int k, int n,
                               int32_t* union_dev, int32_t* count_dev, void* stream) {
  KH_CHECK_ARG(ids_dev && union_dev && count_dev, "null argument");
  KH_CHECK_ARG(n > 0 && n <= 32 * 12288 && k >= 0 && batch >= 0, "bad shape (n <= 393216)");
  const size_t lds = sizeof(uint32_t) * ((n + 31) / 32);
  hipLaunchKernelGGL(union_kernel, dim3(1), dim3(1024), lds, as_stream(stream), ids_dev,
                     static_cast<int>(batch), k, n, union_dev, count_dev);
  KH_LAUNCHED();
  return KH_OK;
}
