// slide_train.hip -- SLIDE training on the GPU (gfx950).
//
// Replaces Layer::backward and Layer::rebuild_index
// (crates/klearu-core/src/network/layer.rs:124-233), Network::train_step /
// predict with compute_loss / compute_loss_gradient (network/net.rs:81-230),
// the SGD and Adam updates (optim/sgd.rs, optim/adam.rs), LshIndexTrait::rebuild
// (lsh/index.rs:302-307) and RebuildScheduler (lsh/maintenance.rs:20-98).
//
// The reference trains one example at a time and updates the weights after
// each one, so example e+1's forward pass reads the weights example e wrote:
// the examples of a batch are a chain.  Each example is a short sequence of
// kernels on one stream; the parallel work is inside an example (the
// neurons of a layer, the dimensions of a gradient, the weights of an update).
//
// Every f32 operation is the reference's, in its order: sums over the active
// list run sequentially in the list's order (the Jacobian and grad_input
// sums keep one lane per output, each lane a chain), the softmax denominator
// is the reference's sequential sum computed by exact_seq_sum, and no
// multiply-add is contracted (the library builds with -ffp-contract=off).
#include <cmath>
#include <cstring>
#include <vector>

#include "exact_sum.hpp"
#include "gather.hpp"
#include "slide_internal.hpp"

namespace kh {

constexpr int kTrThreads = 256;
constexpr int kTrMaxLabels = 1024;   // labels of one example
constexpr int kTrLdsNz = 8192;       // staged input nonzeros (beyond: read from global)
constexpr int kTrMaxNnz = 4096;      // stored entries of one sparse example
constexpr int kGTile = 1024;         // grad_input: (id, lg) pairs per LDS tile
constexpr int kSmCH = 64, kSmM = 128;  // exact softmax sum: 8192 terms per pass

struct OptArgs {
  int kind;       // KH_OPT_SGD / KH_OPT_ADAM
  float lr, momentum, b1, b2, eps, c1, c2;
  float* st_w1;   // SGD momentum / Adam first moments [n][dim]
  float* st_w2;   // Adam second moments [n][dim]
  float* st_b1;   // [n]
  float* st_b2;   // [n]
};

// f32::powi with a run-time exponent: the __powisf2 builtin of Rust's
// compiler-builtins (src/float/pow.rs), square-and-multiply from the low bit.
static float powi_f32(float a, int32_t b) {
  const bool recip = b < 0;
  uint32_t p = recip ? 0u - static_cast<uint32_t>(b) : static_cast<uint32_t>(b);
  float mul = 1.0f;
  for (;;) {
    if (p & 1u) mul = mul * a;
    p >>= 1;
    if (p == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / mul : mul;
}

static OptArgs opt_args(const kh_slide_layer* l, double lr, uint64_t step) {
  OptArgs o{};
  o.kind = l->opt;
  o.lr = static_cast<float>(lr);
  o.momentum = l->momentum;
  o.b1 = l->beta1;
  o.b2 = l->beta2;
  o.eps = l->eps;
  // Adam::update (adam.rs:38-47): step.max(1), `step as i32`
  const uint64_t s = step < 1 ? 1 : step;
  const int32_t si = static_cast<int32_t>(static_cast<uint32_t>(s));
  o.c1 = 1.0f - powi_f32(l->beta1, si);
  o.c2 = 1.0f - powi_f32(l->beta2, si);
  o.st_w1 = l->st_w1;
  o.st_w2 = l->st_w2;
  o.st_b1 = l->st_b1;
  o.st_b2 = l->st_b2;
  return o;
}

// activation_derivative (layer.rs:266-283)
__device__ __forceinline__ float act_deriv(float pre, float post, int act) {
  if (act == KH_ACT_RELU) return pre > 0.0f ? 1.0f : 0.0f;
  if (act == KH_ACT_SIGMOID) return post * (1.0f - post);
  if (act == KH_ACT_TANH) return 1.0f - post * post;
  return 1.0f;
}

// apply_activation (layer.rs:250-261)
__device__ __forceinline__ float act_apply(float z, int act) {
  if (act == KH_ACT_RELU) return fmaxf(z, 0.0f);
  if (act == KH_ACT_SIGMOID) return sigmoid_ref(z);
  if (act == KH_ACT_TANH) return tanhf(z);
  return z;
}

// One optimizer step of a parameter (Sgd::update, sgd.rs:28-56; Adam::update,
// adam.rs:50-76); s1/s2 its state slots.
__device__ __forceinline__ float opt_step(float w, float g, float* s1, float* s2, const OptArgs& o) {
  if (o.kind == KH_OPT_ADAM) {
    const float m = o.b1 * *s1 + (1.0f - o.b1) * g;
    const float gg = (1.0f - o.b2) * g;
    const float v = o.b2 * *s2 + gg * g;
    *s1 = m;
    *s2 = v;
    const float mh = m / o.c1;
    const float vh = v / o.c2;
    return w - (o.lr * mh) / (sqrtf(vh) + o.eps);
  }
  if (o.momentum > 0.0f) {
    const float v = o.momentum * *s1 - o.lr * g;
    *s1 = v;
    return w + v;
  }
  return w - o.lr * g;
}

// Nonzeros of a dense vector in ascending order, as a one-row CSR (xoff[0..1]).
// Dropping zero terms leaves every sequential sum over the vector unchanged
// (x + 0 == x; a zero partial sum only changes the sign of zero), so hashes
// and neuron sums over the list equal the reference's dense loops.
__global__ __launch_bounds__(1024) void tr_stage_nz_kernel(const float* __restrict__ x, int dim,
                                                           uint32_t* __restrict__ nzi,
                                                           float* __restrict__ nzv,
                                                           int64_t* __restrict__ xoff) {
  __shared__ int wsum[16];
  __shared__ int s_total;
  int base = 0;
  for (int c0 = 0; c0 < dim; c0 += blockDim.x) {
    const int d = c0 + threadIdx.x;
    const float v = d < dim ? x[d] : 0.0f;
    const int nz = v != 0.0f ? 1 : 0;
    const int pos = block_excl_scan(nz, wsum, &s_total) + base;
    if (nz) {
      nzi[pos] = static_cast<uint32_t>(d);
      nzv[pos] = v;
    }
    base += s_total;
  }
  if (threadIdx.x == 0) {
    xoff[0] = 0;
    xoff[1] = base;
  }
}

// Example::features.to_dense() (tensor/sparse.rs:77-83) of CSR row `row`:
// later stored entries overwrite earlier ones at the same index, so after a
// sort by (index, position) the last entry of each index is the value; the
// nonzero values in ascending index order become the row's staged list, and
// x_dense gets them (the previous row's entries are cleared first).  Entries
// with index >= dim are skipped (to_dense would panic on them).
__global__ __launch_bounds__(1024) void tr_stage_csr_kernel(
    const int64_t* __restrict__ xoff, const uint32_t* __restrict__ xidx,
    const float* __restrict__ xval, int64_t row, int dim, uint32_t* __restrict__ nzi,
    float* __restrict__ nzv, int64_t* __restrict__ nzoff, float* __restrict__ x_dense) {
  __shared__ uint64_t key[kTrMaxNnz];
  __shared__ int wsum[16];
  __shared__ int s_total;
  const int old = static_cast<int>(nzoff[1]);
  for (int i = threadIdx.x; i < old; i += blockDim.x) x_dense[nzi[i]] = 0.0f;
  const int64_t a = xoff[row];
  const int cnt = static_cast<int>(min<int64_t>(xoff[row + 1] - a, kTrMaxNnz));
  int P = 1;
  while (P < cnt) P <<= 1;
  for (int i = threadIdx.x; i < P; i += blockDim.x)
    key[i] = i < cnt ? (static_cast<uint64_t>(xidx[a + i]) << 32) | static_cast<uint32_t>(i) : ~0ull;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = key[i], y = key[ixj];
          if ((x > y) == ((i & k) == 0)) {
            key[i] = y;
            key[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  int base = 0;
  for (int c0 = 0; c0 < P; c0 += blockDim.x) {
    const int i = c0 + threadIdx.x;
    int keep = 0;
    uint32_t idx = 0;
    float v = 0.0f;
    if (i < cnt) {
      idx = static_cast<uint32_t>(key[i] >> 32);
      const bool last = i + 1 == cnt || static_cast<uint32_t>(key[i + 1] >> 32) != idx;
      v = xval[a + static_cast<uint32_t>(key[i])];
      keep = last && v != 0.0f && idx < static_cast<uint32_t>(dim);
    }
    const int pos = block_excl_scan(keep, wsum, &s_total) + base;
    if (keep) {
      nzi[pos] = idx;
      nzv[pos] = v;
      x_dense[idx] = v;
    }
    base += s_total;
  }
  if (threadIdx.x == 0) {
    nzoff[0] = 0;
    nzoff[1] = base;
  }
}

// Neuron::forward (neuron.rs:47-62) for one sample's active list: the
// sequential sum of w*x over the staged nonzeros, + bias; then the
// activation (not softmax) into post and the dense activation vector.
__global__ __launch_bounds__(kTrThreads) void tr_neuron_kernel(
    const float* __restrict__ W, const float* __restrict__ bias, int dim,
    const uint32_t* __restrict__ nzi, const float* __restrict__ nzv,
    const int64_t* __restrict__ xoff, const uint32_t* __restrict__ aids,
    const int32_t* __restrict__ alen, int cap, int act, float* __restrict__ pre,
    float* __restrict__ post, float* __restrict__ dense) {
  extern __shared__ unsigned char smem[];
  const int nnz = static_cast<int>(xoff[1]);
  const uint32_t* li = nzi;
  const float* lv = nzv;
  if (nnz <= kTrLdsNz) {
    uint32_t* si = reinterpret_cast<uint32_t*>(smem);
    float* sv = reinterpret_cast<float*>(smem + sizeof(uint32_t) * kTrLdsNz);
    for (int i = threadIdx.x; i < nnz; i += blockDim.x) {
      si[i] = nzi[i];
      sv[i] = nzv[i];
    }
    __syncthreads();
    li = si;
    lv = sv;
  }
  const int n = min(alen[0], cap);
  for (int a = blockIdx.x * blockDim.x + threadIdx.x; a < n; a += gridDim.x * blockDim.x) {
    const uint32_t id = aids[a];
    const float* w = W + static_cast<size_t>(id) * dim;
    float s = -0.0f;
    int e = 0;
    for (; e + 16 <= nnz; e += 16) {  // sixteen loads in flight, added in order
      float wv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) wv[q] = w[li[e + q]];
#pragma unroll
      for (int q = 0; q < 16; ++q) s = s + wv[q] * lv[e + q];
    }
    for (; e < nnz; ++e) s = s + w[li[e]] * lv[e];
    const float z = s + bias[id];
    pre[a] = z;
    if (act != KH_ACT_SOFTMAX) {
      const float r = act_apply(z, act);
      post[a] = r;
      if (dense) dense[id] = r;
    }
  }
}

// apply_softmax (layer.rs:286-308) over the active list in its order: max,
// exp(z - max) with glibc's expf, the sequential sum (exact_seq_sum, 8192
// terms a pass), then e / sum (or 1/n when the sum is not positive).  Lists
// of up to 8192 stay in registers (32 per thread, all loads in flight);
// longer ones go through `post` in passes.
__global__ __launch_bounds__(kTrThreads) void tr_softmax_kernel(const float* __restrict__ pre,
                                                                const uint32_t* __restrict__ aids,
                                                                const int32_t* __restrict__ alen,
                                                                int cap, float* __restrict__ post,
                                                                float* __restrict__ dense) {
  constexpr int kPass = kSmCH * kSmM;
  constexpr int kPer = kPass / kTrThreads;
  __shared__ EsLds<kSmCH, kSmM> es;
  __shared__ float red[kTrThreads / 64];
  __shared__ uint64_t s_tab[32];  // kExp2Tab: the exps' table lookups stay in LDS
  const int n = min(alen[0], cap);
  if (n <= 0) return;
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  float v[kPer];
  float mx = -INFINITY;
  if (n <= kPass) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) v[k] = pre[min(k * kTrThreads + static_cast<int>(threadIdx.x), n - 1)];
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      v[k] = k * kTrThreads + static_cast<int>(threadIdx.x) < n ? v[k] : -INFINITY;
#pragma unroll
    for (int k = 0; k < kPer; ++k) mx = fmaxf(mx, v[k]);
  } else {
    for (int a = threadIdx.x; a < n; a += blockDim.x) mx = fmaxf(mx, pre[a]);
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = red[0];
  for (int i = 1; i < kTrThreads / 64; ++i) mx = fmaxf(mx, red[i]);
  float s = -0.0f;
  if (n <= kPass) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int a = k * kTrThreads + threadIdx.x;
      v[k] = a < n ? expf_glibc_t(v[k] - mx, s_tab) : -0.0f;
      es.TP[es_slot<kSmCH, kSmM>(a)] = v[k];
    }
    __syncthreads();
    s = exact_seq_sum<kTrThreads / 64, kSmCH, kSmM>(n, s, es);
    const float u = 1.0f / static_cast<float>(n);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int a = k * kTrThreads + threadIdx.x;
      if (a < n) {
        const float r = s > 0.0f ? v[k] / s : u;
        post[a] = r;
        if (dense) dense[aids[a]] = r;
      }
    }
    return;
  }
  for (int a = threadIdx.x; a < n; a += blockDim.x) post[a] = expf_glibc_t(pre[a] - mx, s_tab);
  __syncthreads();
  for (int c0 = 0; c0 < n; c0 += kPass) {
    const int cnt = min(kPass, n - c0);
    for (int i = threadIdx.x; i < kPass; i += blockDim.x)
      es.TP[es_slot<kSmCH, kSmM>(i)] = i < cnt ? post[c0 + i] : -0.0f;
    __syncthreads();
    s = exact_seq_sum<kTrThreads / 64, kSmCH, kSmM>(cnt, s, es);
  }
  const float u = 1.0f / static_cast<float>(n);
  for (int a = threadIdx.x; a < n; a += blockDim.x) {
    const float r = s > 0.0f ? post[a] / s : u;
    post[a] = r;
    if (dense) dense[aids[a]] = r;
  }
}

// compute_loss and compute_loss_gradient (net.rs:180-230) of one example at
// the last layer's active entries: go[a] = activations[id] minus 1/|labels|
// per occurrence of id among the labels (all zero without labels); lg[a] =
// go * activation_derivative unless the layer is softmax (the Jacobian kernel
// follows).  One thread adds the example's loss to *loss_total, so the total
// is the reference's sequential f32 sum over the batch.
__global__ __launch_bounds__(kTrThreads) void tr_loss_grad_kernel(
    const float* __restrict__ pre, const float* __restrict__ post,
    const uint32_t* __restrict__ aids, const int32_t* __restrict__ alen, int cap, int act,
    const float* __restrict__ dense, const uint32_t* __restrict__ labels, int nl,
    float* __restrict__ go, float* __restrict__ lg, float* __restrict__ loss_total) {
  __shared__ int found[kTrMaxLabels];
  __shared__ uint32_t lab[kTrMaxLabels];
  const int n = min(alen[0], cap);
  for (int l = threadIdx.x; l < nl; l += blockDim.x) {
    found[l] = 0;
    lab[l] = labels[l];
  }
  __syncthreads();
  const float w = nl > 0 ? 1.0f / static_cast<float>(nl) : 0.0f;
  for (int a = threadIdx.x; a < n; a += blockDim.x) {
    const uint32_t id = aids[a];
    float g = nl > 0 ? post[a] : 0.0f;
    for (int l = 0; l < nl; ++l)
      if (lab[l] == id) {
        g = g - w;
        found[l] = 1;
      }
    go[a] = g;
    if (act != KH_ACT_SOFTMAX) lg[a] = g * act_deriv(pre[a], post[a], act);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float loss = 0.0f;
    if (nl > 0) {
      const float eps = 1e-7f;
      for (int l = 0; l < nl; ++l) {
        const float prob = found[l] ? fmaxf(dense[lab[l]], eps) : eps;
        loss = loss - logf(prob);
      }
      loss = loss / static_cast<float>(nl);
    }
    *loss_total = *loss_total + loss;
  }
}

// Sequential sums r + t[0] + t[1] + ... over quads of one chain's terms in LDS
// (quad q of this lane's chain at base[q * C]), with the LDS reads of the next
// eight quads issued before the adds of the current ones and pinned there
// (left to the scheduler, each read sinks to its first use and the chain waits
// out the LDS latency every four adds).
__device__ __forceinline__ float add_quads8(const float4* v, float r) {
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    r = r + v[b].x;
    r = r + v[b].y;
    r = r + v[b].z;
    r = r + v[b].w;
  }
  return r;
}

// NQ (a multiple of 8) quads, fully unrolled: every register index is a
// compile-time constant, so no value is copied.
template <int NQ, int C>
__device__ __forceinline__ float chain_add_static(const float4* base, float r) {
  static_assert(NQ % 8 == 0, "whole groups of quads");
  float4 v[16];
#pragma unroll
  for (int b = 0; b < 8; ++b) v[b] = base[b * C];
#pragma unroll
  for (int g = 0; g < NQ / 8; ++g) {
    if (g + 1 < NQ / 8) {
#pragma unroll
      for (int b = 0; b < 8; ++b) v[((g + 1) % 2) * 8 + b] = base[((g + 1) * 8 + b) * C];
    }
    __builtin_amdgcn_sched_barrier(0);
    r = add_quads8(&v[(g % 2) * 8], r);
  }
  return r;
}

// nq quads (a multiple of 8) as a loop over groups: the next group is read
// into a second set of registers while the current one is added, then copied
// over (measured faster than the copy-free pair loop for the long grad_input
// chains).
template <int C>
__device__ __forceinline__ float chain_add_quads(const float4* base, int nq, float r) {
  float4 v[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) v[b] = base[b * C];
  for (int g = 0; g < nq; g += 8) {
    const float4* nb = base + min(g + 8, nq - 8) * C;  // the last group re-reads itself
    float4 nv[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) nv[b] = nb[b * C];
    __builtin_amdgcn_sched_barrier(0);
    r = add_quads8(v, r);
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = nv[b];
  }
  return r;
}

// The softmax branch of Layer::backward (layer.rs:141-175): output i's local
// gradient is the sequential sum over j (from +0.0) of go_j*s_j*(1-s_j) when
// j == i, else go_j*(-s_i*s_j).  A block owns 64 outputs, one chain per lane
// of wave 0 (the consumer).  The terms depend on (i, j) through two rounded
// products each, so waves 1..3 form them into LDS one chunk of kJStep steps
// ahead of the consumer, whose only work per step is the dependent add (four
// steps per LDS read); wave 4 loads the (s, go) pairs two chunks ahead into a
// ring of three LDS slots, so no other wave waits on global memory.  Blocks
// loop over groups of 64 outputs.
constexpr int kJc = 64;                      // chains per block
constexpr int kJStep = 96;                   // steps per chunk
constexpr int kJProd = 3;                    // producer waves
constexpr int kJThreads = 64 * (2 + kJProd); // consumer, producers, loader
constexpr int kJBlocks = 256;                // grid (groups of 64 outputs are strided over it)
static_assert((kJStep / 4) % kJProd == 0 && (kJStep / 4) % 8 == 0 && kJStep <= 128, "chunk layout");

__device__ __forceinline__ float jac_off(float gj, float sj, float nsi) { return gj * (nsi * sj); }

__global__ __launch_bounds__(kJThreads) void tr_softmax_jacobian_kernel(
    const float* __restrict__ s, const float* __restrict__ go, const int32_t* __restrict__ alen,
    int cap, float* __restrict__ lg) {
  __shared__ float4 jb[2][kJStep / 4][kJc];    // two chunks of terms, [step/4][chain]
  __shared__ float4 ring[3][2][kJStep / 4];    // (s, go) of three chunks
  const int n = min(alen[0], cap);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nch = (n + kJStep - 1) / kJStep;
  const int p = wave - 1;                      // producer index (waves 1..kJProd)
  const bool prod = wave >= 1 && wave <= kJProd, loader = wave == kJProd + 1;
  // loader: chunk c's (s, go) into ring slot c % 3 (past n: the last pair,
  // formed but never added)
  auto load = [&](int c) {
    float* rs = reinterpret_cast<float*>(&ring[c % 3][0][0]);
    float* rg = reinterpret_cast<float*>(&ring[c % 3][1][0]);
    for (int k = lane; k < kJStep; k += 64) {
      const int j = min(c * kJStep + k, n - 1);
      rs[k] = s[j];
      rg[k] = go[j];
    }
  };
  for (int i0 = blockIdx.x * kJc; i0 < n; i0 += gridDim.x * kJc) {
    const int i = min(i0 + lane, n - 1);
    const float si = s[i], gi = go[i];
    const float nsi = -si;
    const float dterm = (gi * si) * (1.0f - si);  // the diagonal term, j == i
    // producer p forms quads p, p + kJProd, ... of chunk c
    auto produce = [&](int c) {
      const int jc = c * kJStep;
      const bool diag = jc < i0 + kJc && i0 < jc + kJStep;  // the chunk meets this block's diagonal
      constexpr int kQ = kJStep / 4 / kJProd;
      float4 sv[kQ], gv[kQ];
#pragma unroll
      for (int u = 0; u < kQ; ++u) {
        sv[u] = ring[c % 3][0][p + kJProd * u];
        gv[u] = ring[c % 3][1][p + kJProd * u];
      }
#pragma unroll
      for (int u = 0; u < kQ; ++u) {
        const int q = p + kJProd * u;
        float t0 = jac_off(gv[u].x, sv[u].x, nsi), t1 = jac_off(gv[u].y, sv[u].y, nsi);
        float t2 = jac_off(gv[u].z, sv[u].z, nsi), t3 = jac_off(gv[u].w, sv[u].w, nsi);
        if (diag) {
          const int d = i0 + lane - (jc + 4 * q);
          t0 = d == 0 ? dterm : t0;
          t1 = d == 1 ? dterm : t1;
          t2 = d == 2 ? dterm : t2;
          t3 = d == 3 ? dterm : t3;
        }
        jb[c & 1][q][lane] = make_float4(t0, t1, t2, t3);
      }
    };
    float r = 0.0f;
    lds_barrier();  // the previous group's last chunk is consumed
    if (loader) {
      load(0);
      if (nch > 1) load(1);
    }
    lds_barrier();
    if (prod) produce(0);
    lds_barrier();
    for (int c = 0; c < nch; ++c) {
      if (prod) {
        if (c + 1 < nch) produce(c + 1);
      } else if (loader) {
        if (c + 2 < nch) load(c + 2);
      } else if (wave == 0) {
        const int cnt = min(kJStep, n - c * kJStep);
        const float4(*src)[kJc] = jb[c & 1];
        if (cnt == kJStep) {
          r = chain_add_static<kJStep / 4, kJc>(&src[0][lane], r);
        } else {
          const float* sf = reinterpret_cast<const float*>(&src[0][0]);
          for (int j = 0; j < cnt; ++j) r = r + sf[((j >> 2) * kJc + lane) * 4 + (j & 3)];
        }
      }
      lds_barrier();
    }
    if (wave == 0 && i0 + lane < n) lg[i0 + lane] = r;
  }
}

// Local gradients of a layer from the gradient w.r.t. its output: go = the
// entry at the neuron's id (0 past the length); non-softmax layers get
// lg = go * activation_derivative(pre, activations[id]); softmax layers keep
// go for the Jacobian.
__global__ __launch_bounds__(kTrThreads) void tr_local_grad_kernel(
    const uint32_t* __restrict__ aids, const int32_t* __restrict__ alen, int cap,
    const float* __restrict__ pre, const float* __restrict__ dense, int act,
    const float* __restrict__ grad_out, int64_t grad_len, float* __restrict__ go,
    float* __restrict__ lg) {
  const int n = min(alen[0], cap);
  const int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= n) return;
  const uint32_t id = aids[a];
  const float g = static_cast<int64_t>(id) < grad_len ? grad_out[id] : 0.0f;
  if (act == KH_ACT_SOFTMAX)
    go[a] = g;
  else
    lg[a] = g * act_deriv(pre[a], dense[id], act);
}

// grad_input[j] = sum over the active list (in order, from +0.0) of
// lg[a] * w[id_a][j], with the weights before this example's update
// (layer.rs:203-207).  Each j is one chain of |A| dependent adds.  A block owns
// kGc columns, one chain per lane of wave 0 (the consumer); waves 1..7 gather
// the products for the next kGStep active rows into LDS (16 lanes read one
// 64-byte piece of a weight row) while the consumer adds the current ones,
// four per LDS read.
constexpr int kGc = 8;          // columns (chains) per block
constexpr int kGStep = 1024;    // active rows per chunk
constexpr int kGThreads = 512;

__global__ __launch_bounds__(kGThreads) void tr_grad_input_kernel(
    const float* __restrict__ W, int dim, const uint32_t* __restrict__ aids,
    const int32_t* __restrict__ alen, int cap, const float* __restrict__ lg,
    float* __restrict__ gi) {
  __shared__ float4 gb[2][kGStep / 4][kGc];   // two chunks of products, [row/4][column]
  constexpr int kProdThreads = kGThreads - 64;
  constexpr int kSlots = kProdThreads / kGc;  // rows gathered per producer pass
  constexpr int kPer = (kGStep + kSlots - 1) / kSlots;
  const int n = min(alen[0], cap);
  const int j0 = blockIdx.x * kGc;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nch = (n + kGStep - 1) / kGStep;
  const int pt = static_cast<int>(threadIdx.x) - 64;   // producer thread
  const int col = pt & (kGc - 1), slot = pt / kGc;
  const int jc = min(j0 + col, dim - 1);
  // A producer holds the weights and local gradients of the next chunk and
  // the row ids of the one after (unconditional loads of clamped rows, all in
  // flight at once), so each load has a chunk's worth of adds to arrive in.
  uint32_t id[kPer];
  float l[kPer], w[kPer], ln[kPer];
  auto fetch_ids = [&](int c) {
    const int r0 = c * kGStep;
    const int cnt = min(kGStep, n - r0);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int a = r0 + min(slot + u * kSlots, cnt - 1);
      id[u] = aids[a];
      ln[u] = lg[a];
    }
  };
  auto fetch_w = [&]() {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      w[u] = W[static_cast<size_t>(id[u]) * dim + jc];
      l[u] = ln[u];
    }
  };
  auto produce = [&](int c) {
    float wc[kPer], lc[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      wc[u] = w[u];
      lc[u] = l[u];
    }
    if (c + 1 < nch) fetch_w();           // chunk c + 1 (its ids arrived a chunk ago)
    if (c + 2 < nch) fetch_ids(c + 2);
    float* dst = reinterpret_cast<float*>(&gb[c & 1][0][0]);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int rr = slot + u * kSlots;
      if (rr < kGStep) dst[((rr >> 2) * kGc + col) * 4 + (rr & 3)] = lc[u] * wc[u];
    }
  };
  if (wave > 0 && nch > 0) {
    fetch_ids(0);
    fetch_w();
    if (nch > 1) fetch_ids(1);
    produce(0);
  }
  lds_barrier();
  float r = 0.0f;
  for (int c = 0; c < nch; ++c) {
    if (wave > 0) {
      if (c + 1 < nch) produce(c + 1);
    } else if (lane < kGc) {
      const int cnt = min(kGStep, n - c * kGStep);
      const float4(*src)[kGc] = gb[c & 1];
      if (cnt == kGStep) {
        r = chain_add_quads<kGc>(&src[0][lane], kGStep / 4, r);
      } else {
        const float* sf = reinterpret_cast<const float*>(&src[0][0]);
        for (int j = 0; j < cnt; ++j) r = r + sf[((j >> 2) * kGc + lane) * 4 + (j & 3)];
      }
    }
    lds_barrier();
  }
  if (wave == 0 && lane < kGc && j0 + lane < dim) gi[j0 + lane] = r;
}

// Optimizer::update of every active neuron (layer.rs:209-222): grad_weights[j]
// = lg * x[j] over all dim inputs (zeros included: momentum and Adam state
// move every step), grad_bias = lg.  The transposed copy follows the rows.
// Grid: x over 2048-column slices of a row, y over active neurons.
constexpr int kUCols = 2048;
__global__ __launch_bounds__(kTrThreads) void tr_update_kernel(
    float* __restrict__ W, float* __restrict__ WTN, float* __restrict__ bias, int n, int dim,
    const uint32_t* __restrict__ aids, const int32_t* __restrict__ alen, int cap,
    const float* __restrict__ lg, const float* __restrict__ x, OptArgs o) {
  const int na = min(alen[0], cap);
  const int j0 = blockIdx.x * kUCols, j1 = min(dim, j0 + kUCols);
  for (int a = blockIdx.y; a < na; a += gridDim.y) {
    const uint32_t id = aids[a];
    if (id >= static_cast<uint32_t>(n)) continue;
    const float g = lg[a];
    const size_t row = static_cast<size_t>(id) * dim;
    float* w = W + row;
    for (int j = j0 + threadIdx.x; j < j1; j += blockDim.x) {
      const float gw = g * x[j];
      float* s1 = o.st_w1 ? o.st_w1 + row + j : nullptr;
      float* s2 = o.st_w2 ? o.st_w2 + row + j : nullptr;
      const float nw = opt_step(w[j], gw, s1, s2, o);
      w[j] = nw;
      if (WTN) WTN[static_cast<size_t>(j) * n + id] = nw;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      float* s1 = o.st_b1 ? o.st_b1 + id : nullptr;
      float* s2 = o.st_b2 ? o.st_b2 + id : nullptr;
      bias[id] = opt_step(bias[id], g, s1, s2, o);
    }
  }
}

// Local gradients -> (grad_input) -> update of one layer for one example.
// x: the layer's dense input; post: activations in list order (softmax only).
// keep_wtn: write updated rows into the transposed copy too (scattered
// 4-byte stores, one per weight); a network step instead re-transposes once
// after the whole batch (wtn_refresh).
static int layer_backward_launch(kh_slide_layer* l, const float* x, const uint32_t* aids,
                                 const int32_t* alen, int cap, const float* pre,
                                 const float* post, const float* dense, const float* grad_out,
                                 int64_t grad_len, bool lg_ready, float* go, float* lg,
                                 const OptArgs& o, float* gi, bool keep_wtn, hipStream_t st) {
  const unsigned ab = static_cast<unsigned>(ceil_div(cap, kTrThreads));
  if (!lg_ready) {
    hipLaunchKernelGGL(tr_local_grad_kernel, dim3(ab), dim3(kTrThreads), 0, st, aids, alen, cap,
                       pre, dense, l->act, grad_out, grad_len, go, lg);
    KH_LAUNCHED();
  }
  if (l->act == KH_ACT_SOFTMAX) {
    hipLaunchKernelGGL(tr_softmax_jacobian_kernel, dim3((unsigned)std::min(ceil_div(cap, kJc), kJBlocks)),
                       dim3(kJThreads), 0, st, post, go, alen, cap, lg);
    KH_LAUNCHED();
  }
  if (gi) {
    hipLaunchKernelGGL(tr_grad_input_kernel, dim3((unsigned)ceil_div(l->dim, kGc)), dim3(kGThreads), 0, st,
                       l->w, l->dim, aids, alen, cap, lg, gi);
    KH_LAUNCHED();
  }
  const int xs = ceil_div(l->dim, kUCols);
  const int ys = std::max(1, std::min(cap, std::max(1, 4096 / xs)));
  hipLaunchKernelGGL(tr_update_kernel, dim3(xs, ys), dim3(kTrThreads), 0, st, l->w,
                     keep_wtn ? l->wtn : nullptr, l->bias, l->n, l->dim, aids, alen, cap, lg, x, o);
  KH_LAUNCHED();
  return KH_OK;
}

// The transposed copy of a non-softmax layer rebuilt from the weights.
static int wtn_refresh(kh_slide_layer* l, hipStream_t st) {
  if (!l->wtn) return KH_OK;
  hipLaunchKernelGGL(transpose_kernel<float>, dim3(ceil_div(l->dim, 32), ceil_div(l->n, 32)), dim3(256),
                     0, st, l->w, l->n, l->dim, l->wtn);
  KH_LAUNCHED();
  return KH_OK;
}

}  // namespace kh

using namespace kh;

// ======================================================================== scheduler
static uint64_t sched_interval(const kh_rebuild_scheduler* s) {
  // (base as f64 * (decay * count as f64).exp()) as usize, then .max(1)
  const double v = static_cast<double>(s->base_interval) *
                   std::exp(s->decay * static_cast<double>(s->rebuild_count));
  uint64_t n;
  if (!(v > 0.0)) n = 0;                              // NaN and <= 0 saturate to 0
  else if (v >= 18446744073709551616.0) n = UINT64_MAX;
  else n = static_cast<uint64_t>(v);
  return n < 1 ? 1 : n;
}

static int sched_due(kh_rebuild_scheduler* s) {
  if (s->current_step >= s->next_rebuild_step) {
    s->rebuild_count += 1;
    s->next_rebuild_step = s->current_step + sched_interval(s);  // wraps as a release build
    return 1;
  }
  return 0;
}

extern "C" void kh_rebuild_scheduler_init(kh_rebuild_scheduler* s, uint64_t base_interval,
                                          double decay) {
  if (!s) return;
  s->base_interval = base_interval;
  s->decay = decay;
  s->rebuild_count = 0;
  s->next_rebuild_step = base_interval;
  s->current_step = 0;
}

extern "C" int kh_rebuild_scheduler_step(kh_rebuild_scheduler* s) {
  if (!s) return 0;
  s->current_step += 1;
  return sched_due(s);
}

extern "C" int kh_rebuild_scheduler_should_rebuild(kh_rebuild_scheduler* s, uint64_t step) {
  if (!s) return 0;
  s->current_step = step;
  return sched_due(s);
}

// ======================================================================== index / layer
extern "C" int kh_lsh_index_rebuild(kh_lsh_index* idx, const uint32_t* ids_dev, const float* w_dev,
                                    int64_t n, int64_t ldw, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0 && ldw >= idx->h->dim, "bad n/ldw");
  int rc = kh_lsh_index_clear(idx, stream);
  if (rc != KH_OK || n == 0) return rc;
  return kh_lsh_index_insert(idx, ids_dev, w_dev, n, ldw, stream);
}

extern "C" int kh_slide_layer_rebuild_index(kh_slide_layer* l, void* stream) {
  KH_CHECK_ARG(l != nullptr, "null layer");
  uint32_t* ids = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * l->n));
  if (!ids) return KH_ERR_ALLOC;
  std::vector<uint32_t> h(l->n);
  for (int i = 0; i < l->n; ++i) h[i] = static_cast<uint32_t>(i);
  hipStream_t st = as_stream(stream);
  int rc = KH_OK;
  if (hipMemcpyAsync(ids, h.data(), sizeof(uint32_t) * l->n, hipMemcpyHostToDevice, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    set_error("rebuild upload failed");
    rc = KH_ERR_HIP;
  }
  if (rc == KH_OK) rc = kh_lsh_index_rebuild(l->index, ids, l->w, l->n, l->dim, stream);
  if (rc == KH_OK && hipStreamSynchronize(st) != hipSuccess) {
    set_error("rebuild failed");
    rc = KH_ERR_HIP;
  }
  dev_free(ids);
  return rc;
}

extern "C" int kh_slide_layer_init_optimizer(kh_slide_layer* l, int optimizer, float momentum,
                                             float beta1, float beta2, float eps) {
  KH_CHECK_ARG(l != nullptr, "null layer");
  KH_CHECK_ARG(optimizer == KH_OPT_SGD || optimizer == KH_OPT_ADAM, "bad optimizer %d", optimizer);
  l->free_opt();
  const size_t nw = static_cast<size_t>(l->n) * l->dim;
  const bool two = optimizer == KH_OPT_ADAM;
  const bool one = two || momentum > 0.0f;
  if (one) {
    l->st_w1 = static_cast<float*>(dev_alloc(sizeof(float) * nw));
    l->st_b1 = static_cast<float*>(dev_alloc(sizeof(float) * l->n));
    if (!l->st_w1 || !l->st_b1) {
      l->free_opt();
      return KH_ERR_ALLOC;
    }
  }
  if (two) {
    l->st_w2 = static_cast<float*>(dev_alloc(sizeof(float) * nw));
    l->st_b2 = static_cast<float*>(dev_alloc(sizeof(float) * l->n));
    if (!l->st_w2 || !l->st_b2) {
      l->free_opt();
      return KH_ERR_ALLOC;
    }
  }
  float* bufs[4] = {l->st_w1, l->st_w2, l->st_b1, l->st_b2};
  const size_t cnt[4] = {nw, nw, (size_t)l->n, (size_t)l->n};
  for (int i = 0; i < 4; ++i)
    if (bufs[i] && hipMemset(bufs[i], 0, sizeof(float) * cnt[i]) != hipSuccess) {
      l->free_opt();
      set_error("optimizer state clear failed");
      return KH_ERR_HIP;
    }
  l->opt = optimizer;
  l->momentum = momentum;
  l->beta1 = beta1;
  l->beta2 = beta2;
  l->eps = eps;
  return KH_OK;
}

extern "C" int kh_slide_layer_weights(const kh_slide_layer* l, float* w_host, float* bias_host) {
  KH_CHECK_ARG(l != nullptr, "null layer");
  if (w_host)
    KH_HIP(hipMemcpy(w_host, l->w, sizeof(float) * l->n * (size_t)l->dim, hipMemcpyDeviceToHost));
  if (bias_host) KH_HIP(hipMemcpy(bias_host, l->bias, sizeof(float) * l->n, hipMemcpyDeviceToHost));
  return KH_OK;
}

extern "C" int kh_slide_layer_backward(kh_slide_layer* l, const float* x_dev,
                                       const uint32_t* act_ids_dev, const int32_t* n_act_dev,
                                       const float* pre_dev, const float* act_dense_dev,
                                       const float* grad_out_dev, int64_t grad_out_len, double lr,
                                       uint64_t step, float* grad_in_dev, void* stream) {
  KH_CHECK_ARG(l != nullptr, "null layer");
  KH_CHECK_ARG(l->opt >= 0, "kh_slide_layer_init_optimizer was not called");
  KH_CHECK_ARG(x_dev && act_ids_dev && n_act_dev && pre_dev && act_dense_dev, "null argument");
  KH_CHECK_ARG(grad_out_len >= 0 && (grad_out_len == 0 || grad_out_dev), "bad grad_out");
  hipStream_t st = as_stream(stream);
  // An active list holds distinct neuron ids, so at most n entries.
  const int cap = l->n;
  WsSet* w = l->ws.get(st);
  float* go = static_cast<float*>(w->get(0, sizeof(float) * cap));
  float* lg = static_cast<float*>(w->get(1, sizeof(float) * cap));
  float* post = static_cast<float*>(w->get(2, sizeof(float) * cap));
  if (!go || !lg || !post) return KH_ERR_ALLOC;
  if (l->act == KH_ACT_SOFTMAX) {
    // Layer::backward recomputes apply_softmax(pre_activations) (layer.rs:147)
    hipLaunchKernelGGL(tr_softmax_kernel, dim3(1), dim3(kTrThreads), 0, st, pre_dev, act_ids_dev,
                       n_act_dev, cap, post, nullptr);
    KH_LAUNCHED();
  }
  return layer_backward_launch(l, x_dev, act_ids_dev, n_act_dev, cap, pre_dev, post,
                               act_dense_dev, grad_out_dev, grad_out_len, false, go, lg,
                               opt_args(l, lr, step), grad_in_dev, true, st);
}

// ======================================================================== network
namespace {

struct TrainBufs {
  int qs = 0, as = 0;
  uint32_t* codes = nullptr;
  uint32_t* qids = nullptr;
  uint32_t* qcnt = nullptr;
  int32_t* qlen = nullptr;
  uint32_t* aids = nullptr;
  int32_t* alen = nullptr;
  float* pre = nullptr;
  float* post = nullptr;
  float* dense = nullptr;  // [n] the layer's activations (Layer::forward's `activations`)
  float* go = nullptr;
  float* lg = nullptr;
  float* gi = nullptr;     // [dim] gradient w.r.t. the layer's input
  uint32_t* nzi = nullptr;
  float* nzv = nullptr;
  int64_t* xoff = nullptr;
};

}  // namespace

struct kh_slide_network {
  std::vector<kh_slide_layer*> layers;
  std::vector<TrainBufs> b;
  std::vector<void*> allocs;
  uint64_t step = 0;
  kh_rebuild_scheduler sched{};
  float* loss_total = nullptr;
  float* x_dense = nullptr;  // [in_dim] the current sparse example, densified
  uint32_t* labels = nullptr;
  size_t labels_cap = 0;
  int in_dim = 0, out_dim = 0;
  template <typename T>
  T* alloc(size_t n, bool zero = false) {
    void* p = dev_alloc(sizeof(T) * (n ? n : 1));
    if (!p) return nullptr;
    allocs.push_back(p);
    if (zero && hipMemset(p, 0, sizeof(T) * (n ? n : 1)) != hipSuccess) return nullptr;
    return static_cast<T*>(p);
  }
};

extern "C" int kh_slide_network_destroy(kh_slide_network* n) {
  if (!n) return KH_OK;
  for (void* p : n->allocs) dev_free(p);
  dev_free(n->labels);
  delete n;
  return KH_OK;
}

extern "C" int kh_slide_network_create(kh_slide_layer* const* layers, int n_layers, int optimizer,
                                       float momentum, float beta1, float beta2, float eps,
                                       uint64_t rebuild_base, double rebuild_decay,
                                       kh_slide_network** out) {
  KH_CHECK_ARG(out && layers && n_layers > 0, "null argument / no layers");
  *out = nullptr;
  for (int i = 0; i < n_layers; ++i) {
    KH_CHECK_ARG(layers[i] != nullptr, "null layer %d", i);
    KH_CHECK_ARG(i == 0 || layers[i]->dim == layers[i - 1]->n,
                 "layer %d input_dim %d != layer %d num_neurons %d", i, layers[i]->dim, i - 1,
                 layers[i - 1]->n);
    const kh_lsh_index* idx = layers[i]->index;
    KH_CHECK_ARG(layers[i]->sampling != KH_SAMPLING_TOPK || idx->L * idx->cap + 1 <= 8193,
                 "top-k sampling supports num_tables * bucket_capacity <= 8192");
  }
  auto* net = new kh_slide_network();
  net->layers.assign(layers, layers + n_layers);
  net->in_dim = layers[0]->dim;
  net->out_dim = layers[n_layers - 1]->n;
  kh_rebuild_scheduler_init(&net->sched, rebuild_base, rebuild_decay);
  int rc = KH_OK;
  for (int i = 0; i < n_layers && rc == KH_OK; ++i)
    rc = kh_slide_layer_init_optimizer(layers[i], optimizer, momentum, beta1, beta2, eps);
  net->b.resize(n_layers);
  for (int i = 0; i < n_layers && rc == KH_OK; ++i) {
    const kh_slide_layer* l = layers[i];
    TrainBufs& t = net->b[i];
    t.qs = l->index->L * l->index->cap;
    t.as = std::max(t.qs, l->n);
    t.codes = net->alloc<uint32_t>(l->index->L);
    t.qids = net->alloc<uint32_t>(t.qs);
    t.qcnt = net->alloc<uint32_t>(t.qs);
    t.qlen = net->alloc<int32_t>(1, true);
    t.aids = net->alloc<uint32_t>(t.as, true);
    t.alen = net->alloc<int32_t>(1, true);
    t.pre = net->alloc<float>(t.as);
    t.post = net->alloc<float>(t.as);
    t.dense = net->alloc<float>(l->n, true);
    t.go = net->alloc<float>(t.as);
    t.lg = net->alloc<float>(t.as);
    t.gi = net->alloc<float>(l->dim);
    t.nzi = net->alloc<uint32_t>(l->dim);
    t.nzv = net->alloc<float>(l->dim);
    t.xoff = net->alloc<int64_t>(2, true);
    if (!t.codes || !t.qids || !t.qcnt || !t.qlen || !t.aids || !t.alen || !t.pre || !t.post ||
        !t.dense || !t.go || !t.lg || !t.gi || !t.nzi || !t.nzv || !t.xoff)
      rc = KH_ERR_ALLOC;
  }
  if (rc == KH_OK) {
    net->loss_total = net->alloc<float>(1, true);
    net->x_dense = net->alloc<float>(net->in_dim, true);
    if (!net->loss_total || !net->x_dense) rc = KH_ERR_ALLOC;
  }
  if (rc != KH_OK) {
    kh_slide_network_destroy(net);
    return rc;
  }
  *out = net;
  return KH_OK;
}

// Stage example e of a CSR batch as layer 0's input (to_dense semantics).
static int net_stage_sparse(kh_slide_network* net, const int64_t* xoff, const uint32_t* xidx,
                            const float* xval, int64_t e, hipStream_t st) {
  TrainBufs& t = net->b[0];
  hipLaunchKernelGGL(tr_stage_csr_kernel, dim3(1), dim3(1024), 0, st, xoff, xidx, xval, e,
                     net->in_dim, t.nzi, t.nzv, t.xoff, net->x_dense);
  KH_LAUNCHED();
  return KH_OK;
}

// Host check of a CSR batch: offsets nondecreasing, at most kTrMaxNnz stored
// entries per example (reads the offsets back; synchronous).
static int net_check_csr(const int64_t* xoff, int64_t batch, hipStream_t st) {
  std::vector<int64_t> off(batch + 1);
  KH_HIP(hipMemcpyAsync(off.data(), xoff, sizeof(int64_t) * (batch + 1), hipMemcpyDeviceToHost, st));
  KH_HIP(hipStreamSynchronize(st));
  for (int64_t e = 0; e < batch; ++e)
    KH_CHECK_ARG(off[e + 1] >= off[e] && off[e + 1] - off[e] <= kTrMaxNnz,
                 "example %lld: offsets must be nondecreasing with at most %d entries", (long long)e,
                 kTrMaxNnz);
  return KH_OK;
}

// Network::forward for one example (net.rs:62-78), layer by layer: nonzeros of
// the input, hash, query, sampling in the sampler's order (clearing the
// previous example's entries of the dense activations), neuron sums, softmax.
// x == nullptr: layer 0's input was staged from a sparse example.
static int net_forward_one(kh_slide_network* net, const float* x, hipStream_t st) {
  const float* in = x;
  for (size_t i = 0; i < net->layers.size(); ++i) {
    kh_slide_layer* l = net->layers[i];
    TrainBufs& t = net->b[i];
    if (in) {
      hipLaunchKernelGGL(tr_stage_nz_kernel, dim3(1), dim3(1024), 0, st, in, l->dim, t.nzi, t.nzv,
                         t.xoff);
      KH_LAUNCHED();
    }
    int rc = hash_sparse_launch(l->index->h, t.xoff, t.nzi, t.nzv, 1, t.codes, st);
    if (rc != KH_OK) return rc;
    const int qs = query_stride(l->index);
    rc = query_launch(l->index, t.codes, 1, t.qids, t.qcnt, qs, t.qlen, st);
    if (rc != KH_OK) return rc;
    rc = select_launch(l, t.qids, t.qcnt, t.qlen, qs, 1, t.aids, t.as, t.alen, true, t.dense, st);
    if (rc != KH_OK) return rc;
    const unsigned nb = static_cast<unsigned>(std::min(ceil_div(t.as, kTrThreads), 64));
    const size_t lds = (sizeof(uint32_t) + sizeof(float)) * kTrLdsNz;
    hipLaunchKernelGGL(tr_neuron_kernel, dim3(nb), dim3(kTrThreads), lds, st, l->w, l->bias, l->dim,
                       t.nzi, t.nzv, t.xoff, t.aids, t.alen, t.as, l->act, t.pre, t.post, t.dense);
    KH_LAUNCHED();
    if (l->act == KH_ACT_SOFTMAX) {
      hipLaunchKernelGGL(tr_softmax_kernel, dim3(1), dim3(kTrThreads), 0, st, t.pre, t.aids, t.alen,
                         t.as, t.post, t.dense);
      KH_LAUNCHED();
    }
    in = t.dense;
  }
  return KH_OK;
}

static int net_setup_attrs() {
  static int rc = [] {
    const size_t lds = (sizeof(uint32_t) + sizeof(float)) * kTrLdsNz;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&tr_neuron_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) ==
                   hipSuccess
               ? KH_OK
               : KH_ERR_HIP;
  }();
  if (rc != KH_OK) set_error("hipFuncSetAttribute failed");
  return rc;
}

// Network::train_step over dense rows (x_dev) or CSR rows (xoff != nullptr).
static int net_train_step(kh_slide_network* net, const float* x_dev, const int64_t* xoff,
                          const uint32_t* xidx, const float* xval, int64_t batch,
                          const int64_t* label_off_host, const uint32_t* labels_host, double lr,
                          float* loss_out, void* stream) {
  KH_CHECK_ARG(net && loss_out, "null argument");
  KH_CHECK_ARG(batch >= 0, "bad batch");
  *loss_out = 0.0f;
  if (batch == 0) return KH_OK;  // net.rs:82-84: nothing changes
  KH_CHECK_ARG((x_dev || xoff) && label_off_host, "null input");
  KH_CHECK_ARG(label_off_host[0] == 0, "label offsets must start at 0");
  for (int64_t e = 0; e < batch; ++e)
    KH_CHECK_ARG(label_off_host[e + 1] >= label_off_host[e] &&
                     label_off_host[e + 1] - label_off_host[e] <= kTrMaxLabels,
                 "example %lld: label offsets must be nondecreasing with at most %d labels",
                 (long long)e, kTrMaxLabels);
  const int64_t n_labels = label_off_host[batch];
  KH_CHECK_ARG(n_labels == 0 || labels_host, "null labels");
  int rc = net_setup_attrs();
  if (rc != KH_OK) return rc;
  hipStream_t st = as_stream(stream);
  if (xoff) {
    rc = net_check_csr(xoff, batch, st);
    if (rc != KH_OK) return rc;
  }
  if (static_cast<size_t>(n_labels) > net->labels_cap) {
    KH_HIP(hipStreamSynchronize(st));
    dev_free(net->labels);
    net->labels_cap = std::max<size_t>(n_labels, 2 * net->labels_cap);
    net->labels = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * net->labels_cap));
    if (!net->labels) {
      net->labels_cap = 0;
      return KH_ERR_ALLOC;
    }
  }
  if (n_labels)
    KH_HIP(hipMemcpyAsync(net->labels, labels_host, sizeof(uint32_t) * n_labels,
                          hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(fill_f32_kernel<>, dim3(1), dim3(64), 0, st, net->loss_total, (int64_t)1, 0.0f);
  KH_LAUNCHED();
  const int nl_layers = static_cast<int>(net->layers.size());
  std::vector<OptArgs> oa(nl_layers);
  for (int i = 0; i < nl_layers; ++i) oa[i] = opt_args(net->layers[i], lr, net->step);
  for (int64_t e = 0; e < batch; ++e) {
    const float* x = xoff ? net->x_dense : x_dev + e * static_cast<int64_t>(net->in_dim);
    if (xoff) {
      rc = net_stage_sparse(net, xoff, xidx, xval, e, st);
      if (rc != KH_OK) return rc;
    }
    rc = net_forward_one(net, xoff ? nullptr : x, st);
    if (rc != KH_OK) return rc;
    const int last = nl_layers - 1;
    kh_slide_layer* L = net->layers[last];
    TrainBufs& T = net->b[last];
    const int nl = static_cast<int>(label_off_host[e + 1] - label_off_host[e]);
    hipLaunchKernelGGL(tr_loss_grad_kernel, dim3(1), dim3(kTrThreads), 0, st, T.pre, T.post, T.aids,
                       T.alen, T.as, L->act, T.dense, net->labels + label_off_host[e], nl, T.go,
                       T.lg, net->loss_total);
    KH_LAUNCHED();
    // Network::backward (net.rs:122-146): last layer down to the first
    for (int i = last; i >= 0; --i) {
      kh_slide_layer* l = net->layers[i];
      TrainBufs& t = net->b[i];
      const float* in = i == 0 ? x : net->b[i - 1].dense;
      const float* grad_out = i == last ? nullptr : net->b[i + 1].gi;
      // the first layer's grad_input is not used by anything (net.rs:139-144)
      float* gi = i == 0 ? nullptr : t.gi;
      rc = layer_backward_launch(l, in, t.aids, t.alen, t.as, t.pre, t.post, t.dense, grad_out,
                                 l->n, i == last, t.go, t.lg, oa[i], gi, false, st);
      if (rc != KH_OK) return rc;
    }
  }
  for (kh_slide_layer* l : net->layers) {
    rc = wtn_refresh(l, st);
    if (rc != KH_OK) return rc;
  }
  float total = 0.0f;
  KH_HIP(hipMemcpyAsync(&total, net->loss_total, sizeof(float), hipMemcpyDeviceToHost, st));
  KH_HIP(hipStreamSynchronize(st));
  net->step += 1;
  if (kh_rebuild_scheduler_should_rebuild(&net->sched, net->step)) {
    for (kh_slide_layer* l : net->layers) {
      rc = kh_slide_layer_rebuild_index(l, stream);
      if (rc != KH_OK) return rc;
    }
  }
  *loss_out = total / static_cast<float>(batch);
  return KH_OK;
}

extern "C" int kh_slide_network_train_step(kh_slide_network* net, const float* x_dev, int64_t batch,
                                           const int64_t* label_off_host,
                                           const uint32_t* labels_host, double lr, float* loss_out,
                                           void* stream) {
  KH_CHECK_ARG(batch == 0 || x_dev, "null input");
  return net_train_step(net, x_dev, nullptr, nullptr, nullptr, batch, label_off_host, labels_host,
                        lr, loss_out, stream);
}

extern "C" int kh_slide_network_train_step_sparse(kh_slide_network* net, const int64_t* xoff_dev,
                                                  const uint32_t* xidx_dev, const float* xval_dev,
                                                  int64_t batch, const int64_t* label_off_host,
                                                  const uint32_t* labels_host, double lr,
                                                  float* loss_out, void* stream) {
  KH_CHECK_ARG(batch == 0 || xoff_dev, "null input");
  return net_train_step(net, nullptr, xoff_dev, xidx_dev, xval_dev, batch, label_off_host,
                        labels_host, lr, loss_out, stream);
}

static int net_predict(kh_slide_network* net, const float* x_dev, const int64_t* xoff,
                       const uint32_t* xidx, const float* xval, int64_t batch, float* out_dev,
                       void* stream) {
  KH_CHECK_ARG(net != nullptr, "null network");
  KH_CHECK_ARG(batch >= 0, "bad batch");
  if (batch == 0) return KH_OK;
  KH_CHECK_ARG((x_dev || xoff) && out_dev, "null argument");
  int rc = net_setup_attrs();
  if (rc != KH_OK) return rc;
  hipStream_t st = as_stream(stream);
  if (xoff) {
    rc = net_check_csr(xoff, batch, st);
    if (rc != KH_OK) return rc;
  }
  for (int64_t e = 0; e < batch; ++e) {
    if (xoff) {
      rc = net_stage_sparse(net, xoff, xidx, xval, e, st);
      if (rc != KH_OK) return rc;
    }
    rc = net_forward_one(net, xoff ? nullptr : x_dev + e * static_cast<int64_t>(net->in_dim), st);
    if (rc != KH_OK) return rc;
    KH_HIP(hipMemcpyAsync(out_dev + e * static_cast<int64_t>(net->out_dim), net->b.back().dense,
                          sizeof(float) * net->out_dim, hipMemcpyDeviceToDevice, st));
  }
  return KH_OK;
}

extern "C" int kh_slide_network_predict(kh_slide_network* net, const float* x_dev, int64_t batch,
                                        float* out_dev, void* stream) {
  return net_predict(net, x_dev, nullptr, nullptr, nullptr, batch, out_dev, stream);
}

extern "C" int kh_slide_network_predict_sparse(kh_slide_network* net, const int64_t* xoff_dev,
                                               const uint32_t* xidx_dev, const float* xval_dev,
                                               int64_t batch, float* out_dev, void* stream) {
  return net_predict(net, nullptr, xoff_dev, xidx_dev, xval_dev, batch, out_dev, stream);
}

extern "C" int kh_slide_network_state(const kh_slide_network* net, uint64_t* step,
                                      kh_rebuild_scheduler* scheduler) {
  KH_CHECK_ARG(net != nullptr, "null network");
  if (step) *step = net->step;
  if (scheduler) *scheduler = net->sched;
  return KH_OK;
}
