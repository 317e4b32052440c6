// slide.hip -- SLIDE sparse layer forward on the GPU (gfx950).
//
// Replaces Layer::forward (crates/klearu-core/src/network/layer.rs:65-120) with
// Neuron::forward / forward_sparse (network/neuron.rs:47-68), the sampling
// strategies (sampling/{vanilla,topk,threshold}.rs) and the activations
// (layer.rs:250-308); plus a dense layer over sparse inputs (every neuron,
// Neuron::forward_sparse) for the hidden layer of the extreme-classification net.
//
// Per batch: hash (lsh.hip) -> query (unique ids + hit counts, ascending) ->
// select_kernel (sampling, empty -> all neurons, ids < n) -> neuron_kernel
// (one block per sample; each thread replays the reference's sequential f32
// sum for one active neuron over the sample's nonzero inputs, then the
// activation; softmax reduces over the block) -> CSR.
//
// Skipping zero inputs leaves a sequential sum unchanged (adding +-0 to a
// nonzero partial sum returns it; a zero partial sum only changes the sign of
// zero), so pre-activations are bit-identical to the reference's dense loop.
#include <algorithm>
#include <mutex>
#include <vector>

#include "gather.hpp"
#include "slide_internal.hpp"

namespace kh {

constexpr int kSlideThreads = 256;
constexpr int kMaxCountBins = 8193;

// Top-k sampling in the sampler's own order (count descending, then id, as
// TopKSampling::select sorts, sampling/topk.rs:19-34): a stable counting sort
// of the ascending candidates.  hist[c] becomes the number of candidates with
// a count above c; wave 0 then walks the candidates in id order and places
// each after the earlier ones of its count.  Returns min(m, top_k), the
// sampler's pick count; picks with ids >= num_neurons are dropped in order.
__device__ int select_topk_count_order(const uint32_t* __restrict__ ids,
                                       const uint32_t* __restrict__ cnt, int m, int top_k,
                                       int num_neurons, int nbins, unsigned* hist, int* wsum,
                                       int* s_total, uint32_t* __restrict__ out, int* n_kept) {
  for (int i = threadIdx.x; i < nbins; i += blockDim.x) hist[i] = 0u;
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += blockDim.x) atomicAdd(&hist[cnt[i]], 1u);
  __syncthreads();
  // exclusive suffix sums: thread t owns a run of bins, thread 0 the highest
  const int seg = (nbins + (int)blockDim.x - 1) / (int)blockDim.x;
  const int hi = nbins - 1 - (int)threadIdx.x * seg;
  const int lo = max(hi - seg + 1, 0);
  int run = 0;
  for (int c = hi; c >= lo; --c) run += (int)hist[c];
  int above = block_excl_scan(run, wsum, s_total);
  for (int c = hi; c >= lo; --c) {
    const int h = (int)hist[c];
    hist[c] = (unsigned)above;
    above += h;
  }
  __syncthreads();
  const int take = min(m, top_k);
  if ((threadIdx.x >> 6) == 0) {
    const int lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int c0 = 0; c0 < m; c0 += 64) {
      const int i = c0 + lane;
      const int c = i < m ? (int)cnt[i] : -1;
      uint64_t pend = __ballot(i < m);
      while (pend) {
        const int leader = __ffsll((unsigned long long)pend) - 1;
        const int cl = __shfl(c, leader);
        const uint64_t same = __ballot(c == cl);
        const int base = (int)hist[cl];
        if (c == cl) {
          const int pos = base + __popcll(same & below);
          if (pos < take) out[pos] = ids[i];
        }
        __builtin_amdgcn_wave_barrier();
        if (lane == leader) hist[cl] = (unsigned)(base + __popcll(same));
        __builtin_amdgcn_wave_barrier();
        pend &= ~same;
      }
    }
  }
  __syncthreads();
  // drop ids >= num_neurons, keeping the order (layer.rs:87)
  int base = 0;
  for (int c0 = 0; c0 < take; c0 += blockDim.x) {
    const int i = c0 + threadIdx.x;
    const uint32_t id = i < take ? out[i] : 0u;
    const int keep = i < take && id < (uint32_t)num_neurons;
    const int pos = block_excl_scan(keep, wsum, s_total) + base;
    if (keep) out[pos] = id;
    base += *s_total;
    __syncthreads();
  }
  *n_kept = base;
  return take;
}

// clear_dense (training): the row's dense activation vector [num_neurons];
// the entries of the previous active list (aids/alen still hold it) are
// zeroed before the new list is written.  count_order: top-k picks in the
// sampler's order instead of ascending ids.
__global__ __launch_bounds__(kSlideThreads) void select_kernel(
    const uint32_t* __restrict__ qids, const uint32_t* __restrict__ qcnt,
    const int32_t* __restrict__ qlen, int qstride, int sampling, int top_k, int threshold,
    int num_neurons, int nbins, uint32_t* __restrict__ aids, int astride,
    int32_t* __restrict__ alen, int count_order, float* __restrict__ clear_dense, int fallback) {
  extern __shared__ unsigned hist[];
  __shared__ int wsum[kSlideThreads / 64];
  __shared__ int s_total;
  __shared__ int s_cstar, s_take, s_best_id;
  const int64_t row = blockIdx.x;
  const uint32_t* ids = qids + row * (int64_t)qstride;
  const uint32_t* cnt = qcnt + row * (int64_t)qstride;
  uint32_t* out = aids + row * (int64_t)astride;
  const int m = qlen[row];
  if (clear_dense) {
    float* dn = clear_dense + row * (int64_t)num_neurons;
    const int old = alen[row];
    for (int a = threadIdx.x; a < old; a += blockDim.x) dn[out[a]] = 0.0f;
    __syncthreads();
  }
  int cstar = 0, take_eq = 0;  // topk: take count > cstar, plus take_eq of count == cstar
  int mode = sampling;
  if (sampling == KH_SAMPLING_TOPK && count_order) {
    int n_kept = 0;
    const int n_pre = select_topk_count_order(ids, cnt, m, top_k, num_neurons, nbins, hist, wsum,
                                              &s_total, out, &n_kept);
    int n_sel = n_kept;
    if (n_pre == 0 && fallback) {
      for (int i = threadIdx.x; i < num_neurons; i += blockDim.x) out[i] = (uint32_t)i;
      n_sel = num_neurons;
    }
    if (threadIdx.x == 0) alen[row] = n_sel;
    return;
  }
  if (sampling == KH_SAMPLING_TOPK) {
    if (m <= top_k) {
      mode = KH_SAMPLING_VANILLA;
    } else {
      for (int i = threadIdx.x; i < nbins; i += blockDim.x) hist[i] = 0u;
      __syncthreads();
      for (int i = threadIdx.x; i < m; i += blockDim.x) atomicAdd(&hist[cnt[i]], 1u);
      __syncthreads();
      // Find the count c* where the number of candidates with count >= c*
      // first reaches top_k.  Thread t owns a run of bins, thread 0 the
      // highest; an exclusive scan gives each run the number of candidates
      // above it, and the run holding the crossing walks its bins downwards.
      if (threadIdx.x == 0) {
        s_cstar = 0;
        s_take = top_k;
      }
      const int seg = (nbins + (int)blockDim.x - 1) / (int)blockDim.x;
      const int hi = nbins - 1 - (int)threadIdx.x * seg;
      const int lo = max(hi - seg + 1, 0);
      int run = 0;
      for (int c = hi; c >= lo; --c) run += (int)hist[c];
      const int above = block_excl_scan(run, wsum, &s_total);
      if (hi >= 0 && above < top_k && above + run >= top_k) {
        int a = above, c = hi;
        for (; c > lo; --c) {
          if (a + (int)hist[c] >= top_k) break;
          a += (int)hist[c];
        }
        s_cstar = c;
        s_take = top_k - a;
      }
      __syncthreads();
      cstar = s_cstar;
      take_eq = s_take;
    }
  }
  // n_pre counts the sampler's picks before ids >= num_neurons are dropped:
  // the all-neurons fallback (layer.rs:82-84) runs before that filter (:87).
  int n_sel = 0, n_pre = 0;
  if (mode == KH_SAMPLING_THRESHOLD) {
    int base = 0, passed = 0;
    for (int c0 = 0; c0 < m; c0 += blockDim.x) {
      const int i = c0 + threadIdx.x;
      const int sel = (i < m && cnt[i] >= (uint32_t)threshold) ? 1 : 0;
      const int id = i < m ? (int)ids[i] : 0;
      const int keep = sel && (uint32_t)id < (uint32_t)num_neurons;
      block_excl_scan(sel, wsum, &s_total);
      passed += s_total;
      const int pos = block_excl_scan(keep, wsum, &s_total) + base;
      if (keep) out[pos] = (uint32_t)id;
      base += s_total;
    }
    n_sel = base;
    n_pre = passed;
    if (m > 0 && passed == 0) {
      // threshold.rs:37-42: the single best candidate (highest count, then
      // lowest id; ids are ascending, so the first maximum).
      if (threadIdx.x == 0) {
        uint32_t bc = 0, bi = ids[0];
        for (int i = 0; i < m; ++i)
          if (cnt[i] > bc || i == 0) {
            bc = cnt[i];
            bi = ids[i];
          }
        s_best_id = (int)bi;
      }
      __syncthreads();
      n_pre = 1;
      n_sel = 0;
      if ((uint32_t)s_best_id < (uint32_t)num_neurons) {
        if (threadIdx.x == 0) out[0] = (uint32_t)s_best_id;
        n_sel = 1;
      }
    }
  } else {
    // Thread t owns the candidates [t*R, t*R + R) in order, so one block scan
    // per quantity gives every output position: the rank among the count ==
    // c* candidates (top-k), then the position among the kept ones.
    // No pick at all (no candidates, or top-k of 0) writes nothing: the
    // all-neurons fallback below then owns the output.
    const bool topk = mode == KH_SAMPLING_TOPK;
    n_pre = topk ? min(m, top_k) : m;
    const int R = n_pre > 0 ? (m + (int)blockDim.x - 1) / (int)blockDim.x : 0;
    const int i0 = min((int)threadIdx.x * R, m), i1 = min(i0 + R, m);
    int eq_base = 0;
    if (topk) {
      int n_eq = 0;
      for (int i = i0; i < i1; ++i) n_eq += (int)cnt[i] == cstar ? 1 : 0;
      eq_base = block_excl_scan(n_eq, wsum, &s_total);
    }
    int n_keep = 0;
    for (int i = i0, r = eq_base; i < i1; ++i) {
      bool sel = true;
      if (topk) {
        const int c = (int)cnt[i];
        sel = c > cstar || (c == cstar && r < take_eq);
        r += c == cstar ? 1 : 0;
      }
      n_keep += sel && ids[i] < (uint32_t)num_neurons ? 1 : 0;
    }
    int pos = block_excl_scan(n_keep, wsum, &s_total);
    n_sel = s_total;
    for (int i = i0, r = eq_base; i < i1; ++i) {
      bool sel = true;
      if (topk) {
        const int c = (int)cnt[i];
        sel = c > cstar || (c == cstar && r < take_eq);
        r += c == cstar ? 1 : 0;
      }
      const uint32_t id = ids[i];
      if (sel && id < (uint32_t)num_neurons) out[pos++] = id;
    }
  }
  // empty selection -> every neuron (layer.rs:82-84)
  if (n_pre == 0 && fallback) {
    for (int i = threadIdx.x; i < num_neurons; i += blockDim.x) out[i] = (uint32_t)i;
    n_sel = num_neurons;
  }
  if (threadIdx.x == 0) alen[row] = n_sel;
}

// One block per sample (several per sample without softmax: blockIdx.y takes
// every gridDim.y-th block of active ids).  x is either dense [batch][dim]
// (zeros skipped) or CSR.  TRANS: W is the transposed copy [dim][nn].
// fb_n > 0 (Vanilla sampling read straight from the query, every id below the
// layer's fb_n neurons): a sample whose candidate list is empty takes all fb_n
// neurons (layer.rs:82-84), whose ids the blocks write into its aids row; the
// row lengths the outputs use go to alen_out (vanilla_len decides).
__device__ __forceinline__ int vanilla_len(const int32_t* alen, int64_t row, int fb_n, bool& all) {
  const int n = alen[row];
  all = fb_n > 0 && n == 0;
  return all ? fb_n : n;
}
template <bool SPARSE, bool TRANS>
__global__ __launch_bounds__(kSlideThreads) void neuron_kernel(
    const float* __restrict__ W, int nn, const float* __restrict__ bias, int dim,
    const float* __restrict__ x, const int64_t* __restrict__ xoff,
    const uint32_t* __restrict__ xidx, const float* __restrict__ xval,
    uint32_t* __restrict__ aids, int astride, const int32_t* __restrict__ alen, int act,
    int max_nz, float* __restrict__ pre, float* __restrict__ post, int fb_n = 0,
    int32_t* __restrict__ alen_out = nullptr) {
  extern __shared__ unsigned char smem[];
  uint32_t* nzi = reinterpret_cast<uint32_t*>(smem);
  float* nzv = reinterpret_cast<float*>(smem + sizeof(uint32_t) * max_nz);
  __shared__ int wsum[kSlideThreads / 64];
  __shared__ int s_total;
  __shared__ float red[kSlideThreads / 64];
  const int64_t row = blockIdx.x;
  int nnz;
  const uint32_t* li;
  const float* lv;
  if (SPARSE) {
    const int64_t a = xoff[row];
    nnz = (int)(xoff[row + 1] - a);
    if (nnz <= max_nz) {
      for (int i = threadIdx.x; i < nnz; i += blockDim.x) {
        nzi[i] = xidx[a + i];
        nzv[i] = xval[a + i];
      }
      __syncthreads();
      li = nzi;
      lv = nzv;
    } else {
      li = xidx + a;
      lv = xval + a;
    }
  } else {
    const float* xr = x + row * (int64_t)dim;
    int base = 0;
    for (int c0 = 0; c0 < dim; c0 += blockDim.x) {
      const int d = c0 + threadIdx.x;
      const float v = d < dim ? xr[d] : 0.0f;
      const int nz = v != 0.0f ? 1 : 0;
      const int pos = block_excl_scan(nz, wsum, &s_total) + base;
      if (nz) {
        nzi[pos] = (uint32_t)d;
        nzv[pos] = v;
      }
      base += s_total;
    }
    nnz = base;
    __syncthreads();
    li = nzi;
    lv = nzv;
  }
  bool all;
  const int n = vanilla_len(alen, row, fb_n, all);
  uint32_t* ids = aids + row * (int64_t)astride;
  float* prow = pre + row * (int64_t)astride;
  float* orow = post + row * (int64_t)astride;
  if (alen_out && blockIdx.y == 0 && threadIdx.x == 0) alen_out[row] = n;
  float lmax = -INFINITY;
  const int a0 = threadIdx.x + blockIdx.y * blockDim.x, astep = blockDim.x * gridDim.y;
  for (int a = a0; a < n; a += astep) {
    const uint32_t id = all ? (uint32_t)a : ids[a];
    if (all) ids[a] = id;
    float s = -0.0f;
    if (TRANS) {
      const float* w = W + id;
      for (int e = 0; e < nnz; ++e) s = __fadd_rn(s, __fmul_rn(w[(size_t)li[e] * nn], lv[e]));
    } else {
      const float* w = W + (size_t)id * dim;
      for (int e = 0; e < nnz; ++e) s = __fadd_rn(s, __fmul_rn(w[li[e]], lv[e]));
    }
    const float z = __fadd_rn(s, bias[id]);
    prow[a] = z;
    lmax = fmaxf(lmax, z);
  }
  if (act != KH_ACT_SOFTMAX) {
    for (int a = a0; a < n; a += astep) {
      const float z = prow[a];
      float r;
      if (act == KH_ACT_RELU) r = fmaxf(z, 0.0f);
      else if (act == KH_ACT_SIGMOID) r = sigmoid_ref(z);
      else if (act == KH_ACT_TANH) r = tanhf(z);
      else r = z;
      orow[a] = r;
    }
    return;
  }
  // softmax over the active set (layer.rs:286-308)
  lmax = wave_max(lmax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lmax;
  __syncthreads();
  float mx = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) mx = fmaxf(mx, red[i]);
  __syncthreads();
  float ls = 0.0f;
  for (int a = threadIdx.x; a < n; a += blockDim.x) {
    const float e = expf_glibc(prow[a] - mx);
    orow[a] = e;
    ls += e;
  }
  ls = wave_sum(ls);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ls;
  __syncthreads();
  float tot = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += red[i];
  if (tot > 0.0f) {
    for (int a = threadIdx.x; a < n; a += blockDim.x) orow[a] = orow[a] / tot;
  } else {
    const float u = 1.0f / (float)n;
    for (int a = threadIdx.x; a < n; a += blockDim.x) orow[a] = u;
  }
}

// Row-major layers over dense inputs of at most kTileMaxDim features (cfg5's
// output layer): each wave takes 64 active neurons at a time and loads their
// weight rows cooperatively, 32 lanes per 512-byte row (two whole rows per load
// instruction, instead of 64 scattered rows per instruction), into an LDS tile
// whose odd row stride makes the per-lane column reads conflict-free; lane j
// then runs neuron j's sequential sum over the input's nonzeros (ascending, as
// neuron_kernel does).  The next tile's loads are in flight during the sums.
constexpr int kTileN = 64;
constexpr int kTileStride = 129;   // floats per LDS row
constexpr int kTileMaxDim = 128;
constexpr int kTileWaves = kSlideThreads / 64;
constexpr size_t kTileLds = sizeof(float) * kTileWaves * kTileN * kTileStride;

__global__ __launch_bounds__(kSlideThreads) void neuron_tile_kernel(
    const float* __restrict__ W, const float* __restrict__ bias, int dim, const float* __restrict__ x,
    uint32_t* __restrict__ aids, int astride, const int32_t* __restrict__ alen, int act,
    float* __restrict__ pre, float* __restrict__ post, int fb_n = 0,
    int32_t* __restrict__ alen_out = nullptr) {
  extern __shared__ float tl[];
  __shared__ uint32_t nzi[kTileMaxDim];
  __shared__ float nzv[kTileMaxDim];
  __shared__ int wsum[kTileWaves];
  __shared__ int s_total;
  __shared__ float red[kTileWaves];
  const int64_t row = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the input's nonzeros in ascending order (dim <= kSlideThreads)
  {
    const float v = (int)threadIdx.x < dim ? x[row * (int64_t)dim + threadIdx.x] : 0.0f;
    const int nz = v != 0.0f ? 1 : 0;
    const int pos = block_excl_scan(nz, wsum, &s_total);
    if (nz) {
      nzi[pos] = threadIdx.x;
      nzv[pos] = v;
    }
  }
  __syncthreads();
  const int nnz = s_total;
  bool all;
  const int n = vanilla_len(alen, row, fb_n, all);
  uint32_t* ids = aids + row * (int64_t)astride;
  float* prow = pre + row * (int64_t)astride;
  float* orow = post + row * (int64_t)astride;
  if (alen_out && threadIdx.x == 0) alen_out[row] = n;
  if (all)
    for (int a = threadIdx.x; a < n; a += blockDim.x) ids[a] = (uint32_t)a;
  float* buf = tl + (size_t)wave * kTileN * kTileStride;
  const int q4 = dim >> 2;              // float4 per weight row (<= 32)
  const int c = lane & 31;              // this lane's float4 of a row
  const int half = lane >> 5;           // which of the two rows of a load
  const int ntiles = (n + kTileN - 1) / kTileN;
  float4 v[kTileN / 2];
  // rows of tile t: neuron t*64 + j for j < 64 (clamped to the last active id)
  auto issue = [&](int t) {
    const int ia = min(t * kTileN + lane, max(n - 1, 0));
    const uint32_t myid = all ? (uint32_t)ia : ids[ia];
#pragma unroll
    for (int r = 0; r < kTileN / 2; ++r) {
      const uint32_t id = (uint32_t)__shfl((int)myid, 2 * r + half);
      v[r] = reinterpret_cast<const float4*>(W + (size_t)id * dim)[min(c, q4 - 1)];
    }
  };
  float lmax = -INFINITY;
  int t = wave;
  if (t < ntiles) issue(t);
  for (; t < ntiles; t += kTileWaves) {
    // the tile to LDS (column 4c..4c+3 of row 2r + half)
    if (c < q4) {
#pragma unroll
      for (int r = 0; r < kTileN / 2; ++r) {
        float* dst = buf + (2 * r + half) * kTileStride + 4 * c;
        dst[0] = v[r].x;
        dst[1] = v[r].y;
        dst[2] = v[r].z;
        dst[3] = v[r].w;
      }
    }
    if (t + kTileWaves < ntiles) issue(t + kTileWaves);
    const int a = t * kTileN + lane;
    const float* wr = buf + lane * kTileStride;
    float s = -0.0f;
    for (int e = 0; e < nnz; ++e) s = __fadd_rn(s, __fmul_rn(wr[nzi[e]], nzv[e]));
    if (a < n) {
      const float z = __fadd_rn(s, bias[all ? (uint32_t)a : ids[a]]);
      prow[a] = z;
      lmax = fmaxf(lmax, z);
      if (act != KH_ACT_SOFTMAX) {
        float r;
        if (act == KH_ACT_RELU) r = fmaxf(z, 0.0f);
        else if (act == KH_ACT_SIGMOID) r = sigmoid_ref(z);
        else if (act == KH_ACT_TANH) r = tanhf(z);
        else r = z;
        orow[a] = r;
      }
    }
  }
  if (act != KH_ACT_SOFTMAX) return;
  // softmax over the active set (layer.rs:286-308), as neuron_kernel
  lmax = wave_max(lmax);
  if (lane == 0) red[wave] = lmax;
  __syncthreads();
  float mx = red[0];
  for (int i = 1; i < kTileWaves; ++i) mx = fmaxf(mx, red[i]);
  __syncthreads();
  float ls = 0.0f;
  for (int a = threadIdx.x; a < n; a += blockDim.x) {
    const float e = expf_glibc(prow[a] - mx);
    orow[a] = e;
    ls += e;
  }
  ls = wave_sum(ls);
  if (lane == 0) red[wave] = ls;
  __syncthreads();
  float tot = 0.0f;
  for (int i = 0; i < kTileWaves; ++i) tot += red[i];
  if (tot > 0.0f) {
    for (int a = threadIdx.x; a < n; a += blockDim.x) orow[a] = orow[a] / tot;
  } else {
    const float u = 1.0f / (float)n;
    for (int a = threadIdx.x; a < n; a += blockDim.x) orow[a] = u;
  }
}

// neuron_tile_kernel's LDS (above 64 KB) is allowed once per process.
static int tile_kernel_ready() {
  static std::once_flag once;
  static int rc = KH_OK;
  std::call_once(once, [] {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&neuron_tile_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTileLds) != hipSuccess)
      rc = KH_ERR_HIP;
  });
  return rc;
}

// Dense layer over CSR inputs: y[b][o] = act(sum_e val_e * W^T[idx_e][o] + bias[o]).
constexpr int kChainBatch = 16;  // entries in flight per sequential sum
__global__ __launch_bounds__(256) void dense_sparse_kernel(const float* __restrict__ WT, int n,
                                                           const float* __restrict__ bias,
                                                           const int64_t* __restrict__ xoff,
                                                           const uint32_t* __restrict__ xidx,
                                                           const float* __restrict__ xval,
                                                           int act, float* __restrict__ y) {
  const int64_t row = blockIdx.y;
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n) return;
  const int64_t a = xoff[row], b = xoff[row + 1];
  // kChainBatch entries at a time (indices, then the weight rows, all in
  // flight), then added in order: the sum stays sequential
  float s = -0.0f;
  for (int64_t e0 = a; e0 < b; e0 += kChainBatch) {
    uint32_t ix[kChainBatch];
    float xv[kChainBatch], wv[kChainBatch];
#pragma unroll
    for (int j = 0; j < kChainBatch; ++j) {
      const int64_t e = min(e0 + j, b - 1);
      ix[j] = xidx[e];
      xv[j] = xval[e];
    }
#pragma unroll
    for (int j = 0; j < kChainBatch; ++j) wv[j] = WT[(size_t)ix[j] * n + o];
#pragma unroll
    for (int j = 0; j < kChainBatch; ++j)
      if (e0 + j < b) s = __fadd_rn(s, __fmul_rn(xv[j], wv[j]));
  }
  const float z = __fadd_rn(s, bias[o]);
  float r;
  if (act == KH_ACT_RELU) r = fmaxf(z, 0.0f);
  else if (act == KH_ACT_SIGMOID) r = sigmoid_ref(z);
  else if (act == KH_ACT_TANH) r = tanhf(z);
  else r = z;
  y[row * (int64_t)n + o] = r;
}

int select_launch_with(const kh_lsh_index* idx, int sampling, int top_k, int threshold,
                       int num_neurons, const uint32_t* qids, const uint32_t* qcnt,
                       const int32_t* qlen, int qs, int64_t batch, uint32_t* aids, int as,
                       int32_t* alen, bool count_order, float* clear_dense, bool fallback,
                       hipStream_t st) {
  // A candidate's hit count is at most L * cap (every slot of its L buckets).
  const int nbins = idx->L * idx->cap + 1;
  KH_CHECK_ARG(sampling != KH_SAMPLING_TOPK || nbins <= kMaxCountBins,
               "top-k sampling supports num_tables * bucket_capacity <= %d", kMaxCountBins - 1);
  hipLaunchKernelGGL(select_kernel, dim3((unsigned)batch), dim3(kSlideThreads),
                     sampling == KH_SAMPLING_TOPK ? sizeof(unsigned) * nbins : 0, st, qids, qcnt,
                     qlen, qs, sampling, top_k, threshold, num_neurons, nbins, aids, as, alen,
                     count_order ? 1 : 0, clear_dense, fallback ? 1 : 0);
  KH_LAUNCHED();
  return KH_OK;
}

int select_launch(const kh_slide_layer* l, const uint32_t* qids, const uint32_t* qcnt,
                  const int32_t* qlen, int qs, int64_t batch, uint32_t* aids, int as, int32_t* alen,
                  bool count_order, float* clear_dense, hipStream_t st) {
  return select_launch_with(l->index, l->sampling, l->top_k, l->threshold, l->n, qids, qcnt, qlen,
                            qs, batch, aids, as, alen, count_order, clear_dense, true, st);
}

}  // namespace kh

using namespace kh;

struct kh_dense_layer {
  int dim = 0, n = 0, act = 0;
  float* wt = nullptr;  // [dim][n]
  float* bias = nullptr;
};

extern "C" int kh_slide_layer_create(int input_dim, int num_neurons, const float* w_host,
                                     const float* bias_host, kh_lsh_index* index, int sampling,
                                     int top_k, int threshold, int activation,
                                     kh_slide_layer** out) {
  KH_CHECK_ARG(out && w_host && bias_host && index, "null argument");
  KH_CHECK_ARG(input_dim > 0 && num_neurons > 0, "dims must be positive");
  KH_CHECK_ARG(index->h->dim == input_dim, "index input_dim %d != layer input_dim %d",
               index->h->dim, input_dim);
  KH_CHECK_ARG(sampling >= 0 && sampling <= 2 && activation >= 0 && activation <= 4,
               "bad sampling / activation");
  KH_CHECK_ARG(top_k >= 0 && threshold >= 0, "bad top_k / threshold");
  *out = nullptr;
  auto* l = new kh_slide_layer();
  l->dim = input_dim;
  l->n = num_neurons;
  l->index = index;
  l->sampling = sampling;
  l->top_k = top_k;
  l->threshold = threshold;
  l->act = activation;
  const size_t nw = (size_t)input_dim * num_neurons;
  l->w = static_cast<float*>(dev_alloc(sizeof(float) * nw));
  l->bias = static_cast<float*>(dev_alloc(sizeof(float) * num_neurons));
  uint32_t* ids = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * num_neurons));
  int rc = (l->w && l->bias && ids) ? KH_OK : KH_ERR_ALLOC;
  if (rc == KH_OK) {
    std::vector<uint32_t> h(num_neurons);
    for (int i = 0; i < num_neurons; ++i) h[i] = (uint32_t)i;
    if (hipMemcpy(l->w, w_host, sizeof(float) * nw, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(l->bias, bias_host, sizeof(float) * num_neurons, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ids, h.data(), sizeof(uint32_t) * num_neurons, hipMemcpyHostToDevice) != hipSuccess) {
      set_error("layer upload failed");
      rc = KH_ERR_HIP;
    }
  }
  // Transposed copy [dim][n] for the neuron kernel of non-softmax layers: the
  // lanes of a wave take ascending active ids, so one load instruction reads a
  // few adjacent cache lines of one input row instead of 64 weight rows.
  if (rc == KH_OK && activation != KH_ACT_SOFTMAX) {
    l->wtn = static_cast<float*>(dev_alloc(sizeof(float) * nw));
    if (!l->wtn) rc = KH_ERR_ALLOC;
    if (rc == KH_OK) {
      hipLaunchKernelGGL(transpose_kernel<float>, dim3(ceil_div(input_dim, 32), ceil_div(num_neurons, 32)),
                         dim3(256), 0, 0, l->w, num_neurons, input_dim, l->wtn);
      if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        set_error("layer transpose failed");
        rc = KH_ERR_HIP;
      }
    }
  }
  // Layer::new inserts neurons 0..n-1 in order (layer.rs:42-44).
  if (rc == KH_OK) rc = kh_lsh_index_insert(index, ids, l->w, num_neurons, input_dim, nullptr);
  dev_free(ids);
  if (rc != KH_OK) {
    kh_slide_layer_destroy(l);
    return rc;
  }
  *out = l;
  return KH_OK;
}

extern "C" int kh_slide_layer_destroy(kh_slide_layer* l) {
  if (!l) return KH_OK;
  dev_free(l->w);
  dev_free(l->wtn);
  dev_free(l->bias);
  l->free_opt();
  delete l;
  return KH_OK;
}

// Sampling as a SparseInferenceEngine call makes it (bolt/sparse_inference.rs):
// top-k by count in the sampler's order, no all-neurons fallback, and its own
// activation.
struct SelectOverride {
  int top_k;
  int act;
};

static int slide_forward_common(const kh_slide_layer* lc, const float* x, const int64_t* xoff,
                                const uint32_t* xidx, const float* xval, int64_t batch,
                                int64_t* off, uint32_t* act_ids, float* pre_out, float* act_out,
                                int64_t capacity, hipStream_t st,
                                const SelectOverride* ov = nullptr) {
  const kh_slide_layer* l = lc;
  const kh_lsh_index* idx = l->index;
  const int L = idx->L;
  WsSet* w = l->ws.get(st);
  uint32_t* codes = static_cast<uint32_t*>(w->get(0, sizeof(uint32_t) * batch * L));
  // Vanilla sampling with every indexed id below the layer's neuron count
  // keeps the whole query result (layer.rs:65-90), so the neuron kernel reads
  // it directly and applies the empty-set fallback itself: no select launch.
  const bool direct = !ov && l->sampling == KH_SAMPLING_VANILLA && idx->id_bound <= (uint32_t)l->n;
  const int qs = direct ? std::max(query_stride(idx), l->n) : query_stride(idx);
  uint32_t* qids = static_cast<uint32_t*>(w->get(1, sizeof(uint32_t) * batch * qs));
  uint32_t* qcnt = static_cast<uint32_t*>(w->get(2, sizeof(uint32_t) * batch * qs));
  int32_t* qlen = static_cast<int32_t*>(w->get(3, sizeof(int32_t) * batch));
  const int as = std::max(qs, l->n);
  uint32_t* aids = static_cast<uint32_t*>(w->get(4, sizeof(uint32_t) * batch * as));
  int32_t* alen = static_cast<int32_t*>(w->get(5, sizeof(int32_t) * batch));
  float* pre = static_cast<float*>(w->get(6, sizeof(float) * batch * as));
  float* post = static_cast<float*>(w->get(7, sizeof(float) * batch * as));
  if (!codes || !qids || !qcnt || !qlen || !aids || !alen || !pre || !post) return KH_ERR_ALLOC;
  int rc = xoff ? hash_sparse_launch(idx->h, xoff, xidx, xval, batch, codes, st)
                : hash_dense_launch(idx->h, x, l->dim, batch, codes, st);
  if (rc != KH_OK) return rc;
  rc = query_launch(idx, codes, batch, qids, direct ? nullptr : qcnt, qs, qlen, st);
  if (rc != KH_OK) return rc;
  if (direct)
    aids = qids;  // stride qs == as
  else
    rc = ov ? select_launch_with(l->index, KH_SAMPLING_TOPK, ov->top_k, 0, l->n, qids, qcnt, qlen, qs,
                                 batch, aids, as, alen, true, nullptr, false, st)
            : select_launch(l, qids, qcnt, qlen, qs, batch, aids, as, alen, false, nullptr, st);
  if (rc != KH_OK) return rc;
  const int act = ov ? ov->act : l->act;
  const int max_nz = xoff ? 4096 : l->dim;
  KH_CHECK_ARG(xoff || l->dim <= 8192, "dense SLIDE input supports input_dim <= 8192");
  const size_t lds = (sizeof(uint32_t) + sizeof(float)) * max_nz;
  // Without softmax the active ids of a sample are split over kNeuronSplit
  // blocks (softmax needs the whole row's max and sum in one block).
  constexpr int kNeuronSplit = 4;
  const dim3 ng((unsigned)batch, l->wtn ? kNeuronSplit : 1);
  // direct: the candidate lengths come from the query, the fallback is the
  // kernel's, and the kernel writes the lengths the outputs use
  const int32_t* ilen = direct ? qlen : alen;
  const int fb_n = direct ? l->n : 0;
  int32_t* olen = direct ? alen : nullptr;
  if (xoff && l->wtn)
    hipLaunchKernelGGL((neuron_kernel<true, true>), ng, dim3(kSlideThreads), lds, st, l->wtn, l->n,
                       l->bias, l->dim, nullptr, xoff, xidx, xval, aids, as, ilen, act, max_nz,
                       pre, post, fb_n, olen);
  else if (xoff)
    hipLaunchKernelGGL((neuron_kernel<true, false>), ng, dim3(kSlideThreads), lds, st, l->w, l->n,
                       l->bias, l->dim, nullptr, xoff, xidx, xval, aids, as, ilen, act, max_nz,
                       pre, post, fb_n, olen);
  else if (l->wtn)
    hipLaunchKernelGGL((neuron_kernel<false, true>), ng, dim3(kSlideThreads), lds, st, l->wtn, l->n,
                       l->bias, l->dim, x, nullptr, nullptr, nullptr, aids, as, ilen, act,
                       max_nz, pre, post, fb_n, olen);
  else if (l->dim <= kTileMaxDim && l->dim % 4 == 0 && tile_kernel_ready() == KH_OK)
    hipLaunchKernelGGL(neuron_tile_kernel, dim3((unsigned)batch), dim3(kSlideThreads), kTileLds, st, l->w,
                       l->bias, l->dim, x, aids, as, ilen, act, pre, post, fb_n, olen);
  else
    hipLaunchKernelGGL((neuron_kernel<false, false>), ng, dim3(kSlideThreads), lds, st, l->w, l->n,
                       l->bias, l->dim, x, nullptr, nullptr, nullptr, aids, as, ilen, act,
                       max_nz, pre, post, fb_n, olen);
  KH_LAUNCHED();
  return csr_finish(aids, nullptr, pre, post, as, alen, batch, off, act_ids, nullptr, pre_out,
                    act_out, capacity, st);
}

extern "C" int kh_slide_layer_forward(const kh_slide_layer* l, const float* x_dev, int64_t batch,
                                      int64_t* off_dev, uint32_t* act_ids_dev, float* pre_dev,
                                      float* act_dev, int64_t capacity, void* stream) {
  KH_CHECK_ARG(l && off_dev && act_ids_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && capacity >= 0, "bad batch/capacity");
  hipStream_t st = as_stream(stream);
  if (batch == 0) {
    KH_HIP(hipMemsetAsync(off_dev, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  KH_CHECK_ARG(x_dev != nullptr, "null input");
  return slide_forward_common(l, x_dev, nullptr, nullptr, nullptr, batch, off_dev, act_ids_dev,
                              pre_dev, act_dev, capacity, st);
}

extern "C" int kh_slide_layer_forward_sparse(const kh_slide_layer* l, const int64_t* xoff_dev,
                                             const uint32_t* xidx_dev, const float* xval_dev,
                                             int64_t batch, int64_t* off_dev,
                                             uint32_t* act_ids_dev, float* pre_dev, float* act_dev,
                                             int64_t capacity, void* stream) {
  KH_CHECK_ARG(l && off_dev && act_ids_dev && xoff_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && capacity >= 0, "bad batch/capacity");
  hipStream_t st = as_stream(stream);
  if (batch == 0) {
    KH_HIP(hipMemsetAsync(off_dev, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  return slide_forward_common(l, nullptr, xoff_dev, xidx_dev, xval_dev, batch, off_dev,
                              act_ids_dev, pre_dev, act_dev, capacity, st);
}

extern "C" int kh_sparse_inference(const kh_slide_layer* l, const float* x_dev, int64_t batch,
                                   int64_t base_top_k, float sparsity_multiplier, int relu,
                                   int64_t* off_dev, uint32_t* ids_dev, float* act_dev,
                                   int64_t capacity, void* stream) {
  KH_CHECK_ARG(l && off_dev && ids_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && capacity >= 0 && base_top_k >= 0,
               "bad batch/capacity/top_k");
  hipStream_t st = as_stream(stream);
  if (batch == 0) {
    KH_HIP(hipMemsetAsync(off_dev, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  KH_CHECK_ARG(x_dev != nullptr, "null input");
  // (base_top_k as f32 * multiplier) as usize: f32 product, truncated,
  // saturating (NaN and negatives give 0)
  const float ek = static_cast<float>(base_top_k) * sparsity_multiplier;
  const int64_t eff = !(ek > 0.0f) ? 0 : (ek >= 2147483647.0f ? 0x7fffffff : static_cast<int64_t>(ek));
  SelectOverride ov{static_cast<int>(eff), relu ? KH_ACT_RELU : KH_ACT_IDENTITY};
  return slide_forward_common(l, x_dev, nullptr, nullptr, nullptr, batch, off_dev, ids_dev, nullptr,
                              act_dev, capacity, st, &ov);
}

extern "C" int kh_lsh_index_query_top_k(const kh_lsh_index* idx, const float* x_dev, int64_t batch,
                                        int64_t top_k, uint32_t* ids_dev, int32_t* n_dev,
                                        void* stream) {
  KH_CHECK_ARG(idx && n_dev && (ids_dev || top_k == 0), "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && top_k >= 0 && top_k <= 0x7fffffff, "bad batch/top_k");
  if (batch == 0) return KH_OK;
  KH_CHECK_ARG(x_dev != nullptr, "null input");
  hipStream_t st = as_stream(stream);
  WsSet* w = idx->ws.get(st);
  const int L = idx->L;
  const int qs = query_stride(idx);
  uint32_t* codes = static_cast<uint32_t*>(w->get(4, sizeof(uint32_t) * batch * L));
  uint32_t* qids = static_cast<uint32_t*>(w->get(5, sizeof(uint32_t) * batch * qs));
  uint32_t* qcnt = static_cast<uint32_t*>(w->get(6, sizeof(uint32_t) * batch * qs));
  int32_t* qlen = static_cast<int32_t*>(w->get(7, sizeof(int32_t) * batch));
  if (!codes || !qids || !qcnt || !qlen) return KH_ERR_ALLOC;
  int rc = hash_dense_launch(idx->h, x_dev, idx->h->dim, batch, codes, st);
  if (rc == KH_OK) rc = query_launch(idx, codes, batch, qids, qcnt, qs, qlen, st);
  if (rc != KH_OK) return rc;
  // count descending, then id, straight into the caller's [batch][top_k]
  // rows: the count-order selection writes only positions below
  // min(top_k, candidates)
  const int k = static_cast<int>(std::min<int64_t>(top_k, qs));
  return select_launch_with(idx, KH_SAMPLING_TOPK, k, 0, 0x7fffffff, qids, qcnt, qlen, qs, batch, ids_dev,
                            static_cast<int>(top_k), n_dev, true, nullptr, false, st);
}

extern "C" int kh_dense_layer_create(int input_dim, int num_neurons, const float* w_host,
                                     const float* bias_host, int activation,
                                     kh_dense_layer** out) {
  KH_CHECK_ARG(out && w_host && bias_host, "null argument");
  KH_CHECK_ARG(input_dim > 0 && num_neurons > 0 && activation >= 0 && activation <= 4 &&
                   activation != KH_ACT_SOFTMAX,
               "bad dims / activation (softmax is not supported on a dense layer)");
  *out = nullptr;
  auto* l = new kh_dense_layer();
  l->dim = input_dim;
  l->n = num_neurons;
  l->act = activation;
  const size_t nw = (size_t)input_dim * num_neurons;
  std::vector<float> wt(nw);
  for (int o = 0; o < num_neurons; ++o)
    for (int d = 0; d < input_dim; ++d) wt[(size_t)d * num_neurons + o] = w_host[(size_t)o * input_dim + d];
  l->wt = static_cast<float*>(dev_alloc(sizeof(float) * nw));
  l->bias = static_cast<float*>(dev_alloc(sizeof(float) * num_neurons));
  if (!l->wt || !l->bias) {
    kh_dense_layer_destroy(l);
    return KH_ERR_ALLOC;
  }
  if (hipMemcpy(l->wt, wt.data(), sizeof(float) * nw, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(l->bias, bias_host, sizeof(float) * num_neurons, hipMemcpyHostToDevice) != hipSuccess) {
    set_error("dense layer upload failed");
    kh_dense_layer_destroy(l);
    return KH_ERR_HIP;
  }
  *out = l;
  return KH_OK;
}

extern "C" int kh_dense_layer_destroy(kh_dense_layer* l) {
  if (!l) return KH_OK;
  dev_free(l->wt);
  dev_free(l->bias);
  delete l;
  return KH_OK;
}

extern "C" int kh_dense_layer_forward_sparse(const kh_dense_layer* l, const int64_t* xoff_dev,
                                             const uint32_t* xidx_dev, const float* xval_dev,
                                             int64_t batch, float* y_dev, void* stream) {
  KH_CHECK_ARG(l && xoff_dev && y_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 65535, "bad batch");
  if (batch == 0) return KH_OK;
  hipLaunchKernelGGL(dense_sparse_kernel, dim3(ceil_div(l->n, 256), (unsigned)batch), dim3(256), 0,
                     as_stream(stream), l->wt, l->n, l->bias, xoff_dev, xidx_dev, xval_dev, l->act,
                     y_dev);
  KH_LAUNCHED();
  return KH_OK;
}
