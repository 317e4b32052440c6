// attention.hip -- head-sparse decode attention (gfx950).
//
// Replaces sparse_attention::forward_sparse
// (crates/klearu-llm/src/sparse/sparse_attention.rs:7-95) together with
// KvCache::append (model/kv_cache.rs:33-48), RotaryEmbedding (model/rope.rs:17-87)
// and Linear::forward (model/linear.rs:79-104) for q/k/v/o_proj.
//
// HBM layout (written once at create):
//   Wkvq [2*kvd + nh*D][hidden] BF16   K rows, V rows, then Q rows head by head
//   WoT  [nh*D][hidden]        BF16    o_proj transposed: the columns of head h
//                                      are the contiguous rows h*D .. h*D+D-1
//   K, V cache [max_batch][nkv][max_seq][D]  BF16 (default) or f32; all positions
//                                      of one kv head are contiguous, so one
//                                      (token, head) reads 2*len*D*elt bytes
//   cos, sin [max_seq][D/2] f32        rope.rs:23-37, computed with the host libm
//   len [max_batch] int32              cache lengths, advanced by every step
//
// One decode step of `batch` sequences, each with its own selected heads:
//   attn_qkv      one wave per row of Wkvq for every token (tokens staged in LDS):
//                 every K and V row (the cache takes every kv head, :39) and the
//                 Q rows of heads that some token selected; its last block writes
//                 the union of selected heads as the row list of the o_proj gather.
//   attn_decode   split-K over cache positions (a chunk per block) for every
//                 (token, selected head): RoPE on q and on the current k, scores
//                 from 16-byte K loads, chunk max / exp-sum and the un-normalised
//                 V sum.  The current position's K/V come from this step's f32
//                 projections, so the step sees them unrounded as the reference does.
//                 One extra row of blocks appends this step's roped K and V to the
//                 cache and zero-fills the union heads a token did not select (the
//                 reference's zero-filled attn_concat, :44).
//   attn_merge    merges the chunks of each (token, selected head) into the head
//                 output, in union order (batch > 2, or head lists longer than
//                 kOprojMaxSel; otherwise attn_oproj merges the chunks of its rows).
//   attn_oproj (or gather_rows) + partials_reduce (gather.hpp)
//                 o_proj over the union heads' WoT rows only; the reduce advances
//                 each sequence's cache length once its output is complete.
// Bytes per token at 7B shape (hidden 4096, 32 heads x 128, 16 selected, len
// 2048, BF16 cache): K/V rows 2*4096*4096*2 = 64 MiB, Q rows 16 MiB, o_proj
// 16 MiB, cache 16*2048*128*2*2 = 16 MiB.
//
// Parity: q/k/v/o projections and the softmax sums use a different (parallel)
// summation order from the reference's AVX2 dot and sequential loops, so
// outputs agree to rounding (BF16-weight tolerance), not bit for bit.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "gather.hpp"
#include "mfma.hpp"
#include "pred_l1.hpp"

namespace kh {

constexpr int kAttnThreads = 256;
constexpr int kAttnPasses = 8;      // cache rows per thread per chunk (K and V loads in flight)
constexpr int kQkvWaves = 8;        // rows per projection block
constexpr int kQkvChunks = 8;       // 16-byte chunks per lane in flight (hidden <= 4096 per pass)
constexpr int kQkvTok = 4;          // tokens staged in LDS at a time
constexpr int kMaxAttnHeads = 1024;

// RotaryEmbedding::apply (rope.rs:75-87) for element i of a head vector x:
// x[i] = x0*cos - x1*sin and x[half+i] = x1*cos + x0*sin, products rounded
// separately (no FMA contraction in this build).
template <int HALF>
__device__ __forceinline__ float rope_elem(const float* __restrict__ x, const float* __restrict__ c,
                                           const float* __restrict__ s, int i) {
  if (i < HALF) return x[i] * c[i] - x[i + HALF] * s[i];
  const int k = i - HALF;
  return x[i] * c[k] + x[k] * s[k];
}

__device__ __forceinline__ void widen16(const uint4& v, float* f, uint16_t) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}
__device__ __forceinline__ void widen16(const uint4& v, float* f, float) {
  f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
  f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
}
__device__ __forceinline__ void store_kv(uint16_t* p, float v) { *p = f32_to_bf16(v); }
__device__ __forceinline__ void store_kv(float* p, float v) { *p = v; }

// The union of selected heads in ascending order -> rows h*D + r of WoT
// (qrows, their count in *nqrows) and each head's union rank (urank, -1 for
// heads no token selected).  Block-wide; s_flag and s_uh hold nh ints each.
__device__ void qkv_plan(const int32_t* __restrict__ heads, int nent, int nh, int D,
                         int32_t* __restrict__ qrows, int32_t* __restrict__ nqrows,
                         int32_t* __restrict__ urank, int* s_flag, int* s_uh, int* wsum,
                         int* s_total) {
  for (int h = threadIdx.x; h < nh; h += blockDim.x) s_flag[h] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < nent; i += blockDim.x) {
    const int h = heads[i];
    if (h >= 0 && h < nh) s_flag[h] = 1;
  }
  __syncthreads();
  int base = 0;
  for (int h0 = 0; h0 < nh; h0 += blockDim.x) {
    const int h = h0 + threadIdx.x;
    const int f = h < nh ? s_flag[h] : 0;
    const int u = block_excl_scan(f, wsum, s_total) + base;
    if (f) s_uh[u] = h;
    if (h < nh) urank[h] = f ? u : -1;
    base += *s_total;
  }
  __syncthreads();
  const int nq = base * D;
  for (int i = threadIdx.x; i < nq; i += blockDim.x) qrows[i] = s_uh[i / D] * D + i % D;
  if (threadIdx.x == 0) *nqrows = nq;
}

// The head selection of one row (sparse_attention.rs:14-24): the head
// predictor's layer 2 over its layer-1 outputs hpred (mlp_predictor.rs:114-124,
// the same chain as pred_l2_kernel) and the top k of its nh <= 64 scores,
// computed by wave 0 of the block: s_hsel[h] = 1 for a selected head, s_heads
// the k selected heads in ascending order.  phid <= kAttnSelHid.
template <typename PW>
__device__ __forceinline__ void attn_select_heads(const PW* __restrict__ w2, const float* __restrict__ b2,
                                                  const float* __restrict__ hpred, int phid, int nh, int k,
                                                  float* s_hp, uint64_t* s_tab, int* s_hsel,
                                                  int32_t* s_heads) {
  using V = typename Blk8<PW>::V;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int oc = min(lane, nh - 1);
  V w[kAttnSelHid / 8];
  float bv = 0.0f;
  if (wave == 0) {
    l2_load<PW, kAttnSelHid>(w2, phid, nh, oc, w);
    bv = b2[oc];
  }
  for (int i = threadIdx.x; i < phid; i += blockDim.x) s_hp[i] = hpred[i];
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  if (wave == 0) {
    const float score = sigmoid_ref_t(__fadd_rn(l2_chain<PW, kAttnSelHid>(w, phid, s_hp), bv), s_tab);
    const bool ok = lane < nh;
    const int rank = l2_wave_rank(f32_key(score), lane, nh);
    const bool sel = ok && rank < min(k, nh);
    const uint64_t bal = __ballot(sel);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
    if (ok) s_hsel[lane] = sel ? 1 : 0;
    if (sel) s_heads[below] = lane;
  }
  __syncthreads();
}

// The head selections of rows 0 .. batch-1 as attn_select_heads, one row per
// wave (rows w, w + waves, ...) over the head predictor's layer-1 outputs
// hpred[batch][phid]: s_any[h] = 1 when some row selected head h, s_heads[b k
// + i] the k heads of row b in ascending order.  s_hp holds batch rows of
// kSelHs floats.  The block copies W2 (blocked [ceil(phid/8)][nh][8]) to s_w2
// once and every wave reads its lanes' rows from there: many blocks run the
// same selection, and per-wave reads of W2 from global memory would all hit
// the same few L2 lines.  Every wave of the block takes part.
constexpr int kSelHs = kAttnSelHid + 4 * kL2Hw;
template <typename PW>
__device__ __forceinline__ void attn_select_heads_rows(const PW* __restrict__ w2, const float* __restrict__ b2,
                                                       const float* __restrict__ hpred, int phid, int nh, int k,
                                                       int batch, float* s_hp, uint64_t* s_tab, int* s_any,
                                                       int32_t* s_heads, typename Blk8<PW>::V* s_w2) {
  using B8 = Blk8<PW>;
  using V = typename B8::V;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int oc = min(lane, nh - 1);
  const int nblk = (phid + 7) >> 3;
  const V* __restrict__ wv = reinterpret_cast<const V*>(w2);
  for (int i = threadIdx.x; i < nblk * nh; i += blockDim.x) s_w2[i] = wv[i];
  const float bv = b2[oc];
  for (int i = threadIdx.x; i < batch * phid; i += blockDim.x) {
    const int b = i / phid;
    s_hp[b * kSelHs + (i - b * phid)] = hpred[i];
  }
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  if (threadIdx.x < 64) s_any[threadIdx.x] = 0;
  __syncthreads();
  V w[kAttnSelHid / 8];
#pragma unroll
  for (int jb = 0; jb < kAttnSelHid / 8; ++jb) w[jb] = jb < nblk ? s_w2[jb * nh + oc] : B8::zero();
  for (int b = wave; b < batch; b += nw) {
    const float score = sigmoid_ref_t(__fadd_rn(l2_chain<PW, kAttnSelHid>(w, phid, s_hp + b * kSelHs), bv), s_tab);
    const bool ok = lane < nh;
    const int rank = l2_wave_rank(f32_key(score), lane, nh);
    const bool sel = ok && rank < min(k, nh);
    const uint64_t bal = __ballot(sel);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
    if (sel) {
      s_heads[b * k + below] = lane;
      s_any[lane] = 1;  // several waves may write the same 1
    }
  }
  __syncthreads();
}

// y[b][row] = Wkvq[row] . x[b] for the K/V rows and the Q rows of selected
// heads, rows from row_base on (kvrows: the K/V rows were projected already).
// The grid has one extra (last) block that writes the o_proj row list.
// NORM (batch 1): x is the un-normalised hidden row and RmsNorm (weight nw) is
// applied while staging it, with the exact scale at norm_inv (written by the
// head predictor's layer 1 for this row).
template <int NB, bool NORM = false>
__global__ __launch_bounds__(64 * kQkvWaves) void attn_qkv_kernel(
    const uint16_t* __restrict__ W, const float* __restrict__ x, int batch, int H, int kvrows,
    int D, int nh, const int32_t* __restrict__ heads, int nsel, float* __restrict__ y,
    int ystride, int32_t* __restrict__ qrows, int32_t* __restrict__ nqrows,
    int32_t* __restrict__ urank, const float* __restrict__ nw,
    const float* __restrict__ norm_inv, int row_base) {
  extern __shared__ float4 xs4[];  // [kQkvTok][H/4]; the plan block's flags / union list
  __shared__ int wsum[kQkvWaves];
  __shared__ int s_total;
  const int nent = batch * nsel;
  if (blockIdx.x == gridDim.x - 1) {
    int* s_flag = reinterpret_cast<int*>(xs4);
    qkv_plan(heads, nent, nh, D, qrows, nqrows, urank, s_flag, s_flag + nh, wsum, &s_total);
    return;
  }
  {
    const int row0 = row_base + blockIdx.x * kQkvWaves;
    if (row0 >= kvrows) {
      // Q rows of head h (D is a multiple of kQkvWaves): skip unless selected.
      const int h = (row0 - kvrows) / D;
      int any = 0;
      for (int i = threadIdx.x; i < nent; i += blockDim.x) any |= heads[i] == h;
      if (!__syncthreads_or(any)) return;
    }
  }
  const int row0 = row_base + blockIdx.x * kQkvWaves;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = row0 + wave;
  const uint4* __restrict__ w = reinterpret_cast<const uint4*>(W + (size_t)row * H);
  const int nchunk = H >> 3, H4 = H >> 2;
  constexpr int TB = NB < kQkvTok ? NB : kQkvTok;
  if constexpr (NORM) {
    // One token, H <= 4096 (one pass, no loop): the row, the norm weights and
    // the scale are requested first, then the weight row; the norm is formed
    // while the weights stream in (loads complete in issue order).
    constexpr int kXq = 4096 / 4 / (64 * kQkvWaves);
    float4 xv[kXq], wn[kXq];
#pragma unroll
    for (int q = 0; q < kXq; ++q) {
      const int i = min((int)threadIdx.x + q * 64 * kQkvWaves, H4 - 1);
      xv[q] = reinterpret_cast<const float4*>(x)[i];
      wn[q] = reinterpret_cast<const float4*>(nw)[i];
    }
    const float inv = *norm_inv;
    uint4 wv[kQkvChunks];
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) wv[q] = ld_stream(w + min(lane + 64 * q, nchunk - 1));
    __builtin_amdgcn_sched_barrier(0);
    // RmsNorm (model/rms_norm.rs:56-60): (x * inv) * w
#pragma unroll
    for (int q = 0; q < kXq; ++q) {
      float4 v = xv[q];
      v.x = __fmul_rn(__fmul_rn(v.x, inv), wn[q].x);
      v.y = __fmul_rn(__fmul_rn(v.y, inv), wn[q].y);
      v.z = __fmul_rn(__fmul_rn(v.z, inv), wn[q].z);
      v.w = __fmul_rn(__fmul_rn(v.w, inv), wn[q].w);
      xs4[min((int)threadIdx.x + q * 64 * kQkvWaves, H4 - 1)] = v;  // clamped (see stage_f4)
    }
    lds_barrier();
    // branch-free (a branch here lets the compiler sink each weight load to its
    // use): chunks past the row add zero weights times a valid x
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) {
      const int c = lane + 64 * q;
      const int cc = min(c, nchunk - 1);
      float wf[8];
      widen16(wv[q], wf, uint16_t());
#pragma unroll
      for (int e = 0; e < 8; ++e) wf[e] = c < nchunk ? wf[e] : 0.0f;
      const float4 x0 = xs4[2 * cc], x1 = xs4[2 * cc + 1];
      a = fmaf(wf[0], x0.x, a); a = fmaf(wf[1], x0.y, a);
      a = fmaf(wf[2], x0.z, a); a = fmaf(wf[3], x0.w, a);
      a = fmaf(wf[4], x1.x, a); a = fmaf(wf[5], x1.y, a);
      a = fmaf(wf[6], x1.z, a); a = fmaf(wf[7], x1.w, a);
    }
    const float sum = wave_sum(a);
    if (lane == 0) y[row] = sum;
    return;
  }
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
  for (int cbase = 0; cbase < nchunk; cbase += 64 * kQkvChunks) {
    uint4 wv[kQkvChunks];
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) wv[q] = ld_stream(w + min(cbase + lane + 64 * q, nchunk - 1));
#pragma unroll
    for (int t0 = 0; t0 < NB; t0 += TB) {
      if (t0 >= batch) break;
      lds_barrier();
      const int nt = min(TB, batch - t0);
      stage_f4(xs4, reinterpret_cast<const float4*>(x + (size_t)t0 * H), nt * H4);
      lds_barrier();
#pragma unroll
      for (int q = 0; q < kQkvChunks; ++q) {
        const int c = cbase + lane + 64 * q;
        if (c >= nchunk) break;
        float wf[8];
        widen16(wv[q], wf, uint16_t());
#pragma unroll
        for (int t = 0; t < TB; ++t) {
          if (t < nt) {
            const float4 x0 = xs4[t * H4 + 2 * c], x1 = xs4[t * H4 + 2 * c + 1];
            float a = acc[t0 + t];
            a = fmaf(wf[0], x0.x, a); a = fmaf(wf[1], x0.y, a);
            a = fmaf(wf[2], x0.z, a); a = fmaf(wf[3], x0.w, a);
            a = fmaf(wf[4], x1.x, a); a = fmaf(wf[5], x1.y, a);
            a = fmaf(wf[6], x1.z, a); a = fmaf(wf[7], x1.w, a);
            acc[t0 + t] = a;
          }
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < batch) {
      const float s = wave_sum(acc[b]);
      if (lane == 0) y[(size_t)b * ystride + row] = s;
    }
  }
}

// The head predictor's layer 1 and the K/V projections of one decode step
// in one launch.  Every kv head is appended to the cache whatever heads the
// predictor picks (sparse_attention.rs:26-40), so the K and V rows do not
// wait for the selection: blocks [0, nl1) run layer 1 (pred_l1.hpp: exact
// RmsNorm, exact chains; one block per CU, which leaves most CUs idle for
// about 15 us at the 7B shape), the others stream the 2*kvd K/V rows of Wkvq
// meanwhile.  The launch's LDS request (kL1LdsBytes) keeps one block per CU,
// so no projection wave shares a CU with a chain.  A K/V block applies
// RmsNorm with its own scale from an f32 tree sum of the squares: the
// projected rows carry tolerance anyway (their dot products use a parallel
// order), and the scale stays within a few ulps of the exact one, which only
// the selection needs bit for bit.  Row r of wave w of block kb: rows gw,
// gw + nwaves, ... with gw = kb*8 + w, one 8 KB weight row per wave in flight
// ahead of the one being added.
template <typename W>
__global__ __launch_bounds__(kL1LdsThreads) void attn_pred_kv_kernel(
    const W* __restrict__ w1, const float* __restrict__ b1, int hid, float* __restrict__ hbuf,
    const float* __restrict__ x, int H, const float* __restrict__ nw, float* __restrict__ inv_out,
    float eps, const uint16_t* __restrict__ wkvq, int kvrows, float* __restrict__ y, int nl1) {
  extern __shared__ float4 lds4[];
  if ((int)blockIdx.x < nl1) {
    pred_l1_lds_body<W>(blockIdx.x, 0, w1, b1, x, H, hid, hbuf, nw, inv_out, eps, lds4);
    return;
  }
  static_assert(kL1LdsThreads == 64 * kQkvWaves, "one projection row per wave");
  float* red = reinterpret_cast<float*>(lds4 + 1024);  // [kQkvWaves], after xn (H <= 4096)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = ((int)gridDim.x - nl1) * kQkvWaves;
  const int gw = ((int)blockIdx.x - nl1) * kQkvWaves + wave;
  const int nchunk = H >> 3, H4 = H >> 2;
  // the row and the norm weights first, then the first weight row
  constexpr int kXq = 4096 / 4 / (64 * kQkvWaves);
  float4 xv[kXq], wn[kXq];
#pragma unroll
  for (int q = 0; q < kXq; ++q) {
    const int i = min((int)threadIdx.x + q * 64 * kQkvWaves, H4 - 1);
    xv[q] = reinterpret_cast<const float4*>(x)[i];
    wn[q] = reinterpret_cast<const float4*>(nw)[i];
  }
  int row = gw;
  uint4 wv[kQkvChunks];
  {
    const uint4* __restrict__ w = reinterpret_cast<const uint4*>(wkvq + (size_t)min(row, kvrows - 1) * H);
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) wv[q] = ld_stream(w + min(lane + 64 * q, nchunk - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  // sum of squares: per thread, per wave, then the waves in order
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < kXq; ++q)
    if ((int)threadIdx.x + q * 64 * kQkvWaves < H4)
      ss += (xv[q].x * xv[q].x + xv[q].y * xv[q].y) + (xv[q].z * xv[q].z + xv[q].w * xv[q].w);
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  lds_barrier();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kQkvWaves; ++i) tot += red[i];
  const float inv = rms_inv_exact(tot, H, eps);
#pragma unroll
  for (int q = 0; q < kXq; ++q) {
    float4 v = xv[q];
    v.x = __fmul_rn(__fmul_rn(v.x, inv), wn[q].x);
    v.y = __fmul_rn(__fmul_rn(v.y, inv), wn[q].y);
    v.z = __fmul_rn(__fmul_rn(v.z, inv), wn[q].z);
    v.w = __fmul_rn(__fmul_rn(v.w, inv), wn[q].w);
    lds4[min((int)threadIdx.x + q * 64 * kQkvWaves, H4 - 1)] = v;  // clamped (see stage_f4)
  }
  lds_barrier();
  const float4* xs4 = lds4;
  for (; row < kvrows; row += nwaves) {
    // the next row's weights go out before this row's products (the last
    // iteration re-reads its own row, unused)
    uint4 nv[kQkvChunks];
    const int nrow = min(row + nwaves, kvrows - 1);
    const uint4* __restrict__ w = reinterpret_cast<const uint4*>(wkvq + (size_t)nrow * H);
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) nv[q] = ld_stream(w + min(lane + 64 * q, nchunk - 1));
    __builtin_amdgcn_sched_barrier(0);
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) {
      const int c = lane + 64 * q;
      const int cc = min(c, nchunk - 1);
      float wf[8];
      widen16(wv[q], wf, uint16_t());
#pragma unroll
      for (int e = 0; e < 8; ++e) wf[e] = c < nchunk ? wf[e] : 0.0f;
      const float4 x0 = xs4[2 * cc], x1 = xs4[2 * cc + 1];
      a = fmaf(wf[0], x0.x, a); a = fmaf(wf[1], x0.y, a);
      a = fmaf(wf[2], x0.z, a); a = fmaf(wf[3], x0.w, a);
      a = fmaf(wf[4], x1.x, a); a = fmaf(wf[5], x1.y, a);
      a = fmaf(wf[6], x1.z, a); a = fmaf(wf[7], x1.w, a);
    }
    const float sum = wave_sum(a);
    if (lane == 0) y[row] = sum;
#pragma unroll
    for (int q = 0; q < kQkvChunks; ++q) wv[q] = nv[q];
  }
}

// RmsNorm's output of four elements: (v * inv) * w, each product rounded
// (rms_norm.rs:53-63, the same products as the layer-1 block body's).
__device__ __forceinline__ float4 rms_apply4(const float4& v, float inv, const float4& w) {
  return make_float4(__fmul_rn(__fmul_rn(v.x, inv), w.x), __fmul_rn(__fmul_rn(v.y, inv), w.y),
                     __fmul_rn(__fmul_rn(v.z, inv), w.z), __fmul_rn(__fmul_rn(v.w, inv), w.w));
}

// Batched q/k/v projections (2..16 tokens) on the matrix cores.  A block
// takes 16*T rows (T 16-row tiles per wave sharing the x operand), each of its
// 8 waves one eighth of k; x is split into BF16 hi/lo terms as for the batched
// FFN, and the eighths are added in a fixed order through LDS.
constexpr int kQmTiles = 4;                  // 16-row tiles per wave (whole projection)
constexpr int kQmSplit = 8;                  // waves per block, one k-eighth each
constexpr int kQmDepth = 2;                  // k-steps of loads in flight per wave
constexpr int kQmRows = 16 * kQmTiles;       // rows per block
constexpr int kQmAlign = 64 * kQmSplit * kQmDepth;  // hidden must be a multiple
constexpr int kQqTiles = 1, kQqDepth = 4;    // the Q rows alone (the K/V rows projected before)
constexpr int kQqAlign = 64 * kQmSplit * kQqDepth;
// TILED: W is the tiled copy (mfma_tile16x32), so that each weight load
// instruction of a wave reads one contiguous 1 KB tile instead of 64 bytes
// from each of 16 rows: measured 5.9 TB/s for such a stream against 3.2 TB/s
// for the row-major gather.

// Rows [base, base + 16 T) of W times the batch's x rows: y[b][row] for
// b < batch and row < rows.  part: LDS for the waves' partial tiles,
// [kQmSplit - 1][2 T][64].  NORM: x row b is normalised as it is read,
// (x * inv[b]) * nw, with the scales inv in LDS.  Every thread of the block
// calls it (one barrier).
template <bool TILED, int T, int DEP, bool NORM>
__device__ __forceinline__ void qkv_mfma_rows(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                              int batch, int H, int rows, int base, float* __restrict__ y,
                                              int ystride, kh_f32x4* part, const float* __restrict__ nw,
                                              const float* inv) {
  constexpr int S = kQmSplit;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, kb = lane >> 4;
  const int qsteps = H / (64 * S);  // k-steps per eighth, a multiple of DEP (host-checked)
  const int s0 = wave * qsteps;
  const uint4* __restrict__ wp[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if constexpr (TILED)  // tile (16 rows, 32 k) = 64 uint4; lane l reads uint4 l of it
      wp[t] = reinterpret_cast<const uint4*>(W) +
              (size_t)min((base >> 4) + t, rows / 16 - 1) * (H / 32) * 64 + lane;
    else
      wp[t] = reinterpret_cast<const uint4*>(W + (size_t)min(base + 16 * t + r, rows - 1) * H) + kb + 8 * s0;
  }
  // tokens past the batch re-read the last token's row (the same cache lines,
  // so no extra traffic); their results are never written
  const int xr = min(r, batch - 1);
  // x of token r: k-step s, MFMA e reads k = 64 s + 32 e + 8 kb + [0, 8) as two float4
  const float4* __restrict__ xf = reinterpret_cast<const float4*>(x + (size_t)xr * H) + 2 * kb + 16 * s0;
  const float4* __restrict__ nwf = reinterpret_cast<const float4*>(nw) + 2 * kb + 16 * s0;  // NORM
  const float iv = NORM ? inv[xr] : 1.0f;
  kh_f32x4 c[T][2];
#pragma unroll
  for (int t = 0; t < T; ++t) c[t][0] = c[t][1] = kh_f32x4{0, 0, 0, 0};
  uint4 bw[DEP][T][2];
  float4 bx[DEP][2][2];
  float4 bn[DEP][2][2];  // NORM: the norm weights at the same k
  auto load = [&](int d, int st) {  // clamped, unconditional (past the end: reread, unused)
    const int o = 8 * min(st, qsteps - 1);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (TILED) {  // k-step sg = s0 + st covers the 32-k tiles 2 sg and 2 sg + 1
        const size_t tl = (size_t)2 * (s0 + min(st, qsteps - 1)) * 64;
        bw[d][t][0] = ld_stream(wp[t] + tl);
        bw[d][t][1] = ld_stream(wp[t] + tl + 64);
      } else {
        bw[d][t][0] = ld_stream(wp[t] + o);
        bw[d][t][1] = ld_stream(wp[t] + o + 4);
      }
    }
    bx[d][0][0] = xf[2 * o]; bx[d][0][1] = xf[2 * o + 1];
    bx[d][1][0] = xf[2 * o + 8]; bx[d][1][1] = xf[2 * o + 9];
    if constexpr (NORM) {
      bn[d][0][0] = nwf[2 * o]; bn[d][0][1] = nwf[2 * o + 1];
      bn[d][1][0] = nwf[2 * o + 8]; bn[d][1][1] = nwf[2 * o + 9];
    }
  };
#pragma unroll
  for (int d = 0; d < DEP; ++d) load(d, d);
  __builtin_amdgcn_sched_barrier(0);
  for (int st = 0; st < qsteps; st += DEP) {
#pragma unroll
    for (int d = 0; d < DEP; ++d) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        uint4 xh, xl;
        if constexpr (NORM)
          split_bf16x8(rms_apply4(bx[d][e][0], iv, bn[d][e][0]), rms_apply4(bx[d][e][1], iv, bn[d][e][1]), xh, xl);
        else
          split_bf16x8(bx[d][e][0], bx[d][e][1], xh, xl);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          c[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(bw[d][t][e]), as_bf16x8(xh), c[t][0], 0, 0, 0);
          c[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(bw[d][t][e]), as_bf16x8(xl), c[t][1], 0, 0, 0);
        }
      }
      load(d, st + d + DEP);
      // keep the prefetch here: the scheduler would otherwise sink it to its use
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // C[row][token]: lane holds rows 16 t + 4 kb + q (q = 0..3) of token r
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      part[((wave - 1) * 2 * T + 2 * t) * 64 + lane] = c[t][0];
      part[((wave - 1) * 2 * T + 2 * t + 1) * 64 + lane] = c[t][1];
    }
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    kh_f32x4 acc = c[t][0] + c[t][1];
#pragma unroll
    for (int j = 0; j < S - 1; ++j) acc += part[(j * 2 * T + 2 * t) * 64 + lane] + part[(j * 2 * T + 2 * t + 1) * 64 + lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int item = base + 16 * t + 4 * kb + q;
      if (r < batch && item < rows) y[(size_t)r * ystride + item] = acc[q];
    }
  }
}

// The projections of rows [row_base, rows) (the K and V rows, then the Q rows
// of heads that some token selected), 16*T rows per block over
// qkv_mfma_rows.  The last block also writes the o_proj row list, as
// attn_qkv_kernel's extra block does.
// PW (not void): the heads are selected, not read: the Q-row blocks and the
// last block run every row's head predictor layer 2 and top k
// (attn_select_heads_rows over hpred[batch][phid]); the last block writes
// them to heads_out[batch][nsel] for the kernels after this one.  The K/V
// blocks do not wait for the selection.
template <bool TILED, typename PW = void, int T = kQmTiles, int DEP = kQmDepth>
__global__ __launch_bounds__(64 * kQmSplit) void attn_qkv_mfma_kernel(
    const uint16_t* __restrict__ W, const float* __restrict__ x, int batch, int H, int kvrows,
    int rows, int D, int nh,
    const int32_t* __restrict__ heads, int nsel, float* __restrict__ y, int ystride,
    int32_t* __restrict__ qrows, int32_t* __restrict__ nqrows, int32_t* __restrict__ urank,
    int row_base = 0, const PW* __restrict__ w2 = nullptr, const float* __restrict__ b2 = nullptr,
    const float* __restrict__ hpred = nullptr, int phid = 0, int32_t* __restrict__ heads_out = nullptr) {
  constexpr int S = kQmSplit;
  constexpr bool SEL = !std::is_void<PW>::value;
  using WV = typename Blk8<typename std::conditional<SEL, PW, uint16_t>::type>::V;
  __shared__ kh_f32x4 part[(S - 1) * 2 * T * 64];
  __shared__ WV s_w2[SEL ? kAttnSelHid / 8 * 64 : 1];  // the head predictor's W2 (SEL)
  __shared__ int s_flag[kMaxAttnHeads], s_uh[kMaxAttnHeads];
  __shared__ int wsum[S];
  __shared__ int s_total;
  const int nent = batch * nsel;
  const int lane = threadIdx.x & 63;
  const int base = row_base + blockIdx.x * 16 * T;
  // the last block also writes the plan (first: a grid of one block more than
  // the CUs would run that block in a second round)
  const bool plan = blockIdx.x == gridDim.x - 1;
  bool live = true;  // base < rows for every block
  if constexpr (SEL) {
    if (plan || base >= kvrows) {
      // selection scratch in the (not yet used) partial-sum array
      static_assert(sizeof(part) >= sizeof(float) * 16 * kSelHs + sizeof(int) * (64 + 16 * 64) +
                                        sizeof(uint64_t) * 32, "selection scratch fits");
      uint64_t* s_tab = reinterpret_cast<uint64_t*>(part);
      int* s_any = reinterpret_cast<int*>(s_tab + 32);
      int32_t* s_heads = s_any + 64;
      float* s_hp = reinterpret_cast<float*>(s_heads + 16 * 64);
      attn_select_heads_rows<PW>(w2, b2, hpred, phid, nh, nsel, batch, s_hp, s_tab, s_any, s_heads, s_w2);
      if (plan) {
        for (int i = threadIdx.x; i < nent; i += blockDim.x) heads_out[i] = s_heads[i];
        qkv_plan(s_heads, nent, nh, D, qrows, nqrows, urank, s_flag, s_uh, wsum, &s_total);
      }
      if (base >= kvrows) live = s_any[(base - kvrows) / D] != 0;
      __syncthreads();  // every wave has read s_any before part is written
    }
  } else {
    if (plan) qkv_plan(heads, nent, nh, D, qrows, nqrows, urank, s_flag, s_uh, wsum, &s_total);
    if (base >= kvrows) {
      // Q rows of head h (D is a multiple of 16 T): skipped unless some token selected h
      const int h = (base - kvrows) / D;
      int any = 0;
      for (int i = lane; i < nent; i += 64) any |= heads[i] == h;
      live = __ballot(any) != 0;
    }
  }
  if (!live) return;  // uniform
  qkv_mfma_rows<TILED, T, DEP, false>(W, x, batch, H, rows, base, y, ystride, part, nullptr, nullptr);
}

// The head predictor's layer 1 and the K/V projections of a batched decode
// step in one launch (the batch-1 form is attn_pred_kv_kernel): blocks
// [0, nl1 * batch) run layer 1 of row b = block / nl1 (pred_l1.hpp: exact
// RmsNorm, exact chains; block 0 of each row writes the row's scale to
// inv_out and the normalised row to xn_out), the others project 16 kQmTiles
// K/V rows each (qkv_mfma_rows) meanwhile.  The launch asks for the layer-1
// LDS size, so one block fits per CU.  A K/V block normalises x with scales
// of its own, from an f32 tree sum of the squares per row: the projected rows
// carry tolerance anyway, and only the selection needs the exact scale.
template <typename W, bool TILED>
__global__ __launch_bounds__(kL1LdsThreads) void attn_pred_kv_mfma_kernel(
    const W* __restrict__ w1, const float* __restrict__ b1, int hid, float* __restrict__ hbuf,
    const float* __restrict__ x, int batch, int H, const float* __restrict__ nw, float* __restrict__ inv_out,
    float eps, float* __restrict__ xn_out, const uint16_t* __restrict__ wkvq, int rows, float* __restrict__ y,
    int ystride, int nl1) {
  static_assert(kL1LdsThreads == 64 * kQmSplit, "one k-eighth per wave");
  static_assert(sizeof(float4) * 16 + sizeof(kh_f32x4) * (kQmSplit - 1) * 2 * kQmTiles * 64 <= kL1LdsBytes,
                "the K/V blocks' LDS fits the launch's");
  extern __shared__ float4 lds4[];
  const int nlb = nl1 * batch;
  if ((int)blockIdx.x < nlb) {
    pred_l1_lds_body<W>((int)blockIdx.x % nl1, (int)blockIdx.x / nl1, w1, b1, x, H, hid, hbuf, nw, inv_out,
                        eps, lds4, xn_out);
    return;
  }
  float* s_inv = reinterpret_cast<float*>(lds4);               // [16]
  kh_f32x4* part = reinterpret_cast<kh_f32x4*>(lds4 + 16);     // [S - 1][2 T][64]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int b = wave; b < batch; b += kQmSplit) {
    const float4* xb = reinterpret_cast<const float4*>(x + (size_t)b * H);
    float ss = 0.0f;
    for (int i = lane; i < (H >> 2); i += 64) {
      const float4 v = xb[i];
      ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    ss = wave_sum(ss);
    if (lane == 0) s_inv[b] = rms_inv_exact(ss, H, eps);
  }
  __syncthreads();
  qkv_mfma_rows<TILED, kQmTiles, kQmDepth, true>(wkvq, x, batch, H, rows, ((int)blockIdx.x - nlb) * kQmRows, y,
                                                 ystride, part, nw, s_inv);
}

// Cache positions per decode block: kAttnPasses rows per thread.
template <typename KV, int D>
constexpr int attn_chunk() {
  return kAttnThreads / (D / (16 / (int)sizeof(KV))) * kAttnPasses;
}

// n floats (a multiple of 4) from 16-byte aligned p.
template <int N>
__device__ __forceinline__ void load_f4s(const float* __restrict__ p, float* f) {
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const float4 v = reinterpret_cast<const float4*>(p)[i];
    f[4 * i] = v.x; f[4 * i + 1] = v.y; f[4 * i + 2] = v.z; f[4 * i + 3] = v.w;
  }
}

// The cache of sequence b holds rows [0, pre[b]) in BF16 (kc16/vc16: rows
// loaded as BF16 values, so the storage is exact) and rows [pre[b], len[b]) in
// f32 (kc32/vc32: rows appended by decode steps, and loaded rows that are not
// BF16 values), both arrays [max_batch][nkv][max_seq][D] at the rows'
// positions.  Every row then holds exactly what the reference's f32 KvCache
// holds (kv_cache.rs:33-48), and the bulk of a long prompt streams at BF16 width.
//
// Grid (nsel + 1, batch, nsplit), slot index slowest: every block of slot s
// is dispatched before any of slot s + 1, so the blocks past a sequence's
// slots (nsplit covers a full-length cache in f32, far more slots than a
// BF16 prefix takes) come last and exit while the last chunks run.  The slots
// of sequence b follow its positions: slots [0, n16b) with n16b =
// ceil(pre[b] / CH16) are the BF16 chunks of the prefix (slot c: positions
// c*CH16 ..), then the f32 chunks of the rest (slot n16b + c: positions
// pre[b] + c*CH32 ..), up to and including this step's row len[b] (taken from
// the projection).  Block (a < nsel, b, s) takes slot s and writes its
// un-normalised head output po[b][a][s][D] and (max, exp-sum) pml[b][a][s].
// Block (nsel, b, s): appends this step's roped K and V of kv heads s,
// s+nsplit, ... at position len[b] (f32 rows; decode blocks never read row len
// from the cache), and writes zeros for union heads s, s+nsplit, ... that
// token b did not select (the reference's zero-filled attn_concat, :44).
template <typename KV, int D>
__device__ __forceinline__ void attn_decode_chunk(
    const KV* __restrict__ kc, const KV* __restrict__ vc, int start, int seg_end, int slot,
    const float* __restrict__ yb, int kvd, int nh, int nkv, const int32_t* __restrict__ hb,
    int a, int b, int len, const float* __restrict__ ct, const float* __restrict__ st,
    int max_seq, float inv_sqrt, int nsel, int nsplit, float* __restrict__ po,
    float2* __restrict__ pml) {
  constexpr int EPL = 16 / sizeof(KV);          // elements per 16-byte load
  constexpr int LPR = D / EPL;                  // lanes per cache row
  constexpr int RPP = kAttnThreads / LPR;       // rows per pass
  constexpr int NP = kAttnPasses;               // passes per chunk
  constexpr int CH = RPP * NP;                  // positions per chunk
  constexpr int HALF = D / 2;
  constexpr int NW = kAttnThreads / 64;
  // Only f32 chunks can hold position len (BF16 chunks cover [0, pre) and
  // pre <= len), so only they load this step's k and v.
  constexpr bool kCur = std::is_same<KV, float>::value;
  static_assert(LPR <= 64 && kAttnThreads % LPR == 0 && CH <= kAttnThreads, "tiling");
  static_assert(HALF % EPL == 0 && EPL % 4 == 0, "a lane's slice lies in one half of the head");
  __shared__ float s_p[CH];
  __shared__ float s_red[RPP][D];
  __shared__ float s_wm[NW], s_wl[NW];
  __shared__ uint64_t s_tab[32];  // kExp2Tab
  const int t = threadIdx.x;
  const int h = hb[a];
  if (h < 0 || h >= nh) return;  // sparse_attention.rs:48-50
  if (start >= seg_end) return;
  const int n = min(CH, seg_end - start);
  const int kvh = h / (nh / nkv);
  const int sl = t % LPR, r0 = t / LPR;
  const int e0 = sl * EPL;
  // This lane's q, current k and v slices with their RoPE partners (unconditional
  // 16-byte loads), then every K and V load of the chunk, all in flight before
  // the first use.  RotaryEmbedding::apply (rope.rs:75-87): x[i]*cos -
  // x[i+half]*sin in the first half, x[i]*cos + x[i-half]*sin in the second
  // (products rounded separately; x - y is x + (-y) exactly).
  const uint64_t tabv = kExp2Tab[t & 31];
  const bool first = e0 < HALF;
  const int ec = first ? e0 : e0 - HALF;
  const int ep = first ? e0 + HALF : e0 - HALF;
  const float* qsrc = yb + 2 * kvd + h * D;
  const float* kcur = yb + kvh * D;
  float qx[EPL], qp[EPL], kx[EPL], kp[EPL], vn[EPL], cs[EPL], sn[EPL];
  load_f4s<EPL>(qsrc + e0, qx);
  load_f4s<EPL>(qsrc + ep, qp);
  if constexpr (kCur) {
    load_f4s<EPL>(kcur + e0, kx);
    load_f4s<EPL>(kcur + ep, kp);
    load_f4s<EPL>(kcur + kvd + e0, vn);
  }
  load_f4s<EPL>(ct + ec, cs);
  load_f4s<EPL>(st + ec, sn);
  __builtin_amdgcn_sched_barrier(0);
  // Rows past the segment's last cached one are clamped to it (position len
  // itself is taken from this step's k/v; with no cached row in the segment,
  // its first row is read and never used).
  const size_t rowbase = ((size_t)b * nkv + kvh) * (size_t)max_seq;
  const int last = max(0, min(seg_end, len) - 1);
  uint4 kr[NP], vr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int j = min(start + p * RPP + r0, last);
    kr[p] = ld_stream(reinterpret_cast<const uint4*>(kc + (rowbase + j) * D + e0));
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int j = min(start + p * RPP + r0, last);
    vr[p] = ld_stream(reinterpret_cast<const uint4*>(vc + (rowbase + j) * D + e0));
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any wait
  float qv[EPL], kn[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    qv[e] = qx[e] * cs[e] + (first ? -qp[e] : qp[e]) * sn[e];
    if constexpr (kCur) kn[e] = kx[e] * cs[e] + (first ? -kp[e] : kp[e]) * sn[e];
  }
  // scores: dense_dot(q, k_j) * inv_sqrt_dk (:55-58)
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int j = start + p * RPP + r0;
    float kf[EPL];
    widen16(kr[p], kf, KV());
    if constexpr (kCur) {
      if (j == len) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) kf[e] = kn[e];
      }
    }
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = fmaf(qv[e], kf[e], d);
    if constexpr (LPR <= 16) {
      d = group_sum<LPR>(d);
    } else {
      d = group_sum<16>(d);
      d += __shfl_xor(d, 16, 64);
      if constexpr (LPR == 64) d += __shfl_xor(d, 32, 64);
    }
    if (sl == 0 && j - start < n) s_p[j - start] = d * inv_sqrt;
  }
  if (t < 32) s_tab[t] = tabv;
  lds_barrier();
  // chunk max and exp-sum (softmax_inplace, :81-95, split over chunks)
  float m = t < n ? s_p[t] : -INFINITY;
  m = wave_max(m);
  if ((t & 63) == 0) s_wm[t >> 6] = m;
  lds_barrier();
  m = s_wm[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = fmaxf(m, s_wm[w]);
  float ex = 0.0f;
  if (t < n) {
    ex = expf_glibc_t(s_p[t] - m, s_tab);
    s_p[t] = ex;
  }
  const float ls = wave_sum(ex);
  if ((t & 63) == 0) s_wl[t >> 6] = ls;
  lds_barrier();
  // un-normalised V sum over the chunk (:61-67)
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int jj = p * RPP + r0;
    if (jj < n) {
      float vf[EPL];
      widen16(vr[p], vf, KV());
      if constexpr (kCur) {
        if (start + jj == len) {
#pragma unroll
          for (int e = 0; e < EPL; ++e) vf[e] = vn[e];
        }
      }
      const float pj = s_p[jj];
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = fmaf(pj, vf[e], acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) s_red[r0][e0 + e] = acc[e];
  lds_barrier();
  const size_t so = ((size_t)b * nsel + a) * nsplit + slot;
  if (t < D) {
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < RPP; ++r) o += s_red[r][t];
    po[so * D + t] = o;
  }
  if (t == 0) {
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) l += s_wl[w];
    pml[so] = make_float2(m, l);
  }
}


// PW (not void; batch 1, with the projections of every head done): the heads
// are selected, not read: every live chunk block runs the head predictor's
// layer 2 and top k (attn_select_heads over hpred), and block (0, 0, 0) writes
// them to heads_out and the o_proj row list to qrows_out / nqrows_out for the
// kernel after this one.  The union is then the token's own selection, so the
// append blocks zero-fill nothing.
template <int D, typename PW = void>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(
    const uint16_t* __restrict__ kc16, const uint16_t* __restrict__ vc16, float* __restrict__ kc32,
    float* __restrict__ vc32, const int32_t* __restrict__ pre, const float* __restrict__ y,
    int ystride, int nkv, int nh, const int32_t* __restrict__ heads, int nsel,
    const int32_t* __restrict__ lens, const int64_t* __restrict__ positions,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int max_seq, float inv_sqrt,
    int nsplit, const int32_t* __restrict__ urank, float* __restrict__ po, float2* __restrict__ pml,
    float* __restrict__ cat, int catstride, const PW* __restrict__ w2 = nullptr,
    const float* __restrict__ b2 = nullptr, const float* __restrict__ hpred = nullptr, int phid = 0,
    int32_t* __restrict__ heads_out = nullptr, int32_t* __restrict__ qrows_out = nullptr,
    int32_t* __restrict__ nqrows_out = nullptr) {
  constexpr bool SEL = !std::is_void<PW>::value;
  __shared__ int s_hsel[SEL ? 64 : 1];
  __shared__ int32_t s_heads[SEL ? 64 : 1];
  __shared__ __align__(16) float s_hp[SEL ? kAttnSelHid + 4 * kL2Hw : 4];
  __shared__ uint64_t s_stab[SEL ? 32 : 1];
  constexpr int HALF = D / 2;
  constexpr int CH16 = attn_chunk<uint16_t, D>(), CH32 = attn_chunk<float, D>();
  const int a = blockIdx.x, b = blockIdx.y, s = blockIdx.z, t = threadIdx.x;
  const int len = lens[b];
  const bool valid = len < max_seq;  // a full cache refuses the step for this sequence
  int64_t pos = positions ? positions[b] : len;
  pos = pos < 0 ? 0 : (pos >= max_seq ? max_seq - 1 : pos);
  const int kvd = nkv * D;
  const float* yb = y + (size_t)b * ystride;
  const float* ct = cos_t + pos * HALF;
  const float* st = sin_t + pos * HALF;
  const int32_t* hb = SEL ? s_heads : heads + (size_t)b * nsel;
  if (a == nsel) {
    if (valid) {
      // KvCache::append (kv_cache.rs:33-48) of the roped k (sparse_attention.rs:33-39)
      for (int hh = s; hh < nkv; hh += (int)gridDim.z) {
        const float* kx = yb + (size_t)hh * D;
        const float* vx = kx + kvd;
        const size_t dst = (((size_t)b * nkv + hh) * max_seq + len) * D;
        for (int i = t; i < D; i += kAttnThreads) {
          float kr;
          if (i < HALF) kr = kx[i] * ct[i] - kx[i + HALF] * st[i];
          else kr = kx[i] * ct[i - HALF] + kx[i - HALF] * st[i - HALF];
          kc32[dst + i] = kr;
          vc32[dst + i] = vx[i];
        }
      }
    }
    if constexpr (!SEL) {
      for (int hu = s; hu < nh; hu += (int)gridDim.z) {
        const int u = urank[hu];
        if (u < 0) continue;
        int sel = 0;
        if (valid)
          for (int i = 0; i < nsel; ++i) sel |= hb[i] == hu;
        if (!sel)
          for (int i = t; i < D; i += kAttnThreads) cat[(size_t)b * catstride + (size_t)u * D + i] = 0.0f;
      }
    }
    return;
  }
  if (!valid) return;
  const int pb = pre[b];
  const int n16b = (pb + CH16 - 1) / CH16;
  const int ns = n16b + (len + 1 - pb + CH32 - 1) / CH32;
  if (s >= ns) return;
  if constexpr (SEL) {
    attn_select_heads<PW>(w2, b2, hpred, phid, nh, nsel, s_hp, s_stab, s_hsel, s_heads);
    if (a == 0 && s == 0) {
      for (int i = t; i < nsel; i += kAttnThreads) heads_out[i] = s_heads[i];
      // the o_proj rows: each selected head's D rows, heads ascending
      for (int i = t; i < nsel * D; i += kAttnThreads) qrows_out[i] = s_heads[i / D] * D + i % D;
      if (t == 0) *nqrows_out = nsel * D;
    }
  }
  if (s < n16b)
    attn_decode_chunk<uint16_t, D>(kc16, vc16, s * CH16, pb, s, yb, kvd, nh, nkv, hb, a, b, len, ct, st,
                                   max_seq, inv_sqrt, nsel, nsplit, po, pml);
  else
    attn_decode_chunk<float, D>(kc32, vc32, pb + (s - n16b) * CH32, len + 1, s, yb, kvd, nh, nkv, hb, a, b, len,
                                ct, st, max_seq, inv_sqrt, nsel, nsplit, po, pml);
}

// Decode slots of a sequence: the BF16 chunks covering rows [0, pre), then the
// f32 chunks covering rows [pre, len] (len: this step's row).
__device__ __forceinline__ int attn_nslots(int pre, int len, int ch16, int ch32) {
  return (pre + ch16 - 1) / ch16 + (len + 1 - pre + ch32 - 1) / ch32;
}

// One entry's head output, for R head dimensions e[r] per lane, from its ns
// decode chunks at slots sa .. sa+ns-1: out[r] += sum_j w_j po_j[e] / sum_j w_j l_j
// with w_j = exp(m_j - M), M the largest chunk max; both sums sequential in j.
// The weights are formed one per lane, so the whole wave must be active.
template <int R>
__device__ __forceinline__ void merge_chunks(const float* __restrict__ po,
                                             const float2* __restrict__ pml, size_t sa, int ns,
                                             int D, const int (&e)[R], const uint64_t* tab,
                                             float (&out)[R]) {
  const int lane = threadIdx.x & 63;
  float M = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += 64)
    M = fmaxf(M, wave_max(s0 + lane < ns ? pml[sa + min(s0 + lane, ns - 1)].x : -INFINITY));
  float L = 0.0f, o[R];
#pragma unroll
  for (int r = 0; r < R; ++r) o[r] = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += 64) {
    const float2 mlv = pml[sa + min(s0 + lane, ns - 1)];
    const float wv = expf_glibc_t(mlv.x - M, tab);
    const int cnt = min(64, ns - s0);
    for (int k0 = 0; k0 < cnt; k0 += 16) {
      float pv[R][16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const size_t sl = sa + s0 + min(k0 + k, cnt - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) pv[r][k] = po[sl * D + e[r]];
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k0 + k < cnt) {
          const float wk = readlane_f(wv, k0 + k);
          L = fmaf(readlane_f(mlv.y, k0 + k), wk, L);
#pragma unroll
          for (int r = 0; r < R; ++r) o[r] = fmaf(pv[r][k], wk, o[r]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] += o[r] / L;
}

// One block per (selected-head entry a, token b) whose head h is valid and not
// named by an earlier entry of b: merges the chunks of every entry of b naming
// h (duplicates summed in entry order, as the reference's += into one
// attn_concat slice) into the head output cat[b][u*D ..], u = union rank of h.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(
    const float* __restrict__ po, const float2* __restrict__ pml, int nsplit, int ch16, int ch32,
    const int32_t* __restrict__ pre, const int32_t* __restrict__ heads, int nsel, int nh,
    const int32_t* __restrict__ lens, int max_seq, const int32_t* __restrict__ urank,
    float* __restrict__ cat, int catstride) {
  static_assert(D % 64 == 0, "whole waves");
  __shared__ uint64_t s_tab[32];  // kExp2Tab
  const int a = blockIdx.x, b = blockIdx.y, t = threadIdx.x, lane = t & 63;
  const int32_t* hb = heads + (size_t)b * nsel;
  const int h = hb[a];
  const int len = lens[b];
  if (h < 0 || h >= nh || len >= max_seq) return;
  const uint64_t tabv = kExp2Tab[t & 31];
  for (int i0 = 0; i0 < a; i0 += 64)
    if (__ballot(i0 + lane < a && hb[min(i0 + lane, a - 1)] == h)) return;  // not the first
  const int ns = attn_nslots(pre[b], len, ch16, ch32);
  if (t < 32) s_tab[t] = tabv;
  __syncthreads();
  float out[1] = {0.0f};
  const int e[1] = {t};
  for (int a0 = a; a0 < nsel; a0 += 64) {
    uint64_t hit = __ballot(a0 + lane < nsel && hb[min(a0 + lane, nsel - 1)] == h);
    while (hit) {
      const int a2 = a0 + __builtin_ctzll(hit);
      hit &= hit - 1;
      merge_chunks<1>(po, pml, ((size_t)b * nsel + a2) * nsplit, ns, D, e, s_tab, out);
    }
  }
  cat[(size_t)b * catstride + (size_t)urank[h] * D + t] = out[0];
}

__global__ void attn_set_len_kernel(int32_t* __restrict__ lens, int n, int value) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) lens[i] = value;
}

// src [nkv][len][D] f32 -> one sequence's cache rows 0..len-1 (dst [nkv][max_seq][D]).
template <typename KV>
__global__ __launch_bounds__(256) void attn_fill_cache_kernel(const float* __restrict__ src,
                                                              int64_t len, int D, int64_t total,
                                                              int max_seq, KV* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t per = len * D;
  const int64_t h = i / per, r = i - h * per;
  store_kv(dst + (h * max_seq) * (int64_t)D + r, src[i]);
}

// Device-loaded rows of a KH_KV_BF16 handle: both the f32 and the BF16 copy
// are written, and *notbf records whether any value of k or v carries bits a
// BF16 cannot hold; attn_set_pre_kernel then makes the rows a BF16 prefix
// only when none does (so the cache always holds the values exactly).
__global__ __launch_bounds__(256) void attn_fill_cache2_kernel(
    const float* __restrict__ k, const float* __restrict__ v, int64_t len, int D, int64_t total,
    int max_seq, float* __restrict__ k32, float* __restrict__ v32, uint16_t* __restrict__ k16,
    uint16_t* __restrict__ v16, int32_t* __restrict__ notbf) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool bad = false;
  if (i < total) {
    const int64_t per = len * D;
    const int64_t h = i / per, r = i - h * per;
    const int64_t o = (h * max_seq) * (int64_t)D + r;
    const uint32_t kb = __float_as_uint(k[i]), vb = __float_as_uint(v[i]);
    k32[o] = k[i];
    v32[o] = v[i];
    k16[o] = static_cast<uint16_t>(kb >> 16);
    v16[o] = static_cast<uint16_t>(vb >> 16);
    bad = ((kb | vb) & 0xffffu) != 0;
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(notbf, 1);
}

__global__ void attn_set_pre_kernel(int32_t* __restrict__ pre, const int32_t* __restrict__ notbf,
                                    int len) {
  if (threadIdx.x == 0) pre[0] = notbf[0] ? 0 : len;
}

// o_proj for batch <= 2 with the chunk merge folded in: gather_rows_kernel's
// column slice x row group over the union rows of WoT, where the value of row
// h*D + e for token b is computed in the block from the decode chunks (the
// attn_merge_kernel arithmetic, so the result is the same).  Waves 0-3 issue
// the weight loads and accumulate; waves 4-7 merge the chunks meanwhile (each
// wave waits only for its own loads).
constexpr int kOprojMaxSel = 256;  // head-list entries staged per token
constexpr int kOprojThreads = 2 * kDownThreads;
template <int NB>
__global__ __launch_bounds__(kOprojThreads) void attn_oproj_kernel(
    const uint16_t* __restrict__ WoT, int H, int D, const int32_t* __restrict__ rows,
    int n_rows, const int32_t* __restrict__ n_rows_dev, const float* __restrict__ po,
    const float2* __restrict__ pml, int nsplit, int ch16, int ch32, const int32_t* __restrict__ pre,
    const int32_t* __restrict__ heads, int nsel, const int32_t* __restrict__ lens, int max_seq,
    int batch, int groups, float* __restrict__ partial) {
  __shared__ float red[4][NB][kSlice];
  __shared__ int s_ids[kDownRows];
  __shared__ float s_h[NB][kDownRows];
  __shared__ int s_hd[NB][kOprojMaxSel];
  __shared__ uint64_t s_tab[32];  // kExp2Tab
  __shared__ int s_len[NB], s_pre[NB];
  const int n = min(n_rows, *n_rows_dev);
  const int slice = blockIdx.x, grp = blockIdx.y;
  const int tid = threadIdx.x;
  const bool gather = tid < kDownThreads;
  const int per = (n + groups - 1) / groups;
  const int r0 = min(n, grp * per);
  const int r1 = min(n, r0 + per);
  const int nr = r1 - r0;  // <= kDownRows by construction of `groups`
  const int rlast = max(nr, 1) - 1;
  const uint64_t tabv = kExp2Tab[tid & 31];
  if (tid < nr) s_ids[tid] = rows[r0 + tid];
  if (tid == 0 && nr == 0) s_ids[0] = 0;  // an empty group reads row 0, unused
  for (int i = tid; i < NB * nsel; i += kOprojThreads) {
    const int b = i / nsel;
    s_hd[b][i - b * nsel] = b < batch ? heads[i] : -1;
  }
  if (tid < NB) s_len[tid] = tid < batch ? lens[tid] : max_seq;
  if (tid < NB) s_pre[tid] = tid < batch ? pre[tid] : 0;
  if (tid < 32) s_tab[tid] = tabv;
  __syncthreads();
  constexpr int RPL = kDownRows / 8;  // rows per row lane
  const int sub = (tid & (kDownThreads - 1)) >> 5;
  const int cl = tid & 31;
  const int col = slice * kSlice + cl * 8;
  uint4 w[RPL];
  if (gather) {
    // Unconditional (clamped) loads: rows past the group and columns past H
    // re-read valid ones that are never used.
    const int colc = col < H ? col : H - 8;
#pragma unroll
    for (int m = 0; m < RPL; ++m)
      w[m] = ld_stream(reinterpret_cast<const uint4*>(WoT + (size_t)s_ids[min(sub + 8 * m, rlast)] * H + colc));
  } else {
    // Merge waves: one (token b, head slot j) pair per wave at a time; a slot
    // is the run of the group's rows that belong to one head.  For each entry
    // of b naming the head (ascending), the chunk weights w_j = exp(m_j - M)
    // are formed one per lane, and each lane accumulates its rows (at most
    // two) as sum_j w_j po_j / sum_j w_j l_j, sequential in j.  Heads b did
    // not select give 0.
    const int mw = (tid - kDownThreads) >> 6, lane = tid & 63;
    const int i0 = s_ids[0] % D;  // head dimension of the group's first row
    const int nslot = nr > 0 ? (i0 + nr - 1) / D + 1 : 0;
    for (int p = mw; p < batch * nslot; p += kDownThreads / 64) {
      const int b = p / nslot, j = p - b * nslot;
      const int rb = max(0, j * D - i0), re = min(nr, (j + 1) * D - i0);  // rows [rb, re)
      const int h = s_ids[rb] / D;
      const int len = s_len[b];
      const int ns = len < max_seq ? attn_nslots(s_pre[b], len, ch16, ch32) : 0;
      const int ra = rb + lane, rc = rb + lane + 64;
      const int ea = (i0 + min(ra, re - 1)) % D, ec = (i0 + min(rc, re - 1)) % D;
      float out[2] = {0.0f, 0.0f};
      const int ee[2] = {ea, ec};
      for (int a0 = 0; a0 < nsel && ns > 0; a0 += 64) {
        uint64_t hit = __ballot(a0 + lane < nsel && s_hd[b][min(a0 + lane, nsel - 1)] == h);
        while (hit) {
          const int a = a0 + __builtin_ctzll(hit);
          hit &= hit - 1;
          merge_chunks<2>(po, pml, ((size_t)b * nsel + a) * nsplit, ns, D, ee, s_tab, out);
        }
      }
      const float outa = out[0], outc = out[1];
      if (b < NB && ra < re) s_h[b][ra] = outa;
      if (b < NB && rc < re) s_h[b][rc] = outc;
    }
  }
  __syncthreads();
  if (gather) {
    float acc[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[b][e] = 0.0f;
#pragma unroll
    for (int m = 0; m < RPL; ++m) {
      const int r = sub + 8 * m;
      if (r >= nr) break;
      const float wf[8] = {bf16_lo(w[m].x), bf16_hi(w[m].x), bf16_lo(w[m].y), bf16_hi(w[m].y),
                           bf16_lo(w[m].z), bf16_hi(w[m].z), bf16_lo(w[m].w), bf16_hi(w[m].w)};
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float hv = s_h[b][r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[b][e] = fmaf(hv, wf[e], acc[b][e]);
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[b][e] += __shfl_xor(acc[b][e], 32, 64);
    const int wv = tid >> 6;
    if ((tid & 63) < 32) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wv][b][cl * 8 + e] = acc[b][e];
    }
  }
  __syncthreads();
  if (gather) {
    const int ocol = slice * kSlice + tid;
    for (int b = 0; b < batch; ++b) {
      const float sm = (red[0][b][tid] + red[1][b][tid]) + (red[2][b][tid] + red[3][b][tid]);
      if (ocol < H) partial[((size_t)grp * NB + b) * H + ocol] = sm;
    }
  }
}


}  // namespace kh

using namespace kh;

// T[rt][kt][kb][r][e] = W[16 rt + r][32 kt + 8 kb + e] (BF16): each 16-row x
// 32-k tile is one contiguous kilobyte, laid out so that lane l = 16 kb + r of
// a wave reads exactly the 16 bytes it feeds to v_mfma_f32_16x16x32_bf16.
// One thread per 16-byte piece (rows a multiple of 16, H of 32).
__global__ void mfma_tile16x32_kernel(const uint16_t* __restrict__ W, int rows, int H,
                                      uint16_t* __restrict__ T) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte piece of T
  const int64_t n = (int64_t)rows * H / 8;
  if (i >= n) return;
  const int lane = (int)(i & 63);
  const int64_t tile = i >> 6;
  const int kts = H / 32;
  const int64_t rt = tile / kts;
  const int kt = (int)(tile - rt * kts);
  const int r = lane & 15, kb = lane >> 4;
  reinterpret_cast<uint4*>(T)[i] =
      *reinterpret_cast<const uint4*>(W + (size_t)(16 * rt + r) * H + 32 * kt + 8 * kb);
}

// Compute units of the current device (cached per device).
static int attn_device_cus() {
  static std::mutex mu;
  static std::vector<int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(mu);
  if ((int)cus.size() <= dev) cus.resize(dev + 1, 0);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

struct kh_sparse_attn {
  int hidden = 0, nh = 0, nkv = 0, d = 0, max_seq = 0, max_batch = 0, kv_f32 = 0;
  uint16_t* wkvq = nullptr;  // [2*kvd + nh*d][hidden]
  uint16_t* wot = nullptr;   // [nh*d][hidden]
  // cache rows of sequence b: [0, pre[b]) in kc16/vc16 (BF16 values, KH_KV_BF16
  // handles only), [pre[b], len[b]) in kc32/vc32; all [max_batch][nkv][max_seq][d]
  uint16_t* kc16 = nullptr;
  uint16_t* vc16 = nullptr;
  float* kc32 = nullptr;
  float* vc32 = nullptr;
  int32_t* pre = nullptr;    // [max_batch]
  int32_t* notbf = nullptr;  // [1] device-side load check (kh_sparse_attn_load_cache_dev)
  float* cos_t = nullptr;    // [max_seq][d/2]
  float* sin_t = nullptr;
  int32_t* lens = nullptr;   // [max_batch]
  float* y = nullptr;        // [max_batch][2*kvd + nh*d]
  float* cat = nullptr;      // [max_batch][nh*d]
  int32_t* qrows = nullptr;  // [nh*d + 1 + nh]: rows, their count, union rank per head (-1: none)
  uint16_t* wkvq_t = nullptr;  // wkvq in 16 x 32 tiles (mfma_tile16x32) for the batched projections
  std::vector<int64_t> len_host, pre_host;
  Scratch po, pml, partial;
  Scratch xn;  // normalised rows of the batched fused block
  int kvd() const { return nkv * d; }
  int ystride() const { return 2 * nkv * d + nh * d; }
  size_t seq_elems() const { return (size_t)nkv * max_seq * d; }
};

extern "C" int kh_sparse_attn_destroy(kh_sparse_attn* a) {
  if (!a) return KH_OK;
  dev_free(a->wkvq);
  dev_free(a->wkvq_t);
  dev_free(a->wot);
  dev_free(a->kc16);
  dev_free(a->vc16);
  dev_free(a->kc32);
  dev_free(a->vc32);
  dev_free(a->pre);
  dev_free(a->notbf);
  dev_free(a->cos_t);
  dev_free(a->sin_t);
  dev_free(a->lens);
  dev_free(a->y);
  dev_free(a->cat);
  dev_free(a->qrows);
  delete a;
  return KH_OK;
}

// Shape checks, allocation and the RoPE tables; weights are filled by the caller.
static int attn_alloc(int hidden, int num_heads, int num_kv_heads, int head_dim, int max_seq,
                      int max_batch, float rope_theta, int kv_dtype, kh_sparse_attn** out) {
  KH_CHECK_ARG(out != nullptr, "null out");
  *out = nullptr;
  KH_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "hidden (%d) must be a positive multiple of 8",
               hidden);
  KH_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256,
               "head_dim %d not supported (64, 128 or 256)", head_dim);
  KH_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
                   num_heads <= kMaxAttnHeads,
               "num_heads (%d) must be a multiple of num_kv_heads (%d) and <= %d", num_heads,
               num_kv_heads, kMaxAttnHeads);
  KH_CHECK_ARG(max_seq > 0 && max_batch >= 1 && max_batch <= 16,
               "max_seq must be positive and max_batch in [1,16]");
  KH_CHECK_ARG(kv_dtype == KH_KV_BF16 || kv_dtype == KH_KV_F32, "bad kv_dtype %d", kv_dtype);
  KH_CHECK_ARG(rope_theta > 0.0f, "rope_theta must be positive");
  auto* a = new kh_sparse_attn();
  a->hidden = hidden;
  a->nh = num_heads;
  a->nkv = num_kv_heads;
  a->d = head_dim;
  a->max_seq = max_seq;
  a->max_batch = max_batch;
  a->kv_f32 = kv_dtype == KH_KV_F32;
  a->len_host.assign(max_batch, 0);
  a->pre_host.assign(max_batch, 0);
  const size_t H = hidden, qd = (size_t)num_heads * head_dim, kvd = (size_t)num_kv_heads * head_dim;
  const size_t half = head_dim / 2;
  a->wkvq = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * (2 * kvd + qd) * H));
  a->wot = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * qd * H));
  if (!a->kv_f32) {
    a->kc16 = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * a->seq_elems() * max_batch));
    a->vc16 = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * a->seq_elems() * max_batch));
  }
  a->kc32 = static_cast<float*>(dev_alloc(sizeof(float) * a->seq_elems() * max_batch));
  a->vc32 = static_cast<float*>(dev_alloc(sizeof(float) * a->seq_elems() * max_batch));
  a->pre = static_cast<int32_t*>(dev_alloc(sizeof(int32_t) * max_batch));
  a->notbf = static_cast<int32_t*>(dev_alloc(sizeof(int32_t)));
  a->cos_t = static_cast<float*>(dev_alloc(sizeof(float) * max_seq * half));
  a->sin_t = static_cast<float*>(dev_alloc(sizeof(float) * max_seq * half));
  a->lens = static_cast<int32_t*>(dev_alloc(sizeof(int32_t) * max_batch));
  a->y = static_cast<float*>(dev_alloc(sizeof(float) * max_batch * a->ystride()));
  a->cat = static_cast<float*>(dev_alloc(sizeof(float) * max_batch * qd));
  a->qrows = static_cast<int32_t*>(dev_alloc(sizeof(int32_t) * (qd + 1 + num_heads)));
  if (max_batch > 1 && H % 32 == 0 && (2 * kvd + qd) % 16 == 0)
    a->wkvq_t = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * (2 * kvd + qd) * H));
  if (!a->wkvq || !a->wot || (!a->kv_f32 && (!a->kc16 || !a->vc16)) || !a->kc32 || !a->vc32 || !a->pre || !a->notbf ||
      !a->cos_t || !a->sin_t || !a->lens || !a->y || !a->cat || !a->qrows) {
    kh_sparse_attn_destroy(a);
    return KH_ERR_ALLOC;
  }
  // RotaryEmbedding::new_partial (rope.rs:23-37) with the full head rotated,
  // evaluated in f32 with the host libm as the reference does.
  std::vector<float> c(max_seq * half), s(max_seq * half);
  for (int p = 0; p < max_seq; ++p)
    for (size_t i = 0; i < half; ++i) {
      const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(head_dim);
      const float freq = 1.0f / powf(rope_theta, e);
      const float ang = static_cast<float>(p) * freq;
      c[p * half + i] = cosf(ang);
      s[p * half + i] = sinf(ang);
    }
  if (hipMemcpy(a->cos_t, c.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(a->sin_t, s.data(), sizeof(float) * s.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemset(a->lens, 0, sizeof(int32_t) * max_batch) != hipSuccess ||
      hipMemset(a->pre, 0, sizeof(int32_t) * max_batch) != hipSuccess) {
    set_error("attention table upload failed");
    kh_sparse_attn_destroy(a);
    return KH_ERR_HIP;
  }
  *out = a;
  return KH_OK;
}

// The tiled copy of wkvq for the batched projections (a no-op without one).
static hipError_t attn_tile_weights(kh_sparse_attn* a) {
  if (!a->wkvq_t) return hipSuccess;
  const int rows = 2 * a->kvd() + a->nh * a->d;
  const int64_t pieces = (int64_t)rows * a->hidden / 8;
  hipLaunchKernelGGL(mfma_tile16x32_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, 0,
                     a->wkvq, rows, a->hidden, a->wkvq_t);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? hipDeviceSynchronize() : e;
}

extern "C" int kh_sparse_attn_create(int hidden, int num_heads, int num_kv_heads, int head_dim,
                                     int max_seq, int max_batch, float rope_theta, int kv_dtype,
                                     const uint16_t* wq_host, const uint16_t* wk_host,
                                     const uint16_t* wv_host, const uint16_t* wo_host,
                                     kh_sparse_attn** out) {
  KH_CHECK_ARG(wq_host && wk_host && wv_host && wo_host, "null weights");
  kh_sparse_attn* a = nullptr;
  int rc = attn_alloc(hidden, num_heads, num_kv_heads, head_dim, max_seq, max_batch, rope_theta,
                      kv_dtype, &a);
  if (rc != KH_OK) return rc;
  const size_t H = hidden, qd = (size_t)num_heads * head_dim, kvd = (size_t)num_kv_heads * head_dim;
  const size_t row = sizeof(uint16_t) * H;
  uint16_t* ot = static_cast<uint16_t*>(malloc(sizeof(uint16_t) * qd * H));
  if (!ot) {
    kh_sparse_attn_destroy(a);
    set_error("host allocation failed");
    return KH_ERR_ALLOC;
  }
  // wo[hidden][qd] -> WoT[qd][hidden], blocked for locality
  const size_t TB = 64;
  for (size_t j0 = 0; j0 < H; j0 += TB)
    for (size_t i0 = 0; i0 < qd; i0 += TB)
      for (size_t j = j0; j < std::min(H, j0 + TB); ++j)
        for (size_t i = i0; i < std::min(qd, i0 + TB); ++i) ot[i * H + j] = wo_host[j * qd + i];
  hipError_t e = hipMemcpy(a->wkvq, wk_host, row * kvd, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(a->wkvq + kvd * H, wv_host, row * kvd, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(a->wkvq + 2 * kvd * H, wq_host, row * qd, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(a->wot, ot, row * qd, hipMemcpyHostToDevice);
  free(ot);
  if (e == hipSuccess) e = attn_tile_weights(a);
  if (e != hipSuccess) {
    set_error("attention weight upload failed: %s", hipGetErrorString(e));
    kh_sparse_attn_destroy(a);
    return KH_ERR_HIP;
  }
  *out = a;
  return KH_OK;
}

extern "C" int kh_sparse_attn_create_dev(int hidden, int num_heads, int num_kv_heads,
                                         int head_dim, int max_seq, int max_batch,
                                         float rope_theta, int kv_dtype, const uint16_t* wq_dev,
                                         const uint16_t* wk_dev, const uint16_t* wv_dev,
                                         const uint16_t* wo_dev, kh_sparse_attn** out) {
  KH_CHECK_ARG(wq_dev && wk_dev && wv_dev && wo_dev, "null weights");
  kh_sparse_attn* a = nullptr;
  int rc = attn_alloc(hidden, num_heads, num_kv_heads, head_dim, max_seq, max_batch, rope_theta,
                      kv_dtype, &a);
  if (rc != KH_OK) return rc;
  const size_t H = hidden, qd = (size_t)num_heads * head_dim, kvd = (size_t)num_kv_heads * head_dim;
  const size_t row = sizeof(uint16_t) * H;
  hipError_t e = hipMemcpy(a->wkvq, wk_dev, row * kvd, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(a->wkvq + kvd * H, wv_dev, row * kvd, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(a->wkvq + 2 * kvd * H, wq_dev, row * qd, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, dim3(ceil_div(qd, 32), ceil_div(H, 32)), dim3(256), 0,
                       0, wo_dev, hidden, static_cast<int>(qd), a->wot);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = attn_tile_weights(a);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    set_error("attention weight repack failed: %s", hipGetErrorString(e));
    kh_sparse_attn_destroy(a);
    return KH_ERR_HIP;
  }
  *out = a;
  return KH_OK;
}

extern "C" int kh_sparse_attn_load_cache(kh_sparse_attn* a, int64_t b, const float* k_host,
                                         const float* v_host, int64_t len) {
  KH_CHECK_ARG(a != nullptr, "null handle");
  KH_CHECK_ARG(b >= 0 && b < a->max_batch, "sequence %lld not in [0,%d)", (long long)b, a->max_batch);
  KH_CHECK_ARG(len >= 0 && len <= a->max_seq, "len %lld not in [0,%d]", (long long)len, a->max_seq);
  KH_CHECK_ARG(len == 0 || (k_host && v_host), "null cache data");
  const size_t D = a->d, rows = (size_t)len, n = (size_t)a->nkv * rows * D;
  // BF16 storage only when it holds the rows exactly
  bool bf16 = !a->kv_f32 && rows > 0;
  for (size_t i = 0; bf16 && i < n; ++i) {
    uint32_t uk, uv;
    memcpy(&uk, k_host + i, 4);
    memcpy(&uv, v_host + i, 4);
    bf16 = ((uk | uv) & 0xffffu) == 0;
  }
  for (int kv = 0; kv < 2 && rows; ++kv) {
    const float* src = kv ? v_host : k_host;
    for (int hh = 0; hh < a->nkv; ++hh) {
      const float* sp = src + (size_t)hh * rows * D;
      const size_t off = ((size_t)b * a->nkv + hh) * a->max_seq * D;
      if (bf16) {
        std::vector<uint16_t> tmp(rows * D);
        for (size_t i = 0; i < tmp.size(); ++i) tmp[i] = f32_to_bf16(sp[i]);
        KH_HIP(hipMemcpy((kv ? a->vc16 : a->kc16) + off, tmp.data(), sizeof(uint16_t) * tmp.size(),
                         hipMemcpyHostToDevice));
      } else {
        KH_HIP(hipMemcpy((kv ? a->vc32 : a->kc32) + off, sp, sizeof(float) * rows * D, hipMemcpyHostToDevice));
      }
    }
  }
  const int32_t l32 = static_cast<int32_t>(len), p32 = bf16 ? l32 : 0;
  KH_HIP(hipMemcpy(a->lens + b, &l32, sizeof(int32_t), hipMemcpyHostToDevice));
  KH_HIP(hipMemcpy(a->pre + b, &p32, sizeof(int32_t), hipMemcpyHostToDevice));
  a->len_host[b] = len;
  a->pre_host[b] = p32;
  return KH_OK;
}

extern "C" int kh_sparse_attn_load_cache_dev(kh_sparse_attn* a, int64_t b, const float* k_dev,
                                             const float* v_dev, int64_t len, void* stream) {
  KH_CHECK_ARG(a != nullptr, "null handle");
  KH_CHECK_ARG(b >= 0 && b < a->max_batch, "sequence %lld not in [0,%d)", (long long)b, a->max_batch);
  KH_CHECK_ARG(len >= 0 && len <= a->max_seq, "len %lld not in [0,%d]", (long long)len, a->max_seq);
  KH_CHECK_ARG(len == 0 || (k_dev && v_dev), "null cache data");
  hipStream_t st = as_stream(stream);
  const int64_t total = (int64_t)a->nkv * len * a->d;
  const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
  const size_t off = (size_t)b * a->seq_elems();
  if (total > 0 && !a->kv_f32) {
    // both copies, and on the device: a BF16 prefix when every value is a
    // BF16 value (a BF16 model's prefill), else f32 rows (pre = 0)
    hipLaunchKernelGGL(attn_set_len_kernel, dim3(1), dim3(64), 0, st, a->notbf, 1, 0);
    hipLaunchKernelGGL(attn_fill_cache2_kernel, dim3(blocks), dim3(256), 0, st, k_dev, v_dev, len, a->d,
                       total, a->max_seq, a->kc32 + off, a->vc32 + off, a->kc16 + off, a->vc16 + off,
                       a->notbf);
    hipLaunchKernelGGL(attn_set_pre_kernel, dim3(1), dim3(64), 0, st, a->pre + b, a->notbf,
                       static_cast<int>(len));
  } else {
    if (total > 0) {
      hipLaunchKernelGGL(attn_fill_cache_kernel<float>, dim3(blocks), dim3(256), 0, st, k_dev, len, a->d,
                         total, a->max_seq, a->kc32 + off);
      hipLaunchKernelGGL(attn_fill_cache_kernel<float>, dim3(blocks), dim3(256), 0, st, v_dev, len, a->d,
                         total, a->max_seq, a->vc32 + off);
    }
    hipLaunchKernelGGL(attn_set_len_kernel, dim3(1), dim3(64), 0, st, a->pre + b, 1, 0);
  }
  hipLaunchKernelGGL(attn_set_len_kernel, dim3(1), dim3(64), 0, st, a->lens + b, 1,
                     static_cast<int>(len));
  KH_LAUNCHED();
  a->len_host[b] = len;
  a->pre_host[b] = -1;  // decided on the device
  return KH_OK;
}

extern "C" int kh_sparse_attn_read_cache(const kh_sparse_attn* a, int64_t b, float* k_host,
                                         float* v_host, int64_t len) {
  KH_CHECK_ARG(a != nullptr, "null handle");
  KH_CHECK_ARG(b >= 0 && b < a->max_batch, "sequence %lld not in [0,%d)", (long long)b, a->max_batch);
  KH_CHECK_ARG(len >= 0 && len <= a->max_seq, "len %lld not in [0,%d]", (long long)len, a->max_seq);
  KH_CHECK_ARG(len == 0 || (k_host && v_host), "null output");
  const size_t D = a->d, rows = (size_t)len;
  int32_t pre = 0;
  KH_HIP(hipMemcpy(&pre, a->pre + b, sizeof(int32_t), hipMemcpyDeviceToHost));
  const size_t r16 = std::min(rows, (size_t)pre);
  for (int kv = 0; kv < 2 && rows; ++kv) {
    float* dstf = kv ? v_host : k_host;
    for (int hh = 0; hh < a->nkv; ++hh) {
      const size_t off = ((size_t)b * a->nkv + hh) * a->max_seq * D;
      float* d = dstf + (size_t)hh * rows * D;
      if (r16) {
        std::vector<uint16_t> tmp(r16 * D);
        KH_HIP(hipMemcpy(tmp.data(), (kv ? a->vc16 : a->kc16) + off, sizeof(uint16_t) * tmp.size(),
                         hipMemcpyDeviceToHost));
        for (size_t i = 0; i < tmp.size(); ++i) {
          const uint32_t u = static_cast<uint32_t>(tmp[i]) << 16;
          memcpy(d + i, &u, 4);
        }
      }
      if (rows > r16)
        KH_HIP(hipMemcpy(d + r16 * D, (kv ? a->vc32 : a->kc32) + off + r16 * D, sizeof(float) * (rows - r16) * D,
                         hipMemcpyDeviceToHost));
    }
  }
  return KH_OK;
}

extern "C" int kh_sparse_attn_cache_len(kh_sparse_attn* a, int64_t b, int64_t* len) {
  KH_CHECK_ARG(a && len, "null argument");
  KH_CHECK_ARG(b >= 0 && b < a->max_batch, "sequence %lld not in [0,%d)", (long long)b, a->max_batch);
  int32_t l = 0;
  KH_HIP(hipMemcpy(&l, a->lens + b, sizeof(int32_t), hipMemcpyDeviceToHost));
  a->len_host[b] = l;
  *len = l;
  return KH_OK;
}

extern "C" int kh_sparse_attn_clear(kh_sparse_attn* a, void* stream) {
  KH_CHECK_ARG(a != nullptr, "null handle");
  hipLaunchKernelGGL(attn_set_len_kernel, dim3(1), dim3(64), 0, as_stream(stream), a->lens,
                     a->max_batch, 0);
  hipLaunchKernelGGL(attn_set_len_kernel, dim3(1), dim3(64), 0, as_stream(stream), a->pre,
                     a->max_batch, 0);
  KH_LAUNCHED();
  std::fill(a->len_host.begin(), a->len_host.end(), 0);
  std::fill(a->pre_host.begin(), a->pre_host.end(), 0);
  return KH_OK;
}

template <int D>
static int attn_decode_launch(kh_sparse_attn* a, int batch, const int64_t* pos,
                              const int32_t* heads, int nsel, int nsplit, float* po,
                              float2* pml, bool merge, hipStream_t st, const PredL1View* hsel = nullptr) {
  const int qd = a->nh * D;
  const dim3 g(nsel + 1, batch, nsplit);
  const float isq = 1.0f / sqrtf(static_cast<float>(D));
  if (!hsel)
    hipLaunchKernelGGL(attn_decode_kernel<D>, g, dim3(kAttnThreads), 0, st, a->kc16, a->vc16, a->kc32, a->vc32,
                       a->pre, a->y, a->ystride(), a->nkv, a->nh, heads, nsel, a->lens, pos, a->cos_t, a->sin_t,
                       a->max_seq, isq, nsplit, a->qrows + qd + 1, po, pml, a->cat, qd);
  else if (hsel->bf16)
    hipLaunchKernelGGL((attn_decode_kernel<D, uint16_t>), g, dim3(kAttnThreads), 0, st, a->kc16, a->vc16, a->kc32,
                       a->vc32, a->pre, a->y, a->ystride(), a->nkv, a->nh, nullptr, nsel, a->lens, pos, a->cos_t,
                       a->sin_t, a->max_seq, isq, nsplit, a->qrows + qd + 1, po, pml, a->cat, qd,
                       static_cast<const uint16_t*>(hsel->w2b), hsel->b2, hsel->hbuf, hsel->hid,
                       const_cast<int32_t*>(heads), a->qrows, a->qrows + qd);
  else
    hipLaunchKernelGGL((attn_decode_kernel<D, float>), g, dim3(kAttnThreads), 0, st, a->kc16, a->vc16, a->kc32,
                       a->vc32, a->pre, a->y, a->ystride(), a->nkv, a->nh, nullptr, nsel, a->lens, pos, a->cos_t,
                       a->sin_t, a->max_seq, isq, nsplit, a->qrows + qd + 1, po, pml, a->cat, qd,
                       static_cast<const float*>(hsel->w2b), hsel->b2, hsel->hbuf, hsel->hid,
                       const_cast<int32_t*>(heads), a->qrows, a->qrows + qd);
  KH_LAUNCHED();
  if (!merge) return KH_OK;
  hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(nsel, batch), dim3(D), 0, st, po, pml, nsplit,
                     attn_chunk<uint16_t, D>(), attn_chunk<float, D>(), a->pre, heads, nsel, a->nh,
                     a->lens, a->max_seq, a->qrows + qd + 1, a->cat, qd);
  KH_LAUNCHED();
  return KH_OK;
}

// attn_qkv_mfma_kernel over rows [row_base, kvrows + qd) (+ the plan block);
// hsel (PW not void): the heads selected inside from hsel's layer-1 outputs.
template <bool TILED, typename PW, int T, int DEP>
static void qm_launch(kh_sparse_attn* a, const uint16_t* w, const float* x, int batch, const int32_t* heads,
                      int nsel, int row_base, const PredL1View* hsel, int32_t* hout, hipStream_t st) {
  const int H = a->hidden, D = a->d, qd = a->nh * D, kvrows = 2 * a->kvd(), rows = kvrows + qd;
  const dim3 g(ceil_div(rows - row_base, 16 * T)), blk(64 * kQmSplit);
  hipLaunchKernelGGL((attn_qkv_mfma_kernel<TILED, PW, T, DEP>), g, blk, 0, st, w, x, batch, H, kvrows, rows, D,
                     a->nh, heads, nsel, a->y, a->ystride(), a->qrows, a->qrows + qd, a->qrows + qd + 1, row_base,
                     hsel ? static_cast<const PW*>(hsel->w2b) : nullptr, hsel ? hsel->b2 : nullptr,
                     hsel ? hsel->hbuf : nullptr, hsel ? hsel->hid : 0, hout);
}

// nrm.w set (batch 1 only): x is the un-normalised hidden row, normalised
// inside the projection kernel with the scale at nrm.inv.
// hsel with batch > 1: x holds the normalised rows, and the heads are selected
// inside the projection (the head predictor's layer 2 over hsel->hbuf) and
// written to heads.
// kv_done (batch 1 with nrm.w, or batch > 1 with hsel): attn_pred_kv_kernel or
// attn_pred_kv_mfma_kernel projected the K/V rows, so only the selected heads'
// Q rows remain.  qkv_done: every projection is done (attn_pred_kv_kernel); with
// hsel at batch 1 the decode kernel selects the heads and writes the o_proj
// row list.
template <int NB>
static int attn_launch(kh_sparse_attn* a, const float* x, int batch, const int64_t* pos,
                       const int32_t* heads, int nsel, float* out, int accumulate,
                       hipStream_t st, const NormIn& nrm = NormIn{}, bool kv_done = false,
                       const PredL1View* hsel = nullptr, bool qkv_done = false) {
  const int H = a->hidden, D = a->d, qd = a->nh * D, kvrows = 2 * a->kvd();
  // 1. projections (+ the o_proj row list in the last block), unless done
  const int rows = kvrows + qd;
  if (qkv_done) {
  } else if (NB > 1 && H % kQmAlign == 0 && !nrm.w) {
    const bool t = a->wkvq_t != nullptr;
    const uint16_t* w = t ? a->wkvq_t : a->wkvq;
    int32_t* hout = const_cast<int32_t*>(heads);
    if (!hsel) {
      if (t) qm_launch<true, void, kQmTiles, kQmDepth>(a, w, x, batch, heads, nsel, 0, nullptr, nullptr, st);
      else qm_launch<false, void, kQmTiles, kQmDepth>(a, w, x, batch, heads, nsel, 0, nullptr, nullptr, st);
    } else if (kv_done) {
      // the K/V rows are projected: the Q rows alone, one 16-row tile per block
      if (H % kQqAlign != 0) {
        set_error("the overlapped batched attention block needs hidden a multiple of %d", kQqAlign);
        return KH_ERR_UNSUPPORTED;
      }
      if (hsel->bf16) {
        if (t) qm_launch<true, uint16_t, kQqTiles, kQqDepth>(a, w, x, batch, nullptr, nsel, kvrows, hsel, hout, st);
        else qm_launch<false, uint16_t, kQqTiles, kQqDepth>(a, w, x, batch, nullptr, nsel, kvrows, hsel, hout, st);
      } else {
        if (t) qm_launch<true, float, kQqTiles, kQqDepth>(a, w, x, batch, nullptr, nsel, kvrows, hsel, hout, st);
        else qm_launch<false, float, kQqTiles, kQqDepth>(a, w, x, batch, nullptr, nsel, kvrows, hsel, hout, st);
      }
    } else if (hsel->bf16) {
      if (t) qm_launch<true, uint16_t, kQmTiles, kQmDepth>(a, w, x, batch, nullptr, nsel, 0, hsel, hout, st);
      else qm_launch<false, uint16_t, kQmTiles, kQmDepth>(a, w, x, batch, nullptr, nsel, 0, hsel, hout, st);
    } else {
      if (t) qm_launch<true, float, kQmTiles, kQmDepth>(a, w, x, batch, nullptr, nsel, 0, hsel, hout, st);
      else qm_launch<false, float, kQmTiles, kQmDepth>(a, w, x, batch, nullptr, nsel, 0, hsel, hout, st);
    }
    KH_LAUNCHED();
  } else if (NB > 1 && hsel) {
    set_error("the batched fused attention block needs hidden a multiple of %d", kQmAlign);
    return KH_ERR_UNSUPPORTED;
  } else {
    static bool attr_set = false;
    if (!attr_set) {
      KH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_qkv_kernel<NB>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds));
      KH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_qkv_kernel<1, true>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds));
      attr_set = true;
    }
    const size_t lds = std::max(sizeof(float) * std::min(NB, kQkvTok) * H,
                                2 * sizeof(int) * (size_t)a->nh);
    if (lds > (size_t)kMaxDynLds) {
      set_error("hidden %d too large to stage %d tokens", H, std::min(NB, kQkvTok));
      return KH_ERR_UNSUPPORTED;
    }
    const int row_base = kv_done ? kvrows : 0;
    if (nrm.w && NB == 1)
      hipLaunchKernelGGL((attn_qkv_kernel<1, true>), dim3((rows - row_base) / kQkvWaves + 1),
                         dim3(64 * kQkvWaves), lds, st, a->wkvq, x, batch, H, kvrows, D, a->nh,
                         heads, nsel, a->y, a->ystride(), a->qrows, a->qrows + qd,
                         a->qrows + qd + 1, nrm.w, nrm.inv, row_base);
    else
      hipLaunchKernelGGL(attn_qkv_kernel<NB>, dim3(rows / kQkvWaves + 1), dim3(64 * kQkvWaves),
                         lds, st, a->wkvq, x, batch, H, kvrows, D, a->nh, heads, nsel, a->y,
                         a->ystride(), a->qrows, a->qrows + qd, a->qrows + qd + 1, nullptr,
                         nullptr, 0);
    KH_LAUNCHED();
  }
  // 2. split-K decode over the cache and the K/V append (then, for batch > 2 or head
  //    lists longer than kOprojMaxSel, the merge of each head's chunks)
  const int ch16 = D == 64 ? attn_chunk<uint16_t, 64>() : D == 128 ? attn_chunk<uint16_t, 128>()
                                                                  : attn_chunk<uint16_t, 256>();
  const int ch32 = D == 64 ? attn_chunk<float, 64>() : D == 128 ? attn_chunk<float, 128>()
                                                               : attn_chunk<float, 256>();
  // worst-case chunk counts (a captured graph replays these launches as the
  // cache grows): BF16 chunks over a full-length prefix, f32 chunks over a
  // full-length rest
  const int n16 = a->kv_f32 ? 0 : ceil_div(a->max_seq, ch16);
  const int nsplit = n16 + ceil_div(a->max_seq, ch32);
  const size_t slots = (size_t)batch * nsel * nsplit;
  float* po = static_cast<float*>(a->po.get(sizeof(float) * slots * D));
  float2* pml = static_cast<float2*>(a->pml.get(sizeof(float2) * slots));
  if (!po || !pml) return KH_ERR_ALLOC;
  // batch <= 2: the merge runs inside the o_proj kernel (for more tokens the
  // separate merge, one block per (entry, token), is faster)
  constexpr int kFoldNB = NB <= 2 ? NB : 2;
  const bool fold = NB <= 2 && nsel <= kOprojMaxSel;
  // qkv_done with hsel (batch 1): the decode kernel selects the heads
  const PredL1View* dsel = qkv_done && NB == 1 && fold ? hsel : nullptr;
  int rc = D == 64 ? attn_decode_launch<64>(a, batch, pos, heads, nsel, nsplit, po, pml, !fold, st, dsel)
         : D == 128 ? attn_decode_launch<128>(a, batch, pos, heads, nsel, nsplit, po, pml, !fold, st, dsel)
                    : attn_decode_launch<256>(a, batch, pos, heads, nsel, nsplit, po, pml, !fold, st, dsel);
  if (rc != KH_OK) return rc;
  // 3. o_proj over the union heads' rows of WoT, then the ordered reduce
  //    (batch > 2: 128-row groups on the BF16 matrix cores)
  constexpr int kDbRowsAttn = 128;
  const bool bf_oproj = !fold && H % kDbCols == 0 && ceil_div(qd, kDbRowsAttn) <= kMaxGroups;
  const int nslices = ceil_div(H, kSlice);
  const int groups = bf_oproj ? ceil_div(qd, kDbRowsAttn) : gather_groups(qd, nslices);
  if (groups == 0) {
    set_error("num_heads*head_dim %d too large for the o_proj gather", qd);
    return KH_ERR_UNSUPPORTED;
  }
  float* partial = static_cast<float*>(a->partial.get(sizeof(float) * groups * NB * H));
  if (!partial) return KH_ERR_ALLOC;
  if (fold)
    hipLaunchKernelGGL(attn_oproj_kernel<kFoldNB>, dim3(nslices, groups), dim3(kOprojThreads), 0,
                       st, a->wot, H, D, a->qrows, qd, a->qrows + qd, po, pml, nsplit, ch16, ch32,
                       a->pre, heads, nsel, a->lens, a->max_seq, batch, groups, partial);
  else if (bf_oproj) {
    static std::once_flag once;
    static hipError_t arc = hipSuccess;
    std::call_once(once, [] {
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&down_bf_kernel<NB, kDbRowsAttn>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)db_lds(kDbRowsAttn));
    });
    KH_HIP(arc);
    hipLaunchKernelGGL((down_bf_kernel<NB, kDbRowsAttn>), dim3(H / kDbCols, groups), dim3(64 * kDbWaves),
                       db_lds(kDbRowsAttn), st, a->wot, H, a->qrows, qd, a->qrows + qd, qd, a->cat, qd, batch,
                       partial);
  } else
    hipLaunchKernelGGL(gather_rows_kernel<NB>, dim3(nslices, groups), dim3(kDownThreads), 0, st,
                       a->wot, H, a->qrows, qd, a->qrows + qd, qd, a->cat, qd, batch, groups,
                       partial);
  KH_LAUNCHED();
  if (groups <= 64)  // few partial rows: 4-wave blocks (16 rows in flight per wave)
    hipLaunchKernelGGL((partials_reduce_kernel<NB, 4>), dim3(ceil_div(H, 64), batch), dim3(64 * 4), 0,
                       st, partial, H, groups, out, accumulate, a->lens, a->max_seq);
  else
    hipLaunchKernelGGL(partials_reduce_kernel<NB>, dim3(ceil_div(H, 64), batch),
                       dim3(64 * kRedWaves), 0, st, partial, H, groups, out, accumulate, a->lens,
                       a->max_seq);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_sparse_attn_forward(kh_sparse_attn* a, const float* x_dev, int64_t batch,
                                      const int64_t* pos_dev, const int32_t* heads_dev,
                                      int n_heads, float* out_dev, int accumulate, void* stream) {
  KH_CHECK_ARG(a && x_dev && out_dev, "null argument");
  KH_CHECK_ARG(batch >= 1 && batch <= a->max_batch, "batch %lld not in [1,%d]", (long long)batch,
               a->max_batch);
  KH_CHECK_ARG(n_heads >= 0 && n_heads <= 4 * a->nh, "n_heads %d not in [0,%d]", n_heads, 4 * a->nh);
  KH_CHECK_ARG(n_heads == 0 || heads_dev, "null head list");
  for (int64_t b = 0; b < batch; ++b)
    if (a->len_host[b] >= a->max_seq) {
      set_error("KV cache of sequence %lld is full (%d positions)", (long long)b, a->max_seq);
      return KH_ERR_CAPACITY;
    }
  hipStream_t st = as_stream(stream);
  // An empty head list is a list whose only entry is skipped.
  static int32_t* none = nullptr;
  if (n_heads == 0) {
    if (!none) {
      none = static_cast<int32_t*>(dev_alloc(sizeof(int32_t) * 16));
      if (!none) return KH_ERR_ALLOC;
      KH_HIP(hipMemset(none, 0xff, sizeof(int32_t) * 16));
    }
    heads_dev = none;
    n_heads = 1;
  }
  const int b = static_cast<int>(batch);
  int rc;
  switch (b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : b <= 8 ? 8 : 16) {
    case 1: rc = attn_launch<1>(a, x_dev, b, pos_dev, heads_dev, n_heads, out_dev, accumulate, st); break;
    case 2: rc = attn_launch<2>(a, x_dev, b, pos_dev, heads_dev, n_heads, out_dev, accumulate, st); break;
    case 4: rc = attn_launch<4>(a, x_dev, b, pos_dev, heads_dev, n_heads, out_dev, accumulate, st); break;
    case 8: rc = attn_launch<8>(a, x_dev, b, pos_dev, heads_dev, n_heads, out_dev, accumulate, st); break;
    default: rc = attn_launch<16>(a, x_dev, b, pos_dev, heads_dev, n_heads, out_dev, accumulate, st); break;
  }
  if (rc == KH_OK)
    for (int64_t i = 0; i < batch; ++i) a->len_host[i] += 1;
  return rc;
}

extern "C" int kh_dejavu_attn_block(const kh_predictor* p, kh_sparse_attn* a, float* hidden_dev,
                                    const float* norm_w_dev, float eps, int k, int32_t* heads_dev,
                                    float* norm_ws_dev, void* stream) {
  KH_CHECK_ARG(p && a && hidden_dev && norm_w_dev && heads_dev && norm_ws_dev, "null argument");
  KH_CHECK_ARG(k >= 1 && k <= a->nh, "k %d not in [1,%d]", k, a->nh);
  KH_CHECK_ARG(predictor_in_dim(p) == a->hidden && predictor_out_dim(p) == a->nh,
               "predictor %d->%d does not match the attention (hidden %d, %d heads)",
               predictor_in_dim(p), predictor_out_dim(p), a->hidden, a->nh);
  KH_CHECK_ARG(a->hidden % 64 == 0 && a->hidden <= 4096,
               "the fused block needs hidden <= 4096 and a multiple of 64 (got %d)", a->hidden);
  if (a->len_host[0] >= a->max_seq) {
    set_error("KV cache of sequence 0 is full (%d positions)", a->max_seq);
    return KH_ERR_CAPACITY;
  }
  hipStream_t st = as_stream(stream);
  NormIn nrm;
  nrm.w = norm_w_dev;
  nrm.inv = norm_ws_dev;
  nrm.eps = eps;
  PredL1View v;
  int rc = predictor_l1_view(p, st, &v);
  if (rc != KH_OK) return rc;
  const int kvrows = 2 * a->kvd();
  const bool overlap = v.in_dim <= kL1LdsIn && kvrows % kQkvWaves == 0;
  if (overlap) {
    // head predictor layer 1 + K/V rows, then layer 2 and the top k, then the Q rows
    static std::once_flag once;
    static hipError_t arc = hipSuccess;
    std::call_once(once, [] {
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_pred_kv_kernel<uint16_t>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kL1LdsBytes);
      if (arc == hipSuccess)
        arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_pred_kv_kernel<float>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kL1LdsBytes);
    });
    KH_HIP(arc);
    const int nl1 = ceil_div(v.hid, kL1Chains);
    // when the head scores fit a wave, the launch also projects the Q rows of
    // every head (the selection, one small kernel after it, then only picks);
    // else the K/V rows, and the Q projection selects after it
    const bool all_q = v.out_dim <= 64 && v.hid <= kAttnSelHid;
    const int prow = all_q ? kvrows + a->nh * a->d : kvrows;
    const int nkv = std::max(1, std::min(attn_device_cus() - nl1, prow / kQkvWaves));
    if (v.bf16)
      hipLaunchKernelGGL(attn_pred_kv_kernel<uint16_t>, dim3(nl1 + nkv), dim3(kL1LdsThreads), kL1LdsBytes,
                         st, static_cast<const uint16_t*>(v.w1b), v.b1, v.hid, v.hbuf, hidden_dev, a->hidden,
                         norm_w_dev, norm_ws_dev, eps, a->wkvq, prow, a->y, nl1);
    else
      hipLaunchKernelGGL(attn_pred_kv_kernel<float>, dim3(nl1 + nkv), dim3(kL1LdsThreads), kL1LdsBytes,
                         st, static_cast<const float*>(v.w1b), v.b1, v.hid, v.hbuf, hidden_dev, a->hidden,
                         norm_w_dev, norm_ws_dev, eps, a->wkvq, prow, a->y, nl1);
    KH_LAUNCHED();
    if (all_q) {
      // the decode kernel's blocks select the heads themselves
      rc = attn_launch<1>(a, hidden_dev, 1, nullptr, heads_dev, k, hidden_dev, 1, st, nrm, true, &v, true);
      if (rc == KH_OK) a->len_host[0] += 1;
      return rc;
    }
    rc = predictor_l2_topk_from_h(p, k, heads_dev, st);
  } else {
    rc = predictor_topk_normed(p, hidden_dev, k, heads_dev, nrm, st);
  }
  if (rc != KH_OK) return rc;
  rc = attn_launch<1>(a, hidden_dev, 1, nullptr, heads_dev, k, hidden_dev, 1, st, nrm, overlap);
  if (rc == KH_OK) a->len_host[0] += 1;
  return rc;
}

extern "C" int kh_dejavu_attn_block_batch(const kh_predictor* p, kh_sparse_attn* a, float* hidden_dev,
                                          int64_t batch, const float* norm_w_dev, float eps, int k,
                                          int32_t* heads_dev, float* norm_ws_dev, void* stream) {
  KH_CHECK_ARG(p && a && hidden_dev && norm_w_dev && heads_dev && norm_ws_dev, "null argument");
  KH_CHECK_ARG(batch >= 1 && batch <= a->max_batch, "batch %lld not in [1,%d]", (long long)batch,
               a->max_batch);
  if (batch == 1)
    return kh_dejavu_attn_block(p, a, hidden_dev, norm_w_dev, eps, k, heads_dev, norm_ws_dev, stream);
  KH_CHECK_ARG(k >= 1 && k <= a->nh, "k %d not in [1,%d]", k, a->nh);
  KH_CHECK_ARG(predictor_in_dim(p) == a->hidden && predictor_out_dim(p) == a->nh,
               "predictor %d->%d does not match the attention (hidden %d, %d heads)",
               predictor_in_dim(p), predictor_out_dim(p), a->hidden, a->nh);
  if (a->hidden % kQmAlign != 0 || a->hidden > kL1LdsIn || a->nh > 64) {
    set_error("the batched fused attention block needs hidden a multiple of %d and at most %d, and at "
              "most 64 heads (got hidden %d, %d heads)", kQmAlign, kL1LdsIn, a->hidden, a->nh);
    return KH_ERR_UNSUPPORTED;
  }
  for (int64_t b = 0; b < batch; ++b)
    if (a->len_host[b] >= a->max_seq) {
      set_error("KV cache of sequence %lld is full (%d positions)", (long long)b, a->max_seq);
      return KH_ERR_CAPACITY;
    }
  hipStream_t st = as_stream(stream);
  NormIn nrm;
  nrm.w = norm_w_dev;
  nrm.inv = norm_ws_dev;
  nrm.eps = eps;
  float* xn = static_cast<float*>(a->xn.get(sizeof(float) * batch * a->hidden));
  if (!xn) return KH_ERR_ALLOC;
  PredL1View v;
  int rc = predictor_l1_view(p, st, &v, batch);
  if (rc != KH_OK) return rc;
  if (v.hid > kAttnSelHid) {
    set_error("the batched fused attention block selects heads of predictors with at most %d hidden "
              "units (got %d)", kAttnSelHid, v.hid);
    return KH_ERR_UNSUPPORTED;
  }
  const int kvrows = 2 * a->kvd();
  const bool kv_done = kvrows % kQmRows == 0 && a->hidden % kQqAlign == 0 && a->wkvq_t;
  if (kv_done) {
    // the head predictor's layer 1 and the K/V rows in one launch, then the
    // selected heads' Q rows
    static std::once_flag once;
    static hipError_t arc = hipSuccess;
    std::call_once(once, [] {
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_pred_kv_mfma_kernel<uint16_t, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kL1LdsBytes);
      if (arc == hipSuccess)
        arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_pred_kv_mfma_kernel<float, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kL1LdsBytes);
    });
    KH_HIP(arc);
    const int nl1 = ceil_div(v.hid, kL1Chains);
    const dim3 g(nl1 * static_cast<unsigned>(batch) + kvrows / kQmRows);
    const int rows = kvrows + a->nh * a->d;
    if (v.bf16)
      hipLaunchKernelGGL((attn_pred_kv_mfma_kernel<uint16_t, true>), g, dim3(kL1LdsThreads), kL1LdsBytes, st,
                         static_cast<const uint16_t*>(v.w1b), v.b1, v.hid, v.hbuf, hidden_dev,
                         static_cast<int>(batch), a->hidden, norm_w_dev, norm_ws_dev, eps, xn, a->wkvq_t, rows,
                         a->y, a->ystride(), nl1);
    else
      hipLaunchKernelGGL((attn_pred_kv_mfma_kernel<float, true>), g, dim3(kL1LdsThreads), kL1LdsBytes, st,
                         static_cast<const float*>(v.w1b), v.b1, v.hid, v.hbuf, hidden_dev,
                         static_cast<int>(batch), a->hidden, norm_w_dev, norm_ws_dev, eps, xn, a->wkvq_t, rows,
                         a->y, a->ystride(), nl1);
    KH_LAUNCHED();
  } else {
    rc = predictor_l1_normed(p, hidden_dev, batch, nrm, xn, st, &v);
    if (rc != KH_OK) return rc;
  }
  const int b = static_cast<int>(batch);
  switch (b <= 2 ? 2 : b <= 4 ? 4 : b <= 8 ? 8 : 16) {
    case 2: rc = attn_launch<2>(a, xn, b, nullptr, heads_dev, k, hidden_dev, 1, st, NormIn{}, kv_done, &v); break;
    case 4: rc = attn_launch<4>(a, xn, b, nullptr, heads_dev, k, hidden_dev, 1, st, NormIn{}, kv_done, &v); break;
    case 8: rc = attn_launch<8>(a, xn, b, nullptr, heads_dev, k, hidden_dev, 1, st, NormIn{}, kv_done, &v); break;
    default: rc = attn_launch<16>(a, xn, b, nullptr, heads_dev, k, hidden_dev, 1, st, NormIn{}, kv_done, &v); break;
  }
  if (rc == KH_OK)
    for (int64_t i = 0; i < batch; ++i) a->len_host[i] += 1;
  return rc;
}
