// ffn.hip -- Deja Vu sparse SwiGLU FFN over an active neuron set (gfx950).
//
// Replaces sparse_mlp::forward_sparse (crates/klearu-llm/src/sparse/sparse_mlp.rs:4-37)
// and Linear::forward_sparse (crates/klearu-llm/src/model/linear.rs:107-114).
//
// HBM layout (BF16, written once at create):
//   Wgu [inter][2][hidden]  gate row then up row of each neuron: one active
//                           neuron is one contiguous 2*hidden*2-byte stretch.
//   WdT [inter][hidden]     down projection transposed, so the down column of
//                           an active neuron is one contiguous row.
// Every weight byte of an active neuron is read exactly once per call with
// 16-byte (dwordx4) loads; that is the algorithmic traffic 3*k*hidden*2 bytes.
//
// Kernels (all loads of a wave are issued before its first wait; the decode
// path is bound by HBM latency and bandwidth, not arithmetic):
//   batch 1:  ffn_fused1   8 active neurons per block; wave w loads the gate
//                          and up rows of neuron w and column slice w of all 8
//                          down rows together, h = silu(g)*u is shared through
//                          LDS, and each wave writes its column slice of the
//                          block's partial row;
//             partials_reduce  adds the partial rows in block order (a kernel
//                          boundary instead of device-scope fences, which on
//                          gfx950 write back and invalidate the whole L2).
//   batch>1:  ffn_gateup_lds (hidden a multiple of 256) 32 active neurons per
//                          block, gate/up rows streamed through LDS with
//                          contiguous loads, 16x16 tiles on MFMA (x split into
//                          BF16 hi/lo); otherwise ffn_gateup, one wave per
//                          active neuron, tokens staged in LDS;
//             down_bf (hidden a multiple of 512; gather.hpp) 256-row groups
//                          x 512-column slices, rows staged transposed through
//                          LDS, BF16 MFMA with h split into hi/lo; otherwise
//                          down_mfma / down_rows / gather_rows;
//             partials_reduce  as above.
// No float atomics: the summation order is fixed, so outputs are deterministic.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "exact_sum.hpp"
#include "gather.hpp"
#include "mfma.hpp"
#include "topk_select.hpp"

namespace kh {


constexpr int kGuWaves = 4;       // neurons per gate/up block
constexpr int kGuChunks = 8;      // 16-byte chunks per lane held in flight (H <= 4096 in one pass)
constexpr int kGuTok = 4;         // tokens staged in LDS at a time

// One wave per active neuron.  x (up to kGuTok tokens at a time) is staged in
// LDS once per block; each lane then issues all of its gate and up loads
// (kGuChunks x 16 B each) before the first use, so a wave keeps 16 KB in
// flight and the whole kernel is one round trip of HBM latency deep.
template <int NB>
__global__ __launch_bounds__(64 * kGuWaves) void ffn_gateup_kernel(
    const uint16_t* __restrict__ Wgu, const float* __restrict__ x, int batch, int H,
    const int32_t* __restrict__ active, int n_active, const int32_t* __restrict__ n_active_dev,
    int inter, int* __restrict__ err, float* __restrict__ hbuf, int hstride) {
  extern __shared__ float4 xs4[];  // [kGuTok][H/4]
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int item = blockIdx.x * kGuWaves + wave;
  if (blockIdx.x * kGuWaves >= n) return;  // whole block idle (uniform)
  const bool live = item < n;
  const int neuron = checked_row(active[live ? item : n - 1], inter, err);
  const uint4* __restrict__ g = reinterpret_cast<const uint4*>(Wgu + (size_t)neuron * 2 * H);
  const uint4* __restrict__ u = g + (H >> 3);
  const int nchunk = H >> 3;
  const int H4 = H >> 2;
  constexpr int TB = NB < kGuTok ? NB : kGuTok;
  float ag[NB], au[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ag[b] = au[b] = 0.0f;
  for (int cbase = 0; cbase < nchunk; cbase += 64 * kGuChunks) {
    uint4 wg[kGuChunks], wu[kGuChunks];
#pragma unroll
    for (int q = 0; q < kGuChunks; ++q) {
      // clamped, branch-free loads: chunks past the row end are never used
      const int c = min(cbase + lane + 64 * q, nchunk - 1);
      wg[q] = ld_stream(g + c);
      wu[q] = ld_stream(u + c);
    }
#pragma unroll
    for (int t0 = 0; t0 < NB; t0 += TB) {
      if (t0 >= batch) break;
      lds_barrier();
      const int nt = min(TB, batch - t0);
      stage_f4(xs4, reinterpret_cast<const float4*>(x + (size_t)t0 * H), nt * H4);
      lds_barrier();
#pragma unroll
      for (int q = 0; q < kGuChunks; ++q) {
        const int c = cbase + lane + 64 * q;
        if (c >= nchunk) break;
        float wgf[8], wuf[8];
        wgf[0] = bf16_lo(wg[q].x); wgf[1] = bf16_hi(wg[q].x); wgf[2] = bf16_lo(wg[q].y); wgf[3] = bf16_hi(wg[q].y);
        wgf[4] = bf16_lo(wg[q].z); wgf[5] = bf16_hi(wg[q].z); wgf[6] = bf16_lo(wg[q].w); wgf[7] = bf16_hi(wg[q].w);
        wuf[0] = bf16_lo(wu[q].x); wuf[1] = bf16_hi(wu[q].x); wuf[2] = bf16_lo(wu[q].y); wuf[3] = bf16_hi(wu[q].y);
        wuf[4] = bf16_lo(wu[q].z); wuf[5] = bf16_hi(wu[q].z); wuf[6] = bf16_lo(wu[q].w); wuf[7] = bf16_hi(wu[q].w);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
          if (t < nt) {
            const float4 x0 = xs4[t * H4 + 2 * c], x1 = xs4[t * H4 + 2 * c + 1];
            const float xf[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const int b = t0 + t;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              ag[b] = fmaf(wgf[e], xf[e], ag[b]);
              au[b] = fmaf(wuf[e], xf[e], au[b]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < batch) {
      const float gs = wave_sum(ag[b]);
      const float us = wave_sum(au[b]);
      if (lane == 0 && live) hbuf[(size_t)b * hstride + item] = silu_ref(gs) * us;
    }
  }
}

// ---------------------------------------------------------------- batched gate/up on MFMA
// Batched gate/up (2..16 tokens) with contiguous weight loads.  A block owns
// kGlRows active neurons (two 16-row MFMA tiles) and streams their gate and
// up rows through LDS in chunks of kGlK columns: every load instruction reads
// 512 contiguous bytes of one row (half a wave per row piece), where loading
// the MFMA operands straight from HBM reads 64 bytes from each of 16 rows per
// instruction.  Wave w then takes k-step w (32 columns) of each chunk for
// both tiles: A from LDS (lane (r, kb) reads row 16t + r, columns 8kb..8kb+7
// of its k-step), B = x of token r split into BF16 hi/lo terms (as in
// ffn_gateup_mfma_kernel), f32 accumulators.  The next chunk's loads are in
// flight while the current one is multiplied (two LDS buffers, one barrier
// per chunk).  The eight waves' k-partial sums are added in wave order
// through LDS at the end, so the result is deterministic.
constexpr int kGlRows = 32;
constexpr int kGlK = 256;
constexpr int kGlMarkPer = 16;  // mark words per thread: intermediate sizes up to 32768
constexpr int kGlWaves = 8;
constexpr int kGlRowQ = kGlK / 8 + 1;                // uint4 per LDS row (one of padding)
constexpr int kGlBuf = 2 * kGlRows * kGlRowQ;        // uint4 per buffer: gate rows, then up rows
constexpr int kGlLds = 2 * kGlBuf * 16;              // two buffers
constexpr int kGlSteps = kGlK / 32 / kGlWaves;     // k-steps of each chunk per wave
constexpr int kGlPer = 2 * kGlRows * (kGlK / 8) / 64 / kGlWaves;  // load instructions per wave per chunk
static_assert(kGlSteps >= 1 && kGlK / 8 <= 64 && 64 % (kGlK / 8) == 0, "chunk layout");
static_assert(kGlWaves * 2 * 4 * 64 * 16 <= kGlLds, "the final reduction fits in the buffers");

__global__ __launch_bounds__(64 * kGlWaves) void ffn_gateup_lds_kernel(
    const uint16_t* __restrict__ Wgu, const float* __restrict__ x, int batch, int H,
    const int32_t* __restrict__ active, int n_active, const int32_t* __restrict__ n_active_dev,
    int inter, int* __restrict__ err, float* __restrict__ hbuf, int hstride,
    const uint32_t* __restrict__ marks = nullptr, int32_t* __restrict__ uni_out = nullptr,
    int32_t* __restrict__ count_out = nullptr) {
  extern __shared__ uint4 gl[];                       // [2][2 * kGlRows][kGlRowQ]
  __shared__ uint64_t s_tab[32];                      // kExp2Tab, for silu after the sums
  __shared__ int s_uid[kGlRows];                      // marks: this block's union ids
  __shared__ int s_ws[kGlWaves];
  __shared__ int s_tot;
  const uint64_t tabv = kExp2Tab[threadIdx.x & 31];   // requested before the weights
  int n = n_active;
  const int base = blockIdx.x * kGlRows;
  if (marks) {
    // The active rows are the union of the byte marks (one byte per neuron, 1
    // when some token selected it), in ascending id order: thread t counts the
    // marks of words [t per, (t + 1) per), a block scan places them, and each
    // block keeps the ids at union positions [base, base + kGlRows) (and writes
    // them to uni_out, block 0 the count, for the down projection).
    const int nwd = (inter + 3) >> 2;
    const int per = (nwd + (int)blockDim.x - 1) / (int)blockDim.x;  // <= kGlMarkPer (host-checked)
    const int w0 = (int)threadIdx.x * per;
    uint32_t wd[kGlMarkPer];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kGlMarkPer; ++j) {
      wd[j] = (j < per && w0 + j < nwd) ? marks[w0 + j] : 0u;
      cnt += __popc(wd[j]);  // set bytes hold 1
    }
    int u = block_excl_scan(cnt, s_ws, &s_tot);
#pragma unroll
    for (int j = 0; j < kGlMarkPer; ++j) {
      uint32_t m = wd[j];
      while (m) {
        const int bit = __ffs(m) - 1;
        if (u >= base && u < base + kGlRows) {
          const int id = 4 * (w0 + j) + (bit >> 3);
          s_uid[u - base] = id;
          uni_out[u] = id;
        }
        ++u;
        m &= m - 1;
      }
    }
    n = s_tot;
    if (blockIdx.x == 0 && threadIdx.x == 0) *count_out = n;
    __syncthreads();
  } else if (n_active_dev) {
    n = min(n, *n_active_dev);
  }
  if (base >= n) return;  // whole block idle (uniform)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // row pieces this lane loads: of the 2*kGlRows pieces (gate rows, then up
  // rows), a load instruction covers kPw pieces of kGlK/8 lanes each; lane
  // reads 16 bytes at column 8*(lane % (kGlK/8))
  constexpr int kQ = kGlK / 8, kPw = 64 / kQ;
  const int half = lane / kQ, col = lane % kQ;
  const uint4* src[kGlPer];
  int dst[kGlPer];
#pragma unroll
  for (int j = 0; j < kGlPer; ++j) {
    const int piece = (wave * kGlPer + j) * kPw + half;
    const int gu = piece / kGlRows, row = piece % kGlRows;
    const int nid = marks ? s_uid[min(row, n - 1 - base)] : checked_row(active[min(base + row, n - 1)], inter, err);
    src[j] = reinterpret_cast<const uint4*>(Wgu + ((size_t)nid * 2 + gu) * H) + col;
    dst[j] = piece * kGlRowQ + col;
  }
  const int nch = H / kGlK;
  uint4 st[kGlPer];
  auto load = [&](int c) {  // clamped past the last chunk (reread, unused)
    const int o = min(c, nch - 1) * (kGlK / 8);
#pragma unroll
    for (int j = 0; j < kGlPer; ++j) st[j] = ld_stream(src[j] + o);
  };
  auto store = [&](int b) {
#pragma unroll
    for (int j = 0; j < kGlPer; ++j) gl[b * kGlBuf + dst[j]] = st[j];
  };
  // B operand: token r (tokens past the batch re-read the last row, unused),
  // columns 32 (w*kGlSteps + s) + 8kb .. +8 of each chunk
  const int r = lane & 15, kb = lane >> 4;
  const float4* __restrict__ xf =
      reinterpret_cast<const float4*>(x + (size_t)min(r, batch - 1) * H) + (32 * wave * kGlSteps + 8 * kb) / 4;
  kh_f32x4 acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[t][a] = kh_f32x4{0, 0, 0, 0};
  // Issue order per wave: x of chunk c + 1 before the weights of chunk c + 2,
  // so that waiting for one chunk's x (vector loads complete in order) never
  // waits for the weights of the chunk after next.
  load(0);
  store(0);
  float4 xn[kGlSteps][2];
#pragma unroll
  for (int s = 0; s < kGlSteps; ++s) {
    xn[s][0] = xf[8 * s];
    xn[s][1] = xf[8 * s + 1];
  }
  load(1);
  lds_barrier();
  for (int c = 0; c < nch; ++c) {
    const uint4* buf = gl + (c & 1) * kGlBuf;
    float4 xc[kGlSteps][2];
    const int cn = min(c + 1, nch - 1);  // past the last chunk: reread, unused
#pragma unroll
    for (int s = 0; s < kGlSteps; ++s) {
      xc[s][0] = xn[s][0];
      xc[s][1] = xn[s][1];
      xn[s][0] = xf[cn * (kGlK / 4) + 8 * s];
      xn[s][1] = xf[cn * (kGlK / 4) + 8 * s + 1];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kGlSteps; ++s) {
      uint4 xh, xl;
      split_bf16x8(xc[s][0], xc[s][1], xh, xl);
      const int q = 4 * (wave * kGlSteps + s) + kb;  // uint4 column of this k-step
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 ag = buf[(16 * t + r) * kGlRowQ + q];
        const uint4 au = buf[(kGlRows + 16 * t + r) * kGlRowQ + q];
        acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ag), as_bf16x8(xh), acc[t][0], 0, 0, 0);
        acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ag), as_bf16x8(xl), acc[t][1], 0, 0, 0);
        acc[t][2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(au), as_bf16x8(xh), acc[t][2], 0, 0, 0);
        acc[t][3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(au), as_bf16x8(xl), acc[t][3], 0, 0, 0);
      }
    }
    // chunk c + 1 into the other buffer (its last readers passed the previous
    // barrier), then chunk c + 2's loads go out
    if (c + 1 < nch) {
      store((c + 1) & 1);
      load(c + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();
  }
  // k-partial sums of the eight waves, added in wave order by waves 0 and 1
  // (tile t = wave); the buffers are free after the last barrier
  kh_f32x4* red = reinterpret_cast<kh_f32x4*>(gl);  // [wave][tile][4][64]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) red[((wave * 2 + t) * 4 + a) * 64 + lane] = acc[t][a];
  if (threadIdx.x < 32) s_tab[threadIdx.x] = tabv;
  lds_barrier();
  if (wave >= 2) return;
  const int t = wave;
  kh_f32x4 tg = {0, 0, 0, 0}, tu = tg;
#pragma unroll
  for (int w = 0; w < kGlWaves; ++w) {
    tg += red[((w * 2 + t) * 4 + 0) * 64 + lane] + red[((w * 2 + t) * 4 + 1) * 64 + lane];
    tu += red[((w * 2 + t) * 4 + 2) * 64 + lane] + red[((w * 2 + t) * 4 + 3) * 64 + lane];
  }
  // C[row][token]: lane holds rows 4kb + q of tile t for token r
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int item = base + 16 * t + 4 * kb + q;
    if (r < batch && item < n) hbuf[(size_t)r * hstride + item] = silu_ref_t(tg[q], s_tab) * tu[q];
  }
}

// Single-token fused FFN: kFuWaves active neurons per block.  Wave w loads the
// gate and up rows of neuron w and, for the down projection, column slice w
// (H/kFuWaves columns) of all kFuWaves neurons' down rows, so every wave has
// 3*H*2 bytes in flight at once.  h = silu(g)*u of each neuron is shared
// through LDS, then each wave adds its column slice over the block's neurons
// in neuron order and writes it to partial[block][H]: no LDS row reduction.
// partials_reduce_kernel adds the partials in block order.
constexpr int kFuWaves = 8;                // neurons (waves) per block; 4 for small hidden sizes
constexpr int kFuWavesMin = 4;
constexpr int kFuMaxH = 4096;              // 8 chunks of 16 B per lane per gate/up row
constexpr int kFuChunks = kFuMaxH / 512;
constexpr int kFuSelKpt = 22;              // scores per thread of the selecting form (11008 / 512; 11 for 5632)
// Dynamic LDS: x [kFuMaxH/4 float4], then h [16 floats] and the block's ids
// [16 ints], then (selecting form) the staged scores.
constexpr int kFuStage = kFuMaxH / 4 + 8;  // float4 offset of the staged scores
constexpr int kFuSelLds = 16 * kFuStage + 4 * kFuSelKpt * 64 * kFuWaves;  // dynamic LDS bound

// The ids of ranks [first, first + NW) of the row's top k, in ascending id
// order (the order of the reference's selection handed to the FFN), chosen by
// this block from the scores alone: every block runs the same exact selection
// (topk_select.hpp) over the same scores, so no block waits for another.  The
// block also writes those ids to active_out.  mm: layer 2's per-block key
// bounds (nmm <= NT pairs).
template <int NW, int KPT>
__device__ __forceinline__ void ffn_select_ids(const float* __restrict__ scores, int n, int k,
                                               const uint32_t* __restrict__ mm, int nmm, int first,
                                               float4* smem4, int32_t* s_ids, TopkLds<64 * NW>& sh,
                                               int32_t* __restrict__ active_out) {
  constexpr int NT = 64 * NW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint2 mmv = (int)threadIdx.x < nmm ? reinterpret_cast<const uint2*>(mm)[threadIdx.x]
                                           : make_uint2(0xffffffffu, 0u);
  // coalesced loads through LDS, then each thread reads its contiguous range
  // (n a multiple of 4, host-checked)
  constexpr int kQ = (KPT + 3) / 4;
  const float4* __restrict__ s4 = reinterpret_cast<const float4*>(scores);
  float4 v[kQ];
#pragma unroll
  for (int q = 0; q < kQ; ++q) v[q] = s4[min((int)threadIdx.x + q * NT, (n >> 2) - 1)];
  {
    const uint32_t a = wave_max_u32(mmv.y), c = wave_min_u32(mmv.x);
    if (lane == 0) {
      sh.wmax[wave] = a;
      sh.wmin[wave] = c;
    }
  }
  float4* stage4 = smem4 + kFuStage;
#pragma unroll
  for (int q = 0; q < kQ; ++q)  // clamped, unconditional (see stage_f4)
    stage4[min((int)threadIdx.x + q * NT, (n >> 2) - 1)] = v[q];
  for (int i = threadIdx.x; i < (1 << kTopkDigit); i += NT) sh.hist[i] = 0;
  if (threadIdx.x == 0) sh.s_ncand = 0;
  lds_barrier();
  const float* stage = reinterpret_cast<const float*>(stage4);
  const int kpt = (n + NT - 1) / NT;  // <= KPT (host-checked)
  const int i0 = threadIdx.x * kpt;
  const int cnt = max(0, min(kpt, n - i0));
  uint32_t key[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) key[j] = f32_key(stage[min(i0 + j, n - 1)]);
  uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mx = max(mx, sh.wmax[w]);
    mn = min(mn, sh.wmin[w]);
  }
  const int kk0 = min(k, n);
  uint32_t T;
  int ties;
  topk_threshold<NT, KPT>(key, cnt, i0, kk0, mx, mn, sh, T, ties);
  int pos;
  auto selm = topk_select_mask<NT, KPT>(key, cnt, T, ties, sh, pos);
  // this thread's selected keys hold ranks pos, pos + 1, ...: keep those in
  // [first, first + NW)
  if (pos < first + NW && pos + (int)__popcll((unsigned long long)selm) > first) {
    int r = pos;
    while (selm && r < first + NW) {
      const int j = __ffsll((unsigned long long)selm) - 1;
      if (r >= first) s_ids[r - first] = i0 + j;
      ++r;
      selm &= selm - 1;
    }
  }
  lds_barrier();
  if ((int)threadIdx.x < NW && first + (int)threadIdx.x < kk0)
    active_out[first + threadIdx.x] = s_ids[threadIdx.x];
}

// KPT > 0: the selecting form (ffn_select_ids): active is not read; the block
// takes ranks [blockIdx.x * NW, ...) of the top n_active of scores[inter].
template <int NW, int KPT = 0>
__global__ __launch_bounds__(64 * NW) void ffn_fused1_kernel(
    const uint16_t* __restrict__ Wgu, const uint16_t* __restrict__ WdT,
    const float* __restrict__ x, int H, const int32_t* __restrict__ active, int n_active,
    const int32_t* __restrict__ n_active_dev, int inter, int* __restrict__ err,
    float* __restrict__ hbuf, float* __restrict__ partial, const float* __restrict__ norm_w,
    const float* __restrict__ norm_inv, const float* __restrict__ scores = nullptr,
    const uint32_t* __restrict__ mm = nullptr, int nmm = 0, int32_t* __restrict__ active_out = nullptr) {
  extern __shared__ float4 smem4[];
  __shared__ uint64_t s_tab[32];                                // kExp2Tab
  float4* xs4 = smem4;                                          // [H/4]
  float* hs = reinterpret_cast<float*>(smem4 + (kFuMaxH >> 2));  // [NW]
  int32_t* s_ids = reinterpret_cast<int32_t*>(hs + 16);         // [NW]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int first = blockIdx.x * NW;
  // the exp table first (vector loads complete in order, so its store below
  // waits for nothing else)
  const uint64_t tabv = kExp2Tab[threadIdx.x & 31];
  // Requests in this order: x and the norm weights (vector loads), then the
  // block's active indices, the device count and the norm scale (scalar
  // loads).  The weight loads go out as soon as the indices arrive; x is
  // waited for after them, which costs nothing because vector loads complete
  // in issue order and x was requested first.
  const int n4 = H >> 2;
  const float4* __restrict__ xsrc = reinterpret_cast<const float4*>(x);
  constexpr int kXq = kFuMaxH / 4 / (64 * NW);  // float4 of x per thread
  float4 xv[kXq], wn[kXq];
#pragma unroll
  for (int q = 0; q < kXq; ++q) xv[q] = xsrc[min((int)threadIdx.x + q * 64 * NW, n4 - 1)];
  // Branch-free requests (without a norm they read x again, unused): a load
  // inside a branch is waited for at the branch's end.
  const float4* __restrict__ nsrc = reinterpret_cast<const float4*>(norm_w ? norm_w : x);
#pragma unroll
  for (int q = 0; q < kXq; ++q) wn[q] = nsrc[min((int)threadIdx.x + q * 64 * NW, n4 - 1)];
  const float inv_ld = *(norm_w ? norm_inv : x);  // unconditional scalar load
  int cand[NW];
  if constexpr (KPT > 0) {
    __shared__ TopkLds<64 * NW> sh;
    ffn_select_ids<NW, KPT>(scores, inter, n_active, mm, nmm, first, smem4, s_ids, sh, active_out);
#pragma unroll
    for (int k = 0; k < NW; ++k) cand[k] = s_ids[k];  // slots past the count: never used
  } else {
#pragma unroll
    for (int k = 0; k < NW; ++k) cand[k] = active[min(first + k, n_active - 1)];
  }
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  // A block past the device count still runs (reading row 0, unused) so that
  // it writes its partial row as zeros for the reduce.
  const int nlive = max(0, min(NW, n - first));
  int nid[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k)  // idle slots read row 0, unused
    nid[k] = k < nlive ? checked_row(cand[k], inter, err) : 0;
  __builtin_amdgcn_sched_barrier(0);
  const int nchunk = H >> 3;
  const int own = nid[wave];
  const uint4* __restrict__ g = reinterpret_cast<const uint4*>(Wgu + (size_t)own * 2 * H);
  const uint4* __restrict__ u = g + nchunk;
  uint4 wg[kFuChunks], wu[kFuChunks], wd[NW];
#pragma unroll
  for (int q = 0; q < kFuChunks; ++q) {
    const int c = min(lane + 64 * q, nchunk - 1);
    wg[q] = ld_stream(g + c);
    wu[q] = ld_stream(u + c);
  }
  // column slice of this wave: H / NW columns, 8 per lane
  const int slice = H / NW;
  const int col = wave * slice + 8 * min(lane, slice / 8 - 1);
#pragma unroll
  for (int k = 0; k < NW; ++k)
    wd[k] = ld_stream(reinterpret_cast<const uint4*>(WdT + (size_t)nid[k] * H + col));
  __builtin_amdgcn_sched_barrier(0);
  if (norm_w) {
    // RmsNorm of the hidden row (model/rms_norm.rs:56-60): (x * inv) * w with
    // the exact scale the predictor's layer 1 computed for this row
    const float inv = inv_ld;
#pragma unroll
    for (int q = 0; q < kXq; ++q) {
      xv[q].x = __fmul_rn(__fmul_rn(xv[q].x, inv), wn[q].x);
      xv[q].y = __fmul_rn(__fmul_rn(xv[q].y, inv), wn[q].y);
      xv[q].z = __fmul_rn(__fmul_rn(xv[q].z, inv), wn[q].z);
      xv[q].w = __fmul_rn(__fmul_rn(xv[q].w, inv), wn[q].w);
    }
  }
  // Unconditional stores (a thread past the end rewrites the last float4 with
  // the value it loaded from there): a conditional store lets the compiler
  // sink each load into its branch, one round trip per load.
#pragma unroll
  for (int q = 0; q < kXq; ++q) xs4[min((int)threadIdx.x + q * 64 * NW, n4 - 1)] = xv[q];
  if (threadIdx.x < 32) s_tab[threadIdx.x] = tabv;
  lds_barrier();
  float ag = 0.0f, au = 0.0f;
#pragma unroll
  for (int q = 0; q < kFuChunks; ++q) {
    const int c = lane + 64 * q;
    if (c < nchunk) {
      const float4 x0 = xs4[2 * c], x1 = xs4[2 * c + 1];
      ag = fmaf(bf16_lo(wg[q].x), x0.x, ag); au = fmaf(bf16_lo(wu[q].x), x0.x, au);
      ag = fmaf(bf16_hi(wg[q].x), x0.y, ag); au = fmaf(bf16_hi(wu[q].x), x0.y, au);
      ag = fmaf(bf16_lo(wg[q].y), x0.z, ag); au = fmaf(bf16_lo(wu[q].y), x0.z, au);
      ag = fmaf(bf16_hi(wg[q].y), x0.w, ag); au = fmaf(bf16_hi(wu[q].y), x0.w, au);
      ag = fmaf(bf16_lo(wg[q].z), x1.x, ag); au = fmaf(bf16_lo(wu[q].z), x1.x, au);
      ag = fmaf(bf16_hi(wg[q].z), x1.y, ag); au = fmaf(bf16_hi(wu[q].z), x1.y, au);
      ag = fmaf(bf16_lo(wg[q].w), x1.z, ag); au = fmaf(bf16_lo(wu[q].w), x1.z, au);
      ag = fmaf(bf16_hi(wg[q].w), x1.w, ag); au = fmaf(bf16_hi(wu[q].w), x1.w, au);
    }
  }
  // wave-uniform values: the exp table lookup inside silu becomes a scalar load
  const float gs = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_sum(ag))));
  const float us = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_sum(au))));
  const float h = wave < nlive ? silu_ref_t(gs, s_tab) * us : 0.0f;
  if (lane == 0) hs[wave] = h;
  if (lane == 0 && wave < nlive && hbuf) hbuf[first + wave] = h;
  lds_barrier();
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    if (k < nlive) {
      const float hk = hs[k];
      acc[0] = fmaf(hk, bf16_lo(wd[k].x), acc[0]); acc[1] = fmaf(hk, bf16_hi(wd[k].x), acc[1]);
      acc[2] = fmaf(hk, bf16_lo(wd[k].y), acc[2]); acc[3] = fmaf(hk, bf16_hi(wd[k].y), acc[3]);
      acc[4] = fmaf(hk, bf16_lo(wd[k].z), acc[4]); acc[5] = fmaf(hk, bf16_hi(wd[k].z), acc[5]);
      acc[6] = fmaf(hk, bf16_lo(wd[k].w), acc[6]); acc[7] = fmaf(hk, bf16_hi(wd[k].w), acc[7]);
    }
  }
  if (8 * lane < slice) {
    float4* o = reinterpret_cast<float4*>(partial + (size_t)blockIdx.x * H + col);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// RmsNorm::forward (crates/klearu-llm/src/model/rms_norm.rs:43-64): one block
// of kRnWaves waves per row.  The row's squares are staged in LDS and summed in
// the reference's sequential order (exact_seq_sum, 32 chunks of M terms); then
// y = (x * inv) * w, and inv_out[row] = inv when inv_out is set.
constexpr int kRnWaves = 8;
constexpr int kRnChunks = 32;
constexpr int kRnMaxN = kRnChunks * 256;  // rows up to 8192 (longer rows: rmsnorm_seq_kernel)

template <int M>
__global__ __launch_bounds__(64 * kRnWaves) void rmsnorm_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ w, int n,
                                                               float eps, float* __restrict__ y,
                                                               float* __restrict__ inv_out = nullptr) {
  __shared__ EsLds<kRnChunks, M> es;
  constexpr int Q = kRnChunks * M / 4 / (64 * kRnWaves);  // float4 of the row per thread
  const float* xr = x + (size_t)blockIdx.x * n;
  float* yr = y + (size_t)blockIdx.x * n;
  const int t = threadIdx.x;
  if ((n & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                        reinterpret_cast<uintptr_t>(y)) & 15) == 0) {
    // Every load of the row and of the weights is requested before the first
    // use (clamped, unconditional: see stage_f4), so the row costs one round
    // trip; four consecutive terms never straddle a chunk (M % 4 == 0).
    const int n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 xv[Q], wv[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) xv[q] = x4[min(t + q * 64 * kRnWaves, n4 - 1)];
#pragma unroll
    for (int q = 0; q < Q; ++q) wv[q] = w4[min(t + q * 64 * kRnWaves, n4 - 1)];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int i4 = t + q * 64 * kRnWaves;
      *reinterpret_cast<float4*>(&es.TP[es_slot<kRnChunks, M>(4 * i4)]) =
          i4 < n4 ? make_float4(__fmul_rn(xv[q].x, xv[q].x), __fmul_rn(xv[q].y, xv[q].y),
                                __fmul_rn(xv[q].z, xv[q].z), __fmul_rn(xv[q].w, xv[q].w))
                  : make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
    }
    lds_barrier();
    const float ss = exact_seq_sum<kRnWaves, kRnChunks, M>(n, 0.0f, es);
    const float inv = rms_inv_exact(ss, n, eps);
    if (inv_out && t == 0) inv_out[blockIdx.x] = inv;
    float4* y4 = reinterpret_cast<float4*>(yr);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int i4 = t + q * 64 * kRnWaves;
      if (i4 < n4)
        y4[i4] = make_float4(__fmul_rn(__fmul_rn(xv[q].x, inv), wv[q].x),
                             __fmul_rn(__fmul_rn(xv[q].y, inv), wv[q].y),
                             __fmul_rn(__fmul_rn(xv[q].z, inv), wv[q].z),
                             __fmul_rn(__fmul_rn(xv[q].w, inv), wv[q].w));
    }
    return;
  }
  for (int i = t; i < kRnChunks * M; i += blockDim.x) {
    const float v = i < n ? xr[i] : 0.0f;
    es.TP[es_slot<kRnChunks, M>(i)] = i < n ? __fmul_rn(v, v) : -0.0f;
  }
  lds_barrier();
  const float ss = exact_seq_sum<kRnWaves, kRnChunks, M>(n, 0.0f, es);
  const float inv = rms_inv_exact(ss, n, eps);
  if (inv_out && t == 0) inv_out[blockIdx.x] = inv;
  for (int i = t; i < n; i += blockDim.x) yr[i] = __fmul_rn(__fmul_rn(xr[i], inv), w[i]);
}

// Rows longer than kRnMaxN: one lane runs the sequential sum.
__global__ __launch_bounds__(256) void rmsnorm_seq_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w, int n,
                                                          float eps, float* __restrict__ y) {
  __shared__ float s_inv;
  const float* xr = x + (size_t)blockIdx.x * n;
  float* yr = y + (size_t)blockIdx.x * n;
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s = __fadd_rn(s, __fmul_rn(xr[i], xr[i]));
    s_inv = rms_inv_exact(s, n, eps);
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = threadIdx.x; i < n; i += blockDim.x) yr[i] = __fmul_rn(__fmul_rn(xr[i], inv), w[i]);
}

}  // namespace kh

using namespace kh;

struct kh_sparse_ffn {
  int hidden = 0, inter = 0, max_batch = 0;
  uint16_t* wgu = nullptr;   // [inter][2][hidden]
  uint16_t* wdt = nullptr;   // [inter][hidden]
  int* err = nullptr;        // set when a call saw an active id outside [0, inter)
  int nslices = 0;
  // per stream: hbuf [max_batch][inter], partial [partial_rows][hidden]
  mutable StreamWs ws;
};

enum { kFwH, kFwPartial, kFwXn, kFwUni, kFwCount };

static size_t partial_rows(int inter, int nbt) {
  return std::max<size_t>((size_t)kMaxGroups * nbt, (size_t)ceil_div(inter, kFuWavesMin));
}

static int ffn_tmpl(int64_t batch) {
  return batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : batch <= 8 ? 8 : 16;
}

extern "C" int kh_sparse_ffn_create(int hidden, int inter, const uint16_t* w_gate_host,
                                    const uint16_t* w_up_host, const uint16_t* w_down_host,
                                    int max_batch, kh_sparse_ffn** out) {
  KH_CHECK_ARG(out && w_gate_host && w_up_host && w_down_host, "null argument");
  KH_CHECK_ARG(hidden > 0 && inter > 0 && hidden % 8 == 0,
               "hidden (%d) must be a positive multiple of 8, inter (%d) positive", hidden, inter);
  KH_CHECK_ARG(max_batch >= 1 && max_batch <= 16, "max_batch %d not in [1,16]", max_batch);
  *out = nullptr;
  auto* f = new kh_sparse_ffn();
  f->hidden = hidden;
  f->inter = inter;
  f->max_batch = max_batch;
  f->nslices = ceil_div(hidden, kSlice);
  const size_t H = hidden, I = inter;
  // Host-side repack into the device layouts.
  uint16_t* gu = static_cast<uint16_t*>(malloc(sizeof(uint16_t) * 2 * H * I));
  uint16_t* dt = static_cast<uint16_t*>(malloc(sizeof(uint16_t) * H * I));
  if (!gu || !dt) {
    free(gu);
    free(dt);
    delete f;
    set_error("host allocation failed");
    return KH_ERR_ALLOC;
  }
  for (size_t i = 0; i < I; ++i) {
    memcpy(gu + i * 2 * H, w_gate_host + i * H, sizeof(uint16_t) * H);
    memcpy(gu + i * 2 * H + H, w_up_host + i * H, sizeof(uint16_t) * H);
  }
  const size_t TB = 64;
  for (size_t j0 = 0; j0 < H; j0 += TB)
    for (size_t i0 = 0; i0 < I; i0 += TB)
      for (size_t j = j0; j < std::min(H, j0 + TB); ++j)
        for (size_t i = i0; i < std::min(I, i0 + TB); ++i) dt[i * H + j] = w_down_host[j * I + i];
  f->wgu = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * 2 * H * I));
  f->wdt = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * H * I));
  f->err = static_cast<int*>(dev_alloc(sizeof(int)));
  int rc = KH_OK;
  if (!f->wgu || !f->wdt || !f->err) rc = KH_ERR_ALLOC;
  if (rc == KH_OK && hipMemset(f->err, 0, sizeof(int)) != hipSuccess) rc = KH_ERR_HIP;
  if (rc == KH_OK) {
    if (hipMemcpy(f->wgu, gu, sizeof(uint16_t) * 2 * H * I, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(f->wdt, dt, sizeof(uint16_t) * H * I, hipMemcpyHostToDevice) != hipSuccess) {
      set_error("weight upload failed");
      rc = KH_ERR_HIP;
    }
  }
  free(gu);
  free(dt);
  if (rc != KH_OK) {
    kh_sparse_ffn_destroy(f);
    return rc;
  }
  *out = f;
  return KH_OK;
}

extern "C" int kh_sparse_ffn_create_dev(int hidden, int inter, const uint16_t* w_gate_dev,
                                        const uint16_t* w_up_dev, const uint16_t* w_down_dev,
                                        int max_batch, kh_sparse_ffn** out) {
  KH_CHECK_ARG(out && w_gate_dev && w_up_dev && w_down_dev, "null argument");
  KH_CHECK_ARG(hidden > 0 && inter > 0 && hidden % 8 == 0,
               "hidden (%d) must be a positive multiple of 8, inter (%d) positive", hidden, inter);
  KH_CHECK_ARG(max_batch >= 1 && max_batch <= 16, "max_batch %d not in [1,16]", max_batch);
  *out = nullptr;
  auto* f = new kh_sparse_ffn();
  f->hidden = hidden;
  f->inter = inter;
  f->max_batch = max_batch;
  f->nslices = ceil_div(hidden, kSlice);
  const size_t H = hidden, I = inter;
  f->wgu = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * 2 * H * I));
  f->wdt = static_cast<uint16_t*>(dev_alloc(sizeof(uint16_t) * H * I));
  f->err = static_cast<int*>(dev_alloc(sizeof(int)));
  if (!f->wgu || !f->wdt || !f->err || hipMemset(f->err, 0, sizeof(int)) != hipSuccess) {
    kh_sparse_ffn_destroy(f);
    return KH_ERR_ALLOC;
  }
  const size_t rowb = sizeof(uint16_t) * H;
  hipError_t e = hipMemcpy2D(f->wgu, 2 * rowb, w_gate_dev, rowb, rowb, I, hipMemcpyDeviceToDevice);
  if (e == hipSuccess)
    e = hipMemcpy2D(f->wgu + H, 2 * rowb, w_up_dev, rowb, rowb, I, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, dim3(ceil_div(I, 32), ceil_div(H, 32)), dim3(256), 0,
                       0, w_down_dev, hidden, inter, f->wdt);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    set_error("device weight repack failed: %s", hipGetErrorString(e));
    kh_sparse_ffn_destroy(f);
    return KH_ERR_HIP;
  }
  *out = f;
  return KH_OK;
}

extern "C" int kh_sparse_ffn_destroy(kh_sparse_ffn* f) {
  if (!f) return KH_OK;
  dev_free(f->wgu);
  dev_free(f->wdt);
  dev_free(f->err);
  delete f;
  return KH_OK;
}

// The stream's h and partial-row buffers of handle f.
static int ffn_bufs(const kh_sparse_ffn* f, hipStream_t st, float** hbuf, float** partial) {
  WsSet* w = f->ws.get(st);
  *hbuf = static_cast<float*>(w->get(kFwH, sizeof(float) * f->max_batch * f->inter));
  *partial = static_cast<float*>(
      w->get(kFwPartial, sizeof(float) * partial_rows(f->inter, ffn_tmpl(f->max_batch)) * f->hidden));
  return *hbuf && *partial ? KH_OK : KH_ERR_ALLOC;
}

// marks (ffn_marks_ok): the active rows are the union of these byte marks,
// computed inside the gate/up kernel, which writes it to active[] and its size
// to n_active_dev (both outputs then); the down kernel clears the marks.
template <int NB>
static int ffn_launch(const kh_sparse_ffn* f, const float* x, int batch, const int32_t* active,
                      int n_active, const int32_t* n_active_dev, float* y, int accumulate,
                      hipStream_t st, const uint8_t* marks = nullptr) {
  const int H = f->hidden;
  float *hbuf = nullptr, *partial = nullptr;
  int rc = ffn_bufs(f, st, &hbuf, &partial);
  if (rc != KH_OK) return rc;
  dim3 g1(ceil_div(n_active, kGuWaves));
  const size_t lds1 = sizeof(float) * std::min(NB, kGuTok) * H;
  static bool attr_set = false;
  if (!attr_set) {
    KH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_gateup_kernel<NB>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds));
    attr_set = true;
  }
  if (lds1 > (size_t)kMaxDynLds) {
    set_error("hidden %d too large for %d staged tokens", H, std::min(NB, kGuTok));
    return KH_ERR_UNSUPPORTED;
  }
  if (NB > 1 && H % kGlK == 0) {
    // several tokens: gate/up as 16 x 16 tile products on MFMA over rows
    // staged through LDS with contiguous loads
    static std::once_flag once;
    static hipError_t arc = hipSuccess;
    std::call_once(once, [] {
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_gateup_lds_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kGlLds);
    });
    KH_HIP(arc);
    hipLaunchKernelGGL(ffn_gateup_lds_kernel, dim3(ceil_div(n_active, kGlRows)), dim3(64 * kGlWaves), kGlLds,
                       st, f->wgu, x, batch, H, active, n_active, n_active_dev, f->inter, f->err, hbuf,
                       f->inter, reinterpret_cast<const uint32_t*>(marks), const_cast<int32_t*>(active),
                       const_cast<int32_t*>(n_active_dev));
  } else if (marks) {
    set_error("the union from marks needs the staged gate/up kernel");
    return KH_ERR_UNSUPPORTED;
  } else {
    hipLaunchKernelGGL(ffn_gateup_kernel<NB>, g1, dim3(64 * kGuWaves), lds1, st, f->wgu, x, batch,
                       H, active, n_active, n_active_dev, f->inter, f->err, hbuf, f->inter);
  }
  KH_LAUNCHED();
  int groups;
  constexpr int kDbRowsFfn = 256;
  if (NB > 1 && H % kDbCols == 0 && ceil_div(n_active, kDbRowsFfn) <= kMaxGroups) {
    // several tokens: 256-row groups on the BF16 matrix cores, weights
    // staged transposed through LDS with contiguous loads
    constexpr int GR = kDbRowsFfn;
    static std::once_flag once;
    static hipError_t arc = hipSuccess;
    std::call_once(once, [] {
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&down_bf_kernel<NB, GR>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)db_lds(GR));
    });
    KH_HIP(arc);
    groups = ceil_div(n_active, GR);
    hipLaunchKernelGGL((down_bf_kernel<NB, GR>), dim3(H / kDbCols, groups), dim3(64 * kDbWaves), db_lds(GR), st,
                       f->wdt, H, active, n_active, n_active_dev, f->inter, hbuf, f->inter, batch, partial,
                       const_cast<uint32_t*>(reinterpret_cast<const uint32_t*>(marks)), (f->inter + 3) >> 2);
  } else if (marks) {
    set_error("the union from marks needs the BF16 down kernel");
    return KH_ERR_UNSUPPORTED;
  } else if (NB > 1 && H % kDmCols == 0) {
    // several tokens: 512-row groups on the matrix cores (f32 MFMA)
    static bool dm_attr = false;
    if (!dm_attr) {
      KH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&down_mfma_kernel<NB>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDmLds));
      dm_attr = true;
    }
    groups = ceil_div(n_active, kDmRows);
    hipLaunchKernelGGL(down_mfma_kernel<NB>, dim3(H / kDmCols, groups), dim3(64 * kDmWaves), kDmLds,
                       st, f->wdt, H, active, n_active, n_active_dev, f->inter, hbuf, f->inter,
                       batch, partial);
  } else if (NB > 1 && H % 8 == 0) {
    // several tokens: 512-row groups streamed with the next rows in flight
    groups = ceil_div(n_active, kDnGroupRows);
    hipLaunchKernelGGL(down_rows_kernel<NB>, dim3(f->nslices, groups), dim3(kDownThreads), 0, st,
                       f->wdt, H, active, n_active, n_active_dev, f->inter, hbuf, f->inter, batch,
                       partial);
  } else {
    groups = gather_groups(n_active, f->nslices);
    if (groups == 0) {
      set_error("n_active %d too large for the down kernel", n_active);
      return KH_ERR_UNSUPPORTED;
    }
    dim3 g2(f->nslices, groups);
    hipLaunchKernelGGL(gather_rows_kernel<NB>, g2, dim3(kDownThreads), 0, st, f->wdt, H, active,
                       n_active, n_active_dev, f->inter, hbuf, f->inter, batch, groups, partial);
  }
  KH_LAUNCHED();
  // few partial rows (at most 64: 4 waves x 16 rows in flight each): 4-wave blocks
  if (groups <= 64)
    hipLaunchKernelGGL((partials_reduce_kernel<NB, 4>), dim3(ceil_div(H, 64), batch), dim3(64 * 4), 0,
                       st, partial, H, groups, y, accumulate, nullptr, 0);
  else
    hipLaunchKernelGGL(partials_reduce_kernel<NB>, dim3(ceil_div(H, 64), batch), dim3(64 * kRedWaves),
                       0, st, partial, H, groups, y, accumulate, nullptr, 0);
  KH_LAUNCHED();
  return KH_OK;
}

static bool ffn_fused_ok(const kh_sparse_ffn* f, int64_t batch) {
  return batch == 1 && f->hidden <= kFuMaxH && f->hidden % (8 * kFuWaves) == 0;
}

// ffn_launch can take the active rows as the union of byte marks (the staged
// gate/up and BF16 down kernels, intermediate sizes up to 32768).
static bool ffn_marks_ok(const kh_sparse_ffn* f, int64_t batch) {
  return batch > 1 && !ffn_fused_ok(f, batch) && f->hidden % kGlK == 0 && f->hidden % kDbCols == 0 &&
         f->inter <= kGlMarkPer * 4 * 64 * kGlWaves && ceil_div(f->inter, 256) <= kMaxGroups;
}

// Four neurons per block when the hidden size allows it (a wave's down slice
// is at most 512 columns) and eight would leave CUs idle: the 1.1B shape
// (hidden 2048, 564 active) gets 141 blocks instead of 71.
static int ffn_fused_wave_count(const kh_sparse_ffn* f, int k) {
  return f->hidden <= 512 * kFuWavesMin && k < 256 * kFuWaves ? kFuWavesMin : kFuWaves;
}
// Whether the fused block's FFN selects its own neurons: always with 8-wave
// blocks (512 threads share the selection), when the row's scores fit
// kFuSelKpt per thread and layer 2's key bounds one slot per thread.  Every
// block then runs the whole selection (about 7 us at the 7B shape, against
// 8.4 us for the one-block top-k kernel and its launch).
static bool ffn_select_ok(const kh_sparse_ffn* f, int k) {
  (void)k;
  constexpr int nt = 64 * kFuWaves;
  return f->inter > 64 && f->inter % 4 == 0 && f->inter < 65536 &&
         ceil_div(f->inter, nt) <= kFuSelKpt && ceil_div(f->inter, 64) <= nt;
}

// Single-token fused FFN + ordered reduce.  With nrm.w set, x is the
// un-normalised hidden row, normalised in the kernel with the scale at nrm.inv.
static int ffn_fused_launch(const kh_sparse_ffn* f, const float* x, const int32_t* active,
                            int n_active, const int32_t* n_active_dev, float* y, int accumulate,
                            const NormIn& nrm, hipStream_t st) {
  const int H = f->hidden;
  float *hbuf = nullptr, *partial = nullptr;
  int rc = ffn_bufs(f, st, &hbuf, &partial);
  if (rc != KH_OK) return rc;
  const int nw = ffn_fused_wave_count(f, n_active);
  const bool small = nw == kFuWavesMin;
  const int blocks = ceil_div(n_active, nw);
  const size_t lds = sizeof(float) * ((size_t)kFuMaxH + kFuWaves);
  static std::once_flag once;
  std::call_once(once, [] {
    hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_fused1_kernel<kFuWaves>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
    hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_fused1_kernel<kFuWavesMin>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
  });
  if (small)
    hipLaunchKernelGGL(ffn_fused1_kernel<kFuWavesMin>, dim3(blocks), dim3(64 * kFuWavesMin), lds, st,
                       f->wgu, f->wdt, x, H, active, n_active, n_active_dev, f->inter, f->err, hbuf,
                       partial, nrm.w, nrm.inv);
  else
    hipLaunchKernelGGL(ffn_fused1_kernel<kFuWaves>, dim3(blocks), dim3(64 * kFuWaves), lds, st,
                       f->wgu, f->wdt, x, H, active, n_active, n_active_dev, f->inter, f->err, hbuf,
                       partial, nrm.w, nrm.inv);
  KH_LAUNCHED();
  partials_reduce_launch(partial, H, blocks, y, accumulate, st);
  KH_LAUNCHED();
  return KH_OK;
}

// The fused block's FFN with its own selection: the top k of the predictor's
// scores (ps) chosen inside the FFN kernel (ffn_select_ids), written to
// active_out, then the same FFN and reduce as ffn_fused_launch.
static int ffn_select_launch(const kh_sparse_ffn* f, const float* x, const PredScores& ps, int k,
                             int32_t* active_out, float* y, int accumulate, const NormIn& nrm,
                             hipStream_t st) {
  const int H = f->hidden;
  if (ps.n != f->inter || !ffn_select_ok(f, k) || ps.nmm > 64 * kFuWaves) {
    set_error("selecting FFN launched outside its limits");
    return KH_ERR_UNSUPPORTED;
  }
  float *hbuf = nullptr, *partial = nullptr;
  int rc = ffn_bufs(f, st, &hbuf, &partial);
  if (rc != KH_OK) return rc;
  const int blocks = ceil_div(k, kFuWaves);
  const size_t lds = sizeof(float4) * kFuStage + sizeof(float) * (size_t)ps.n;
  if (lds > (size_t)kFuSelLds) {
    set_error("selecting FFN: %d scores do not fit its LDS", ps.n);
    return KH_ERR_UNSUPPORTED;
  }
  static std::once_flag once;
  static hipError_t arc = hipSuccess;
  // the kernel's static LDS (the selection's histogram) comes on top of this
  std::call_once(once, [] {
    arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_fused1_kernel<kFuWaves, kFuSelKpt>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kFuSelLds);
    if (arc == hipSuccess)
      arc = hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_fused1_kernel<kFuWaves, kFuSelKpt / 2>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kFuSelLds);
  });
  KH_HIP(arc);
  // half the key registers when they suffice (the 1.1B shape: 5632 scores)
  if (ceil_div(ps.n, 64 * kFuWaves) <= kFuSelKpt / 2)
    hipLaunchKernelGGL((ffn_fused1_kernel<kFuWaves, kFuSelKpt / 2>), dim3(blocks), dim3(64 * kFuWaves), lds,
                       st, f->wgu, f->wdt, x, H, nullptr, k, nullptr, f->inter, f->err, hbuf, partial,
                       nrm.w, nrm.inv, ps.scores, ps.mm, ps.nmm, active_out);
  else
    hipLaunchKernelGGL((ffn_fused1_kernel<kFuWaves, kFuSelKpt>), dim3(blocks), dim3(64 * kFuWaves), lds, st,
                       f->wgu, f->wdt, x, H, nullptr, k, nullptr, f->inter, f->err, hbuf, partial, nrm.w,
                       nrm.inv, ps.scores, ps.mm, ps.nmm, active_out);
  KH_LAUNCHED();
  partials_reduce_launch(partial, H, blocks, y, accumulate, st);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_sparse_ffn_forward(const kh_sparse_ffn* f, const float* x_dev, int64_t batch,
                                     const int32_t* active_dev, int n_active,
                                     const int32_t* n_active_dev, float* y_dev, int accumulate,
                                     void* stream) {
  KH_CHECK_ARG(f && x_dev && y_dev, "null argument");
  KH_CHECK_ARG(batch >= 1 && batch <= f->max_batch, "batch %lld not in [1,%d]", (long long)batch,
               f->max_batch);
  KH_CHECK_ARG(n_active >= 0 && n_active <= f->inter, "n_active %d not in [0,%d]", n_active,
               f->inter);
  hipStream_t st = as_stream(stream);
  if (n_active == 0) {
    if (!accumulate) {
      const int64_t n = batch * f->hidden;
      hipLaunchKernelGGL(fill_f32_kernel<>, dim3(ceil_div(n, 256)), dim3(256), 0, st, y_dev, n, 0.0f);
      KH_LAUNCHED();
    }
    return KH_OK;
  }
  KH_CHECK_ARG(active_dev != nullptr, "null active list");
  const int b = static_cast<int>(batch);
  if (ffn_fused_ok(f, batch))
    return ffn_fused_launch(f, x_dev, active_dev, n_active, n_active_dev, y_dev, accumulate,
                            NormIn{}, st);
  switch (ffn_tmpl(batch)) {
    case 1: return ffn_launch<1>(f, x_dev, b, active_dev, n_active, n_active_dev, y_dev, accumulate, st);
    case 2: return ffn_launch<2>(f, x_dev, b, active_dev, n_active, n_active_dev, y_dev, accumulate, st);
    case 4: return ffn_launch<4>(f, x_dev, b, active_dev, n_active, n_active_dev, y_dev, accumulate, st);
    case 8: return ffn_launch<8>(f, x_dev, b, active_dev, n_active, n_active_dev, y_dev, accumulate, st);
    default: return ffn_launch<16>(f, x_dev, b, active_dev, n_active, n_active_dev, y_dev, accumulate, st);
  }
}

extern "C" int kh_sparse_ffn_last_hidden(const kh_sparse_ffn* f, float* h_dev, int64_t batch,
                                         int n_active, void* stream) {
  KH_CHECK_ARG(f && h_dev, "null argument");
  KH_CHECK_ARG(batch >= 1 && batch <= f->max_batch && n_active >= 0 && n_active <= f->inter,
               "bad batch/n_active");
  hipStream_t st = as_stream(stream);
  float *hbuf = nullptr, *partial = nullptr;
  int rc = ffn_bufs(f, st, &hbuf, &partial);
  if (rc != KH_OK) return rc;
  KH_HIP(hipMemcpy2DAsync(h_dev, sizeof(float) * n_active, hbuf, sizeof(float) * f->inter,
                          sizeof(float) * n_active, batch, hipMemcpyDeviceToDevice, st));
  return KH_OK;
}

extern "C" int kh_sparse_ffn_status(const kh_sparse_ffn* f) {
  KH_CHECK_ARG(f != nullptr, "null argument");
  KH_HIP(hipDeviceSynchronize());
  int v = 0;
  KH_HIP(hipMemcpy(&v, f->err, sizeof(int), hipMemcpyDeviceToHost));
  if (v == 0) return KH_OK;
  KH_HIP(hipMemset(f->err, 0, sizeof(int)));
  set_error("an active neuron id was outside [0, %d) (rows clamped to 0)", f->inter);
  return KH_ERR_ARG;
}

extern "C" int kh_rmsnorm(const float* x_dev, const float* w_dev, int64_t batch, int n, float eps,
                          float* y_dev, void* stream) {
  KH_CHECK_ARG(x_dev && w_dev && y_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && n > 0, "bad shape");
  if (batch == 0) return KH_OK;
  if (n <= kRnChunks * 128)
    hipLaunchKernelGGL(rmsnorm_kernel<128>, dim3(batch), dim3(64 * kRnWaves), 0, as_stream(stream), x_dev,
                       w_dev, n, eps, y_dev);
  else if (n <= kRnMaxN)
    hipLaunchKernelGGL(rmsnorm_kernel<256>, dim3(batch), dim3(64 * kRnWaves), 0, as_stream(stream), x_dev,
                       w_dev, n, eps, y_dev);
  else
    hipLaunchKernelGGL(rmsnorm_seq_kernel, dim3(batch), dim3(256), 0, as_stream(stream), x_dev,
                       w_dev, n, eps, y_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_dejavu_mlp_block(const kh_predictor* p, const kh_sparse_ffn* f, float* hidden_dev,
                                   const float* norm_w_dev, float eps, int k, int32_t* active_dev,
                                   float* norm_ws_dev, void* stream) {
  KH_CHECK_ARG(p && f && hidden_dev && norm_w_dev && active_dev && norm_ws_dev, "null argument");
  KH_CHECK_ARG(k >= 1 && k <= f->inter, "k %d not in [1,%d]", k, f->inter);
  KH_CHECK_ARG(predictor_in_dim(p) == f->hidden && predictor_out_dim(p) == f->inter,
               "predictor %d->%d does not match the FFN (hidden %d, intermediate %d)",
               predictor_in_dim(p), predictor_out_dim(p), f->hidden, f->inter);
  KH_CHECK_ARG(ffn_fused_ok(f, 1) && f->hidden <= 4096,
               "the fused block needs hidden <= 4096 and a multiple of %d", 8 * kFuWaves);
  hipStream_t st = as_stream(stream);
  NormIn nrm;
  nrm.w = norm_w_dev;
  nrm.inv = norm_ws_dev;
  nrm.eps = eps;
  if (ffn_select_ok(f, k)) {
    // layers 1 and 2, then the FFN kernel selects its own neurons
    PredScores ps;
    int rc = predictor_scores_normed(p, hidden_dev, nrm, st, &ps);
    if (rc == KH_OK) return ffn_select_launch(f, hidden_dev, ps, k, active_dev, hidden_dev, 1, nrm, st);
    if (rc != KH_ERR_UNSUPPORTED) return rc;
  }
  int rc = predictor_topk_normed(p, hidden_dev, k, active_dev, nrm, st);
  if (rc != KH_OK) return rc;
  return ffn_fused_launch(f, hidden_dev, active_dev, k, nullptr, hidden_dev, 1, nrm, st);
}

extern "C" int kh_dejavu_mlp_block_batch(const kh_predictor* p, const kh_sparse_ffn* f, float* hidden_dev,
                                         int64_t batch, const float* norm_w_dev, float eps, int k,
                                         int32_t* active_dev, float* norm_ws_dev, void* stream) {
  KH_CHECK_ARG(p && f && hidden_dev && norm_w_dev && active_dev && norm_ws_dev, "null argument");
  KH_CHECK_ARG(batch >= 1 && batch <= f->max_batch, "batch %lld not in [1,%d]", (long long)batch,
               f->max_batch);
  if (batch == 1)
    return kh_dejavu_mlp_block(p, f, hidden_dev, norm_w_dev, eps, k, active_dev, norm_ws_dev, stream);
  KH_CHECK_ARG(k >= 1 && k <= f->inter, "k %d not in [1,%d]", k, f->inter);
  KH_CHECK_ARG(predictor_in_dim(p) == f->hidden && predictor_out_dim(p) == f->inter,
               "predictor %d->%d does not match the FFN (hidden %d, intermediate %d)",
               predictor_in_dim(p), predictor_out_dim(p), f->hidden, f->inter);
  const int H = f->hidden;
  if (H > kRnMaxN) {
    set_error("the batched fused block needs hidden <= %d (got %d)", kRnMaxN, H);
    return KH_ERR_UNSUPPORTED;
  }
  hipStream_t st = as_stream(stream);
  WsSet* w = f->ws.get(st);
  float* xn = static_cast<float*>(w->get(kFwXn, sizeof(float) * f->max_batch * H));
  int32_t* uni = static_cast<int32_t*>(w->get(kFwUni, sizeof(int32_t) * f->inter));
  int32_t* cnt = static_cast<int32_t*>(w->get(kFwCount, sizeof(int32_t)));
  if (!xn || !uni || !cnt) return KH_ERR_ALLOC;
  // the exact RmsNorm of every row, its scale to norm_ws_dev
  if (H <= kRnChunks * 128)
    hipLaunchKernelGGL(rmsnorm_kernel<128>, dim3(batch), dim3(64 * kRnWaves), 0, st, hidden_dev, norm_w_dev, H,
                       eps, xn, norm_ws_dev);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<256>, dim3(batch), dim3(64 * kRnWaves), 0, st, hidden_dev, norm_w_dev, H,
                       eps, xn, norm_ws_dev);
  KH_LAUNCHED();
  // the neurons: each row's top k with byte marks, their union taken inside
  // the FFN's gate/up kernel; else the union kernel and the plain FFN
  const uint8_t* marks = nullptr;
  int rc = KH_ERR_UNSUPPORTED;
  if (ffn_marks_ok(f, batch)) {
    uint8_t* m = nullptr;
    rc = predictor_select_marks(p, xn, batch, k, active_dev, st, &m);
    if (rc != KH_OK && rc != KH_ERR_UNSUPPORTED) return rc;
    marks = m;
  }
  if (rc == KH_ERR_UNSUPPORTED) {
    rc = kh_predictor_select_top_k_union(p, xn, batch, k, active_dev, uni, cnt, stream);
    if (rc != KH_OK) return rc;
  }
  const int b = static_cast<int>(batch);
  switch (ffn_tmpl(batch)) {
    case 2: rc = ffn_launch<2>(f, xn, b, uni, f->inter, cnt, hidden_dev, 1, st, marks); break;
    case 4: rc = ffn_launch<4>(f, xn, b, uni, f->inter, cnt, hidden_dev, 1, st, marks); break;
    case 8: rc = ffn_launch<8>(f, xn, b, uni, f->inter, cnt, hidden_dev, 1, st, marks); break;
    default: rc = ffn_launch<16>(f, xn, b, uni, f->inter, cnt, hidden_dev, 1, st, marks); break;
  }
  if (rc != KH_OK && marks) {
    // the marks must be zero for the next call: clear them where the down kernel did not
    const int nw = (f->inter + 3) >> 2;
    hipLaunchKernelGGL(fill_f32_kernel<>, dim3(ceil_div(nw, 256)), dim3(256), 0, st,
                       reinterpret_cast<float*>(const_cast<uint8_t*>(marks)), (int64_t)nw, 0.0f);
  }
  return rc;
}
