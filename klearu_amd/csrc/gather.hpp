// gather.hpp -- row-gather kernels shared by the sparse FFN and attention.
//
// gather_rows_kernel computes, per column slice and row group, the partial
// sums  sum_r h[b][r] * M[rows[r]][:]  over a list of rows of a [*][H] BF16
// matrix (the down projection over active neurons, the output projection over
// selected heads); partials_reduce_kernel adds the groups' partials in a fixed
// order.  Splitting at a kernel boundary replaces device-scope fences, which
// on gfx950 write back and invalidate the whole L2.
#pragma once

#include "common.hpp"
#include "mfma.hpp"

namespace kh {

constexpr int kSlice = 256;             // output columns per gather block
constexpr int kMaxGroups = 128;         // row groups per slice (partials)
constexpr int kDownThreads = 256;

constexpr int kDownRows = 128;  // max rows per down block (16 per row lane)

// Column slice (256 outputs) x row group.  The group's active ids and h values
// are staged in LDS; every thread then issues all of its (<= 16) row loads of
// 16 bytes before accumulating.  Row lane `sub` (0..7, half a wave each) takes
// rows sub, sub+8, ...; partial sums are reduced across row lanes in LDS and
// written per group; ffn_reduce_kernel then adds the groups' partials in group
// order, so the result is deterministic.
template <int NB>
__global__ __launch_bounds__(kDownThreads) void gather_rows_kernel(
    const uint16_t* __restrict__ WdT, int H, const int32_t* __restrict__ active, int n_active,
    const int32_t* __restrict__ n_active_dev, int nrows, const float* __restrict__ hbuf,
    int hstride, int batch, int groups, float* __restrict__ partial) {
  __shared__ float red[4][NB][kSlice];
  __shared__ int s_ids[kDownRows];
  __shared__ float s_h[NB][kDownRows];
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  const int slice = blockIdx.x, grp = blockIdx.y;
  const int tid = threadIdx.x;
  const int sub = tid >> 5;
  const int cl = tid & 31;
  const int col = slice * kSlice + cl * 8;
  const bool colok = col < H;
  const int per = (n + groups - 1) / groups;
  const int r0 = min(n, grp * per);
  const int r1 = min(n, r0 + per);
  const int nr = r1 - r0;  // <= kDownRows by construction of `groups`
  for (int i = tid; i < nr; i += blockDim.x) s_ids[i] = checked_row(active[r0 + i], nrows, nullptr);
  for (int i = tid; i < nr * NB; i += blockDim.x) {
    const int b = i / nr, r = i - b * nr;
    s_h[b][r] = b < batch ? hbuf[(size_t)b * hstride + r0 + r] : 0.0f;
  }
  __syncthreads();
  constexpr int RPL = kDownRows / 8;  // rows per row lane
  uint4 w[RPL];
#pragma unroll
  for (int m = 0; m < RPL; ++m) {
    const int r = sub + 8 * m;
    w[m] = (r < nr && colok) ? ld_stream(reinterpret_cast<const uint4*>(WdT + (size_t)s_ids[r] * H + col))
                             : make_uint4(0, 0, 0, 0);
  }
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
  __syncthreads();
  const int ocol = slice * kSlice + tid;
  for (int b = 0; b < batch; ++b) {
    const float sm = (red[0][b][tid] + red[1][b][tid]) + (red[2][b][tid] + red[3][b][tid]);
    if (ocol < H) partial[((size_t)grp * NB + b) * H + ocol] = sm;
  }
}

// Down projection of several tokens over many rows: column slice (256
// outputs, 8 per thread) x row group of kDnGroupRows rows.  The group's ids
// and h values are staged in LDS; the rows are then streamed in chunks of 64
// (8 per row lane), the next chunk's loads in flight while the current one is
// accumulated, so one block covers 512 rows and the partial rows written for
// the reduce are few (ceil(n / 512) groups).  Rows past the list end reload
// the last row with h = 0.  The row lanes' sums are added in a fixed order.
constexpr int kDnGroupRows = 512;
constexpr int kDnChunk = 8;  // rows per row lane per chunk

template <int NB>
__global__ __launch_bounds__(kDownThreads) void down_rows_kernel(
    const uint16_t* __restrict__ WdT, int H, const int32_t* __restrict__ active, int n_active,
    const int32_t* __restrict__ n_active_dev, int nrows, const float* __restrict__ hbuf,
    int hstride, int batch, float* __restrict__ partial) {
  constexpr int TB = NB < 4 ? NB : 4;  // tokens per reduction pass
  __shared__ int s_ids[kDnGroupRows];
  __shared__ float s_h[NB][kDnGroupRows];
  __shared__ float red[kDownThreads / 64][TB][kSlice];
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  const int slice = blockIdx.x, grp = blockIdx.y;
  const int tid = threadIdx.x;
  const int r0 = grp * kDnGroupRows;
  const int nr = max(0, min(kDnGroupRows, n - r0));
  for (int i = tid; i < kDnGroupRows; i += kDownThreads)
    s_ids[i] = checked_row(active[min(r0 + i, max(n, 1) - 1)], nrows, nullptr);
  for (int i = tid; i < kDnGroupRows * NB; i += kDownThreads) {
    const int b = i / kDnGroupRows, r = i - b * kDnGroupRows;
    s_h[b][r] = (b < batch && r < nr) ? hbuf[(size_t)b * hstride + r0 + r] : 0.0f;
  }
  __syncthreads();
  const int sub = tid >> 5, cl = tid & 31;
  const int col = min(slice * kSlice + cl * 8, H - 8);  // clamped; columns past H are not written
  float acc[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[b][e] = 0.0f;
  const int nchunks = (nr + 8 * kDnChunk - 1) / (8 * kDnChunk);
  uint4 wa[kDnChunk], wb[kDnChunk];
  auto load = [&](uint4 (&w)[kDnChunk], int c) {
#pragma unroll
    for (int m = 0; m < kDnChunk; ++m) {
      const int r = min(c * 8 * kDnChunk + sub + 8 * m, kDnGroupRows - 1);
      w[m] = *reinterpret_cast<const uint4*>(WdT + (size_t)s_ids[r] * H + col);
    }
  };
  auto accum = [&](const uint4 (&w)[kDnChunk], int c) {
#pragma unroll
    for (int m = 0; m < kDnChunk; ++m) {
      const int r = min(c * 8 * kDnChunk + sub + 8 * m, kDnGroupRows - 1);
      const float wf[8] = {bf16_lo(w[m].x), bf16_hi(w[m].x), bf16_lo(w[m].y), bf16_hi(w[m].y),
                           bf16_lo(w[m].z), bf16_hi(w[m].z), bf16_lo(w[m].w), bf16_hi(w[m].w)};
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float hv = s_h[b][r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[b][e] = fmaf(hv, wf[e], acc[b][e]);
      }
    }
  };
  if (nchunks > 0) load(wa, 0);
  for (int c = 0; c < nchunks; c += 2) {
    load(wb, c + 1);  // past the last chunk: clamped rereads, h = 0
    __builtin_amdgcn_sched_barrier(0);
    accum(wa, c);
    load(wa, c + 2);
    __builtin_amdgcn_sched_barrier(0);
    accum(wb, c + 1);
  }
  // the two row lanes of a wave, then the waves in order
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[b][e] += __shfl_xor(acc[b][e], 32, 64);
  const int wv = tid >> 6;
  const int ocol = slice * kSlice + tid;
#pragma unroll
  for (int b0 = 0; b0 < NB; b0 += TB) {
    if ((tid & 63) < 32) {
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wv][t][cl * 8 + e] = acc[b0 + t][e];
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const float sm = (red[0][t][tid] + red[1][t][tid]) + (red[2][t][tid] + red[3][t][tid]);
      if (ocol < H && b0 + t < batch) partial[((size_t)grp * NB + b0 + t) * H + ocol] = sm;
    }
    __syncthreads();
  }
}

// Down projection of up to 16 tokens on the matrix cores, fed from the
// weight rows as stored (no transpose): v_mfma_f32_16x16x4_f32 takes its B
// operand as B[k][j] = lane 16k + j, so each group of 16 lanes holds 16
// columns of one row -- the natural layout of a 16-byte load per lane.  With
// M = tokens, N = columns and K = four active rows:
//   A[t][k] = h[t][row 4g+k]            (lane l: token l%16, row l/16)
//   B[k][j] = WdT[id(4g+k)][col(j)]     (lane l: row l/16, 8 columns per load)
//   D[t][j] -> lane l holds tokens 4(l/16)+q, column j = l%16, q = 0..3.
// A lane's 16-byte load holds columns c..c+7 of one row; element e of it
// feeds MFMA number e, so MFMA e covers the columns c0 + 8p + e (p = l%16).
// The products are f32 x f32 (no rounding of h or of the weights), so the
// result equals an f32 dot up to summation order.  A block covers 256
// columns (two 128-column halves per lane) and kDmRows rows; its 4 waves
// take contiguous quarters of the rows, keep kDmDepth groups of loads in
// flight, and their sums are added in wave order through LDS.  Rows past the
// device count read the last valid row with h = 0.
constexpr int kDmRows = 512;
constexpr int kDmCols = 256;
constexpr int kDmWaves = 4;
constexpr int kDmDepth = 8;  // 4-row groups of loads in flight per wave
constexpr size_t kDmLds = sizeof(int) * kDmRows +
                          sizeof(float) * (size_t)kDmWaves * 16 * kDmCols;  // ids + max(h, sums)

template <int NB>
__global__ __launch_bounds__(64 * kDmWaves) void down_mfma_kernel(
    const uint16_t* __restrict__ WdT, int H, const int32_t* __restrict__ active, int n_active,
    const int32_t* __restrict__ n_active_dev, int nrows, const float* __restrict__ hbuf,
    int hstride, int batch, float* __restrict__ partial) {
  static_assert(NB <= 16, "16 token rows per MFMA tile");
  extern __shared__ float dm_lds[];
  int* s_ids = reinterpret_cast<int*>(dm_lds);  // [kDmRows]
  float* s_h = dm_lds + kDmRows;                // [kDmRows][16] (then the wave sums)
  float* red = s_h;                             // [kDmWaves][16][kDmCols]
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  const int slice = blockIdx.x, grp = blockIdx.y;
  const int tid = threadIdx.x;
  const int r0 = grp * kDmRows;
  const int nr = max(0, min(kDmRows, n - r0));
  const int last = max(n, 1) - 1;
  if (nr == 0) {
    // a group past the device count contributes zeros (the reduce adds every group)
    for (int t = 0; t < batch; ++t) partial[((size_t)grp * NB + t) * H + slice * kDmCols + tid] = 0.0f;
    return;
  }
  for (int i = tid; i < kDmRows; i += 64 * kDmWaves)
    s_ids[i] = checked_row(active[min(r0 + i, last)], nrows, nullptr);
  lds_barrier();
  const int wave = tid >> 6, lane = tid & 63;
  const int kq = lane >> 4, p = lane & 15;
  const uint16_t* __restrict__ wbase = WdT + (size_t)slice * kDmCols + 8 * p;
  const int ngr = (nr + 3) >> 2;
  const int per = (ngr + kDmWaves - 1) / kDmWaves;
  const int g0 = min(ngr, wave * per), g1 = min(ngr, g0 + per);
  // clamped, unconditional loads: groups past g1 (or a wave's empty range in
  // the last group) reread a valid row, whose h is 0
  constexpr int kSlots = kDmDepth + 1;  // ring: the refill of group j + depth goes out before group j's products
  uint4 wb[kSlots][2];
  auto ldw = [&](int g, uint4(&w)[2]) {
    const int r = min(4 * min(g, max(g1 - 1, 0)) + kq, kDmRows - 1);
    const uint16_t* row = wbase + (size_t)s_ids[r] * H;
    w[0] = ld_stream(reinterpret_cast<const uint4*>(row));
    w[1] = ld_stream(reinterpret_cast<const uint4*>(row + 128));
  };
  // the first groups' weight loads go out before h is staged, so the two
  // round trips overlap
#pragma unroll
  for (int d = 0; d < kDmDepth; ++d) ldw(g0 + d, wb[d]);
  __builtin_amdgcn_sched_barrier(0);
  // h of token t, row r -> s_h[r * 16 + t]; coalesced reads along the rows,
  // every load in flight before the first store
  constexpr int kHPer = kDmRows * 16 / (64 * kDmWaves);
  {
    float v[kHPer];
#pragma unroll
    for (int q = 0; q < kHPer; ++q) {
      const int i = tid + q * 64 * kDmWaves;
      const int t = i / kDmRows, r = i - t * kDmRows;
      v[q] = hbuf[(size_t)min(t, batch - 1) * hstride + min(r0 + r, last)];
    }
#pragma unroll
    for (int q = 0; q < kHPer; ++q) {
      const int i = tid + q * 64 * kDmWaves;
      const int t = i / kDmRows, r = i - t * kDmRows;
      s_h[r * 16 + t] = (t < batch && r < nr) ? v[q] : 0.0f;
    }
  }
  lds_barrier();
  kh_f32x4 acc[2][8];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[c][e] = kh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // Straight-line code over the wave's at most kDmRows / 4 / kDmWaves groups
  // (groups past g1 multiply by h = 0): a loop, or a branch inside one, makes
  // the compiler wait for every load in flight at the loop head, which
  // serialises the prefetch; a branch around it lets the compiler sink the
  // first loads below the h staging.
  constexpr int kPerWave = kDmRows / 4 / kDmWaves;
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    if (j + kDmDepth < kPerWave) ldw(g0 + j + kDmDepth, wb[(j + kDmDepth) % kSlots]);
    const int gd = g0 + j;
    const float hv = s_h[min(4 * gd + kq, kDmRows - 1) * 16 + p];
    const float a = gd < g1 ? hv : 0.0f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint4 w = wb[j % kSlots][c];
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float bv = (e & 1) ? bf16_hi(wv[e >> 1]) : bf16_lo(wv[e >> 1]);
        acc[c][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bv, acc[c][e], 0, 0, 0);
      }
    }
    // keep each group's refill ahead of its products (the scheduler would
    // otherwise move the loads to the end, one round trip per pass)
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // every wave is done with s_h before it is reused for the sums
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[(wave * 16 + 4 * kq + q) * kDmCols + c * 128 + 8 * p + e] = acc[c][e][q];
  __syncthreads();
  const int col = slice * kDmCols + tid;
  for (int t = 0; t < batch; ++t) {
    float sm = 0.0f;
#pragma unroll
    for (int w = 0; w < kDmWaves; ++w) sm += red[(w * 16 + t) * kDmCols + tid];
    partial[((size_t)grp * NB + t) * H + col] = sm;
  }
}

// y[b][j] (=, or +=) sum over g of partial[g][b][j].  A block owns 64 columns;
// its 16 waves take partial rows w, w+16, ... (all loads of a thread issued
// before the first add), then the 16 wave sums are added in wave order, so the
// summation order is fixed for a given number of partial rows.
constexpr int kRedWaves = 16;
// RW waves per block (kRedWaves by default; 4 when there are few partial rows)
template <int NB, int RW = kRedWaves>
__global__ __launch_bounds__(64 * RW) void partials_reduce_kernel(const float* __restrict__ partial,
                                                                    int H, int groups,
                                                                    float* __restrict__ y,
                                                                    int accumulate,
                                                                    int32_t* __restrict__ bump,
                                                                    int bump_limit) {
  __shared__ float sums[RW][64];
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = blockIdx.x * 64 + lane;
  const int jc = min(j, H - 1);
  constexpr int U = 16;
  // the value accumulated into is requested with the partials, not after them
  const float y0 = (accumulate && wave == 0) ? y[(size_t)b * H + jc] : 0.0f;
  float t = 0.0f;
  for (int g0 = wave; g0 < groups; g0 += RW * U) {
    float v[U];
#pragma unroll
    for (int q = 0; q < U; ++q)
      v[q] = partial[((size_t)min(g0 + RW * q, groups - 1) * NB + b) * H + jc];
#pragma unroll
    for (int q = 0; q < U; ++q)
      if (g0 + RW * q < groups) t += v[q];
  }
  sums[wave][lane] = t;
  __syncthreads();
  if (wave == 0) {
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < RW; ++w) tot += sums[w][lane];
    const float yn = accumulate ? y0 + tot : tot;
    if (j < H) y[(size_t)b * H + j] = yn;
  }
  // Optional per-row counter advanced once the row's output is complete
  // (the KV-cache length of decode attention).
  if (bump && blockIdx.x == 0 && threadIdx.x == 0 && bump[b] < bump_limit) bump[b] += 1;
}

// Single-row y (=, or +=) sum over g of partial[g][j] for many partial rows:
// a block owns C columns (C * 4 bytes of each partial row; C = 32 reads whole
// 128-byte lines), so a 4096-wide row spreads over 4096 / C blocks.  Thread t
// adds rows t/C, t/C + 256/C, ... (all loads issued before the first add),
// then the row strips are added in strip order: the summation order is fixed
// for a given number of partial rows.  (A template, so that each translation
// unit including this header keeps its own copy.)
constexpr int kRedCols = 32;
constexpr int kRed16U = 32;     // loads per thread in flight (one pass over up to 256 rows)
template <int C = kRedCols, int U = kRed16U>
__global__ __launch_bounds__(256) void partials_reduce16_kernel(const float* __restrict__ partial, int H,
                                                                 int groups, float* __restrict__ y,
                                                                 int accumulate) {
  constexpr int kStrips = 256 / C;
  __shared__ float sums[kStrips][C];
  const int t = threadIdx.x;
  const int c = t % C, strip = t / C;
  const int j = blockIdx.x * C + c;
  const int jc = min(j, H - 1);
  const float y0 = (accumulate && strip == 0) ? y[jc] : 0.0f;
  float s = 0.0f;
  for (int g0 = strip; g0 < groups; g0 += kStrips * U) {
    float v[U];
#pragma unroll
    for (int q = 0; q < U; ++q) v[q] = partial[(size_t)min(g0 + kStrips * q, groups - 1) * H + jc];
#pragma unroll
    for (int q = 0; q < U; ++q)
      if (g0 + kStrips * q < groups) s += v[q];
  }
  sums[strip][c] = s;
  __syncthreads();
  if (strip == 0) {
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < kStrips; ++r) tot += sums[r][c];
    if (j < H) y[j] = accumulate ? y0 + tot : tot;
  }
}

// One output row from `groups` partial rows of width H: 32-column blocks
// when there are many rows, else 64-column blocks.
inline void partials_reduce_launch(const float* partial, int H, int groups, float* y, int accumulate,
                                   hipStream_t st) {
  if (groups > 64)
    hipLaunchKernelGGL(partials_reduce16_kernel<>, dim3(ceil_div(H, kRedCols)), dim3(256), 0, st, partial, H,
                       groups, y, accumulate);
  else
    hipLaunchKernelGGL((partials_reduce_kernel<1, 4>), dim3(ceil_div(H, 64), 1), dim3(64 * 4), 0, st, partial,
                       H, groups, y, accumulate, nullptr, 0);
}

// dst[i][j] = src[j][i] for a [rows][cols] matrix (32x32 LDS tiles).
// (A template, so that each translation unit including this header keeps its own copy.)
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ src, int rows,
                                                        int cols, T* __restrict__ dst) {
  __shared__ T tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8)
    if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = src[(size_t)(r0 + r) * cols + c0 + tx];
  __syncthreads();
  for (int c = ty; c < 32; c += 8)
    if (c0 + c < cols && r0 + tx < rows) dst[(size_t)(c0 + c) * rows + r0 + tx] = tile[tx][c];
}

// Row groups for gather_rows_kernel: enough blocks to cover the chip, at most
// kDownRows rows each.  Returns 0 when n_rows cannot be covered.
inline int gather_groups(int n_rows, int nslices) {
  int groups = ceil_div(512, nslices);
  groups = groups > ceil_div(n_rows, kDownRows) ? groups : ceil_div(n_rows, kDownRows);
  const int cap = ceil_div(n_rows, 8) > 1 ? ceil_div(n_rows, 8) : 1;
  groups = groups < cap ? groups : cap;
  if (ceil_div(n_rows, groups) > kDownRows || groups > kMaxGroups) return 0;
  return groups;
}

// Down projection of up to 16 tokens on the BF16 matrix cores: the products
// sum_r h[t][r] M[rows[r]][c] as v_mfma_f32_16x16x32_bf16 with h split into
// BF16 hi and lo terms (h = hi + lo + e, |e| <= 2^-17 |h|; the products with
// the BF16 weights are exact in f32), an eighth of the matrix-core time of
// the f32 MFMA.  The MFMA takes 8 consecutive k (here rows) per lane, so each
// 32-row chunk is stored transposed in LDS: wave w loads rows 8 w .. 8 w + 7
// of the chunk (16 bytes of 8 columns per lane, 1 KB per row piece), packs
// each column's 8 values into 16 bytes and writes them at [8-column group]
// [column][8-row block] (column stride kDbE, group stride kDbG: 8 lanes'
// 16-byte writes and 8 lanes' 16-byte operand reads each fall in distinct
// banks).  Block (slice, group): kDbCols columns x GR rows; wave w owns the
// columns [128 w, 128 w + 128) (8 tiles of 16) over every row, so no sum
// across waves is needed.  Chunks are double-buffered: the loads of chunk
// c + 2 are in flight while chunk c is multiplied.  Rows past the group's
// count reread its last row with h = 0.  Partial rows partial[group][token][H]
// as gather_rows_kernel's.  Measured at the 7B shape: batch 16, |U| about
// 7858, 256-row groups: 17.8 us against 21.1 for the same tiling on f32 MFMA
// (B read from row-major LDS); batch 8 o_proj over about 30 heads, 128-row
// groups: 10.2 us against 14.5 for gather_rows_kernel.  Two chunks in flight
// in registers, h staged after the first weight loads, or a slice-major
// weight copy (each block's rows contiguous) changed it by 0.3-0.6 us.
constexpr int kDbCols = 512;
constexpr int kDbChunk = 32;                  // rows per chunk (the MFMA's k)
constexpr int kDbWaves = 4;
constexpr int kDbE = 2 * kDbChunk + 16;       // bytes per column (64 data)
constexpr int kDbG = 8 * kDbE + 16;           // bytes per 8-column group
constexpr int kDbBuf = (kDbCols / 8) * kDbG;  // bytes per chunk buffer
static_assert(kDbChunk == 8 * kDbWaves && kDbCols == 128 * kDbWaves, "tiling");

__host__ __device__ constexpr int db_hs(int GR) { return GR + 8; }  // h row stride (BF16 values)
__host__ __device__ constexpr size_t db_lds(int GR) {
  return 2 * (size_t)kDbBuf + 2 * sizeof(uint16_t) * 16 * db_hs(GR) + sizeof(int) * GR;
}

template <int NB, int GR>
__global__ __launch_bounds__(64 * kDbWaves) void down_bf_kernel(
    const uint16_t* __restrict__ WdT, int H, const int32_t* __restrict__ active, int n_active,
    const int32_t* __restrict__ n_active_dev, int nrows, const float* __restrict__ hbuf,
    int hstride, int batch, float* __restrict__ partial, uint32_t* __restrict__ clear = nullptr,
    int nclear = 0) {
  static_assert(NB <= 16 && GR % kDbChunk == 0, "tiling");
  constexpr int HS = db_hs(GR);
  constexpr int NT = 64 * kDbWaves;
  // clear[0, nclear): words the launch before this one read (the union marks)
  if (clear)
    for (int i = (blockIdx.y * gridDim.x + blockIdx.x) * NT + threadIdx.x; i < nclear;
         i += gridDim.x * gridDim.y * NT)
      clear[i] = 0u;
  extern __shared__ uint4 db_lds_mem[];
  uint8_t* wbuf = reinterpret_cast<uint8_t*>(db_lds_mem);                // [2][kDbBuf]
  uint16_t* s_hh = reinterpret_cast<uint16_t*>(wbuf + 2 * kDbBuf);      // [16][HS]
  uint16_t* s_hl = s_hh + 16 * HS;                                       // [16][HS]
  int* s_ids = reinterpret_cast<int*>(s_hl + 16 * HS);                   // [GR]
  int n = n_active;
  if (n_active_dev) n = min(n, *n_active_dev);
  const int slice = blockIdx.x, grp = blockIdx.y;
  const int tid = threadIdx.x;
  const int r0 = grp * GR;
  const int nr = max(0, min(GR, n - r0));
  if (nr == 0) {
    // a group past the device count contributes zeros (the reduce adds every group)
    for (int t = 0; t < batch; ++t)
      for (int c = tid; c < kDbCols; c += NT) partial[((size_t)grp * NB + t) * H + slice * kDbCols + c] = 0.0f;
    return;
  }
  const int last = n - 1;
  for (int i = tid; i < GR; i += NT) s_ids[i] = checked_row(active[min(r0 + i, last)], nrows, nullptr);
  // h of token t, rows 8 j .. 8 j + 7 -> BF16 hi and lo terms (0 past the batch and past nr)
  for (int i = tid; i < 16 * GR / 8; i += NT) {
    const int t = i / (GR / 8), j = i - t * (GR / 8);
    const float* src = hbuf + (size_t)min(t, batch - 1) * hstride;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = 8 * j + e;
      v[e] = (t < batch && r < nr) ? src[min(r0 + r, last)] : 0.0f;
    }
    uint4 hi, lo;
    split_bf16x8(make_float4(v[0], v[1], v[2], v[3]), make_float4(v[4], v[5], v[6], v[7]), hi, lo);
    *reinterpret_cast<uint4*>(s_hh + t * HS + 8 * j) = hi;
    *reinterpret_cast<uint4*>(s_hl + t * HS + 8 * j) = lo;
  }
  lds_barrier();
  const int wave = tid >> 6, lane = tid & 63;
  const int nch = (nr + kDbChunk - 1) / kDbChunk;
  const uint16_t* __restrict__ wcol = WdT + (size_t)slice * kDbCols + 8 * lane;
  uint4 st[8];
  auto load = [&](int c) {  // clamped: rows past nr reread the last row (h = 0)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(c * kDbChunk + 8 * wave + i, nr - 1);
      st[i] = ld_stream(reinterpret_cast<const uint4*>(wcol + (size_t)s_ids[r] * H));
    }
  };
  // column 8 lane + e of rows 8 wave .. 8 wave + 7 -> 16 bytes at [lane][e][wave]
  auto store = [&](int b) {
    uint8_t* dst = wbuf + b * kDbBuf + lane * kDbG + 16 * wave;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint4 v = st[i];
        w[i] = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
      }
      *reinterpret_cast<uint4*>(dst + e * kDbE) =
          make_uint4(__builtin_amdgcn_perm(w[1], w[0], sel), __builtin_amdgcn_perm(w[3], w[2], sel),
                     __builtin_amdgcn_perm(w[5], w[4], sel), __builtin_amdgcn_perm(w[7], w[6], sel));
    }
  };
  load(0);
  __builtin_amdgcn_sched_barrier(0);
  store(0);
  if (nch > 1) load(1);
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  // operands: A[t][k] = h[t][chunk row k], lane: t = lane % 16, k = 8 (lane / 16) + i;
  // B[k][n] = M[chunk row k][column 128 wave + 16 j + n], n = lane % 16
  const int t = lane & 15, kq = lane >> 4;
  const int bcol = 128 * wave + t;  // + 16 j
  kh_f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = kh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < nch; ++c) {
    const uint8_t* buf = wbuf + (c & 1) * kDbBuf;
    const uint4 ah = *reinterpret_cast<const uint4*>(s_hh + t * HS + c * kDbChunk + 8 * kq);
    const uint4 al = *reinterpret_cast<const uint4*>(s_hl + t * HS + c * kDbChunk + 8 * kq);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int col = bcol + 16 * j;
      const uint4 b = *reinterpret_cast<const uint4*>(buf + (col >> 3) * kDbG + (col & 7) * kDbE + 16 * kq);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ah), as_bf16x8(b), acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al), as_bf16x8(b), acc[j], 0, 0, 0);
    }
    if (c + 1 < nch) {
      store((c + 1) & 1);
      if (c + 2 < nch) load(c + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();
  }
  // C[token 4 kq + q][column 16 j + t]
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int tok = 4 * kq + q;
    if (tok < batch) {
      float* o = partial + ((size_t)grp * NB + tok) * H + slice * kDbCols + bcol;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[16 * j] = acc[j][q];
    }
  }
}

}  // namespace kh
