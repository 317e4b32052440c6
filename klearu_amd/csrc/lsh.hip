// lsh.hip -- SimHash / SRP hashing and the LSH index on the GPU (gfx950).
//
// Replaces HashFamily::hash_dense / hash_sparse (crates/klearu-core/src/hash/
// simhash.rs:75-126, hash/srp.rs:95-161), LshIndexTrait insert / query /
// query_union / clear (crates/klearu-core/src/lsh/index.rs:219-316) and the
// FIFO / reservoir buckets (bucket/fifo.rs:27-33, bucket/reservoir.rs:40-67).
//
// Hashing.  A code bit is the sign of a sequential f32 sum over the input
// dimensions in ascending order, +x where the plane is +1 and -x where it is
// -1.  One thread owns one (table, bit) plane and replays that exact sum over
// the plane's nonzeros (CSR list, ascending dimension), so codes are
// bit-identical to the reference.  SRP is the same computation with a
// different plane distribution.
//
// Large dense batches (index builds and rebuilds) hash on the matrix cores
// instead: x is split into BF16 hi + lo terms, the ternary planes are exact in
// BF16, and v_mfma_f32_16x16x32_bf16 gives every (row, plane) sum S' with
// |S' - S| and |s_seq - S| both below a bound c * sum|x| (S the exact sum,
// s_seq the reference's sequential f32 sum).  Where |S'| exceeds twice that
// bound the sign of s_seq is the sign of S'; every other (row, plane) -- ties
// near zero, non-finite input -- replays the sequential sum in its lane, so
// codes stay bit-identical.
//
// Index build.  Inserting ids in order into L tables is, per bucket, a
// sequence of ids in insertion order.  The build hashes all vectors, sorts the
// (bucket, position) pairs with a stable radix sort so that every bucket's
// inserts are contiguous and in order, then applies them: FIFO (one thread per
// bucket) keeps the last `cap` ids; the reservoir's Algorithm R, whose
// SplitMix64 draws depend only on (count, id), runs one thread per insert, each
// slot keeping the last insert that targeted it.  Buckets are dense
// [L][2^k][cap] u32 with len[L][2^k] and the reservoir insertion count[L][2^k].
//
// Query.  One block per input gathers its L buckets.  When ids are below
// 12288 it counts hits in an LDS array indexed by id and compacts in id
// order; otherwise it sorts the gathered ids in LDS (bitonic) and counts runs.
// Output order is ascending id (the reference returns HashMap order).
#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "lsh_internal.hpp"
#include "mfma.hpp"
#include "rng.hpp"

namespace kh {

constexpr int kHashThreads = 256;   // hash_sparse_kernel
constexpr int kHashBatch = 32;      // plane entries in flight per thread
constexpr int kHashDenseMax = 512;  // hash_dense_kernel threads (one plane each; more planes loop)
constexpr int kQueryThreads = 256;      // query_direct_kernel
constexpr int kQueryBigThreads = 1024;  // query_bitmap_kernel, query_sort_kernel
constexpr int kDirectIds = 12288;  // LDS counting when all ids are below this
constexpr int kQueryBatch = 8;     // bucket entries in flight per thread
constexpr int kMaxTables = 256;    // hash tables per index (one per query thread)
static_assert(kQueryThreads >= kMaxTables && kQueryBigThreads >= kMaxTables,
              "one table per query thread");
constexpr int kMaxGather = 8192;   // L * cap limit of the bitmap and sort paths
constexpr int kGroupWords = 8;     // bitmap words per group offset

// ------------------------------------------------------------------ kernels
__global__ __launch_bounds__(kHashDenseMax) void hash_dense_kernel(
    const int32_t* __restrict__ nnz, const uint32_t* __restrict__ ent_t, int k, int L, int dim,
    const float* __restrict__ x, int64_t ldx, int64_t batch, uint32_t* __restrict__ codes,
    int x_in_lds) {
  extern __shared__ float xs[];
  uint32_t* cw = reinterpret_cast<uint32_t*>(xs + (x_in_lds ? dim : 0));
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  if (x_in_lds)
    for (int d = threadIdx.x; d < dim; d += blockDim.x) xs[d] = xr[d];
  for (int t = threadIdx.x; t < L; t += blockDim.x) cw[t] = 0u;
  __syncthreads();
  const float* xv = x_in_lds ? xs : xr;
  const int P = L * k;
  for (int p = threadIdx.x; p < P; p += blockDim.x) {
    // The plane's entries are requested kHashBatch at a time (the padded rows
    // keep every load in bounds; lanes read adjacent planes, so each load is
    // coalesced) and then added in order: the sum stays sequential.
    float s = 0.0f;
    const int e1 = nnz[p];
    for (int e0 = 0; e0 < e1; e0 += kHashBatch) {
      uint32_t v[kHashBatch];
#pragma unroll
      for (int j = 0; j < kHashBatch; ++j) v[j] = ent_t[(size_t)(e0 + j) * P + p];
      float xd[kHashBatch];
#pragma unroll
      for (int j = 0; j < kHashBatch; ++j) xd[j] = xv[v[j] >> 1];
#pragma unroll
      for (int j = 0; j < kHashBatch; ++j)
        if (e0 + j < e1) s = (v[j] & 1u) ? __fsub_rn(s, xd[j]) : __fadd_rn(s, xd[j]);
    }
    if (s >= 0.0f) atomicOr(&cw[p / k], 1u << (p % k));
  }
  __syncthreads();
  for (int t = threadIdx.x; t < L; t += blockDim.x) codes[row * L + t] = cw[t];
}

// Per-row hashing with the plane signs in LDS (dim <= kHlMaxDim).  Block
// (row, g) hashes tables g*tpb .. g*tpb+tpb-1, i.e. planes q = 0..tpb*k-1 of
// the group, one per thread.  The group's 2-bit signs (kh_hash_family::sg_dev)
// are staged in LDS while the row's nonzero values are compacted in dimension
// order; lane q then adds plane q's term of every compacted value in that
// order, its sign read from LDS.  Two kinds of term are left out against the
// reference's sum over the plane's nonzero coefficients: none (a zero
// coefficient adds +0 here, see below) and those whose x value is zero.
// Adding a zero changes at most the sign of a zero partial sum; every later
// partial sum that is not zero, and the final s >= 0 test (true for either
// zero), come out as before, so the code bits are the reference's.
constexpr int kHlThreads = 256;
constexpr int kHlWaves = kHlThreads / 64;
constexpr int kHlMaxDim = 2048;
constexpr int kHlLoads = 16;   // uint4 sign loads in flight per thread
constexpr int kHlUnroll = 16;  // compacted values per step (the list is padded to a multiple)
constexpr int kHlXIter = kHlMaxDim / kHlThreads;

// Signed 2-bit field of w at bit sh (v_bfe_i32 written out, so that the
// conversion that follows is the signed one).
__device__ __forceinline__ int sfield2(uint32_t w, int sh) {
  int r;
  asm("v_bfe_i32 %0, %1, %2, 2" : "=v"(r) : "v"(w), "v"(sh));
  return r;
}

__host__ __device__ constexpr int hl_pad(int n) { return (n + kHlUnroll - 1) / kHlUnroll * kHlUnroll; }

// At most two blocks fit a CU's LDS at cfg-size groups, so the compiler may
// spend registers on keeping every staging load in flight.
__global__ __launch_bounds__(kHlThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void hash_dense_lds_kernel(
    const uint4* __restrict__ sg, int n4, int nw, int k, int L, int tpb, int dim,
    const float* __restrict__ x, int64_t ldx, uint32_t* __restrict__ codes) {
  extern __shared__ uint4 hl_lds[];
  uint32_t* tab = reinterpret_cast<uint32_t*>(hl_lds);  // [dim][nw] sign words
  uint2* ent = reinterpret_cast<uint2*>(hl_lds + n4);   // (word offset d*nw, x bits), dimension order
  uint32_t* cw = reinterpret_cast<uint32_t*>(ent + hl_pad(dim));
  __shared__ int wcount[kHlWaves];
  const int64_t row = blockIdx.x;
  const int g = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const float* __restrict__ xr = x + row * ldx;
  // Wave w compacts dims [w*span, (w+1)*span): its values come after wave w-1's.
  const int span = (dim + kHlThreads - 1) / kHlThreads * 64;
  // Sign loads first, in flight together with the row's loads.
  const uint4* __restrict__ src = sg + (size_t)g * n4;
  uint4 r[kHlLoads];
#pragma unroll
  for (int j = 0; j < kHlLoads; ++j) r[j] = src[min(j * kHlThreads + t, n4 - 1)];
  // The row's loads are unconditional (clamped) and masked afterwards through
  // an opaque mask, so that the compiler keeps every load in one block, in
  // flight together, instead of branching around them.
  float xv[kHlXIter];
#pragma unroll
  for (int i = 0; i < kHlXIter; ++i) {
    const int d = w * span + i * 64 + lane;
    uint32_t keep = i * 64 < span && d < dim ? ~0u : 0u;
    asm volatile("" : "+v"(keep));
    xv[i] = __uint_as_float(__float_as_uint(xr[min(d, dim - 1)]) & keep);
  }
  // Clamped indices on both sides (the last uint4 is written with its own
  // value by several threads) keep the loads out of branches, all in flight.
  // Two passes cover the largest group (kHlMaxDim * 16 words).
  static_assert(2 * kHlLoads * kHlThreads * 4 >= kHlMaxDim * 16, "sign staging passes");
#pragma unroll
  for (int j = 0; j < kHlLoads; ++j) hl_lds[min(j * kHlThreads + t, n4 - 1)] = r[j];
  if (n4 > kHlLoads * kHlThreads) {
    constexpr int i0 = kHlLoads * kHlThreads;
#pragma unroll
    for (int j = 0; j < kHlLoads; ++j) r[j] = src[min(i0 + j * kHlThreads + t, n4 - 1)];
#pragma unroll
    for (int j = 0; j < kHlLoads; ++j) hl_lds[min(i0 + j * kHlThreads + t, n4 - 1)] = r[j];
  }
  uint64_t m[kHlXIter];
  int cnt = 0;
  bool nf = false;
#pragma unroll
  for (int i = 0; i < kHlXIter; ++i) {
    m[i] = __ballot(xv[i] != 0.0f);
    cnt += __popcll(m[i]);
    nf = nf || !__builtin_isfinite(xv[i]);
  }
  // Count of nonzero values | (1 << 16) if one of them is inf or NaN; every
  // lane stores the same value (no branch).
  wcount[w] = cnt | (__ballot(nf) ? 1 << 16 : 0);
  if (t < tpb) cw[t] = 0u;
  __syncthreads();
  int base = 0, n = 0, nonfinite = 0;
#pragma unroll
  for (int v = 0; v < kHlWaves; ++v) {
    const int c = wcount[v] & 0xffff;
    base += v < w ? c : 0;
    n += c;
    nonfinite |= wcount[v] >> 16;
  }
#pragma unroll
  for (int i = 0; i < kHlXIter; ++i) {
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m[i] >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m[i]), 0));
    if (xv[i] != 0.0f)
      ent[base + below] = make_uint2(static_cast<uint32_t>((w * span + i * 64 + lane) * nw), __float_as_uint(xv[i]));
    base += __popcll(m[i]);
  }
  const int npad = hl_pad(n);
  if (n + t < npad) ent[n + t] = make_uint2(0u, 0u);  // +0.0 terms
  __syncthreads();
  const int Pb = tpb * k;
  const uint32_t* __restrict__ tq = tab + min(t >> 4, nw - 1);
  const int sh = 2 * (t & 15);
  float s = 0.0f;
  if (npad > 0 && !nonfinite) {
    // The 2-bit code read as a signed field is the coefficient (+1, -1, 0),
    // and fma(v, c, s) rounds s + c*v once with c*v exact: s + v, s - v, or
    // s + (+-0) for a finite v.  Sign words are read one group of kHlUnroll
    // ahead and entries two, so LDS latency hides behind the adds.
    const uint4* __restrict__ e4 = reinterpret_cast<const uint4*>(ent);  // two entries each
    constexpr int kQ = kHlUnroll / 2;
    const int last = npad / 2 - kQ;
    // One step: sign words of the next group, entries of the one after, and
    // the adds of the current group.  Three register sets rotate through the
    // roles (current, next, after next) across an unrolled loop of three.
    auto step = [&](const uint4 (&cx)[kQ], const uint32_t (&wx)[kHlUnroll], const uint4 (&cy)[kQ],
                    uint32_t (&wy)[kHlUnroll], uint4 (&cz)[kQ], int e) {
#pragma unroll
      for (int j = 0; j < kQ; ++j) {
        wy[2 * j] = tq[cy[j].x];
        wy[2 * j + 1] = tq[cy[j].z];
      }
#pragma unroll
      for (int j = 0; j < kQ; ++j) cz[j] = e4[min((e + 2 * kHlUnroll) / 2, last) + j];
      // Keeps this step's LDS reads here: left alone, the compiler splits the
      // entry reads and moves the value halves next to their use a step
      // later, which exposes the LDS latency on every step.
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < kQ; ++j) {
        s = __builtin_fmaf(__uint_as_float(cx[j].y), static_cast<float>(sfield2(wx[2 * j], sh)), s);
        s = __builtin_fmaf(__uint_as_float(cx[j].w), static_cast<float>(sfield2(wx[2 * j + 1], sh)), s);
      }
    };
    uint4 c0[kQ], c1[kQ], c2[kQ];
    uint32_t w0[kHlUnroll], w1[kHlUnroll], w2[kHlUnroll];
#pragma unroll
    for (int j = 0; j < kQ; ++j) c0[j] = e4[j];
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      w0[2 * j] = tq[c0[j].x];
      w0[2 * j + 1] = tq[c0[j].z];
    }
#pragma unroll
    for (int j = 0; j < kQ; ++j) c1[j] = e4[min(kQ, last) + j];
    for (int e = 0;;) {
      step(c0, w0, c1, w1, c2, e);
      if ((e += kHlUnroll) >= npad) break;
      step(c1, w1, c2, w2, c0, e);
      if ((e += kHlUnroll) >= npad) break;
      step(c2, w2, c0, w0, c1, e);
      if ((e += kHlUnroll) >= npad) break;
    }
  } else if (npad > 0) {
    // A row with inf or NaN: a zero coefficient must add nothing (0 * inf is
    // NaN), so the term is selected rather than multiplied.
    for (int e0 = 0; e0 < npad; e0 += kHlUnroll) {
      uint2 c[kHlUnroll];
#pragma unroll
      for (int j = 0; j < kHlUnroll; ++j) c[j] = ent[e0 + j];
      uint32_t wd[kHlUnroll];
#pragma unroll
      for (int j = 0; j < kHlUnroll; ++j) wd[j] = tq[c[j].x];
#pragma unroll
      for (int j = 0; j < kHlUnroll; ++j) {
        const uint32_t b = (wd[j] >> sh) & 3u;
        const float v = __uint_as_float(c[j].y);
        s = __fadd_rn(s, b == 1u ? v : (b == 3u ? -v : 0.0f));  // s - v is s + (-v) exactly
      }
    }
  }
  const int l0 = g * tpb;
  if (t < Pb && l0 * k + t < L * k && s >= 0.0f) atomicOr(&cw[t / k], 1u << (t % k));
  __syncthreads();
  if (t < tpb && l0 + t < L) codes[row * L + l0 + t] = cw[t];
}

// Matrix-core hashing: a block of 4 waves hashes 64 rows; wave w owns rows
// 16w..16w+15 and walks the plane tiles (16 planes each) in groups of kHmGroup
// accumulators.  Operands follow mfma.hpp: A = x rows (lane l: row l % 16,
// k (l / 16) * 8 + i), B = planes from the tiled copy bt (the 16 bytes lane l
// feeds), C = row (l / 16) * 4 + q, plane l % 16 of the tile.  A (row, plane)
// whose sign the bound does not settle is queued in LDS and replayed after the
// matrix phase by all threads of the block at once (in place if the queue is
// full), so the rare replays do not serialise the waves.
constexpr int kHmRows = 64;
constexpr int kHmGroup = 8;
constexpr int kHmMaxPlanes = 1024;
constexpr int kHmMaxDim = 8192;
constexpr int kHmQueue = 1024;          // queued replays per block
constexpr int kHmBatch = 8;             // plane entries in flight per replay
constexpr int64_t kHmMinBatch = 1024;   // smaller batches take the per-plane kernel

// Eight x values of row xr at dims d0..d0+7 (0 past dim); VEC: two aligned
// float4 loads (dim a multiple of 32, rows 16-byte aligned).
template <bool VEC>
__device__ __forceinline__ void hm_load8(const float* __restrict__ xr, int d0, int dim, float4& a, float4& b) {
  if constexpr (VEC) {
    a = *reinterpret_cast<const float4*>(xr + d0);
    b = *reinterpret_cast<const float4*>(xr + d0 + 4);
  } else {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float t = xr[min(d0 + i, dim - 1)];
      v[i] = d0 + i < dim ? t : 0.0f;
    }
    a = make_float4(v[0], v[1], v[2], v[3]);
    b = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// The reference's sequential sum for one (row, plane): its sign bit.
__device__ __forceinline__ bool hm_replay(const float* __restrict__ xr, const int32_t* __restrict__ nnz,
                                          const uint32_t* __restrict__ ent_t, int P, int pl) {
  float s = 0.0f;
  const int e1 = nnz[pl];
  for (int e0 = 0; e0 < e1; e0 += kHmBatch) {
    uint32_t v[kHmBatch];
    float xd[kHmBatch];
#pragma unroll
    for (int j = 0; j < kHmBatch; ++j) v[j] = ent_t[(size_t)min(e0 + j, e1 - 1) * P + pl];
#pragma unroll
    for (int j = 0; j < kHmBatch; ++j) xd[j] = xr[v[j] >> 1];
#pragma unroll
    for (int j = 0; j < kHmBatch; ++j)
      if (e0 + j < e1) s = (v[j] & 1u) ? __fsub_rn(s, xd[j]) : __fadd_rn(s, xd[j]);
  }
  return s >= 0.0f;
}

template <bool VEC>
__global__ __launch_bounds__(256) void hash_dense_mfma_kernel(
    const uint4* __restrict__ bt, int ksteps, int ntiles, const int32_t* __restrict__ nnz,
    const uint32_t* __restrict__ ent_t, int k, int L, int dim, const float* __restrict__ x,
    int64_t ldx, int64_t batch, uint32_t* __restrict__ codes) {
  constexpr int kW = kHmMaxPlanes / 32 + 1;  // 32-plane words per row (one spare for the code window)
  __shared__ uint32_t pm[kHmRows][kW];
  __shared__ uint32_t queue[kHmQueue];
  __shared__ int nq;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int P = L * k;
  const int64_t rb = (int64_t)blockIdx.x * kHmRows;
  const int64_t r0 = rb + wave * 16;
  for (int i = threadIdx.x; i < kHmRows * kW; i += blockDim.x) (&pm[0][0])[i] = 0u;
  if (threadIdx.x == 0) nq = 0;
  // A operand row of this lane (rows past the batch repeat the last one)
  const float* __restrict__ xa = x + min(r0 + (lane & 15), batch - 1) * ldx;
  const int kq = (lane >> 4) * 8;
  // sum |x| of row lane % 16 (the four lanes of a row hold disjoint k ranges),
  // then of the lane's four output rows
  float ax = 0.0f;
  for (int st = 0; st < ksteps; ++st) {
    float4 a, b;
    hm_load8<VEC>(xa, st * 32 + kq, dim, a, b);
    ax += (fabsf(a.x) + fabsf(a.y)) + (fabsf(a.z) + fabsf(a.w)) + (fabsf(b.x) + fabsf(b.y)) + (fabsf(b.z) + fabsf(b.w));
  }
  ax += __shfl_xor(ax, 16);
  ax += __shfl_xor(ax, 32);
  // Bound on |S' - S| + |s_seq - S| per unit of sum|x|, generous: the lo term's
  // residual (2^-17), the matrix cores' f32 accumulation over 2 * 32 * ksteps
  // products (an ulp per add), the sequential sum's dim adds (half an ulp each),
  // doubled; plus an absolute term for denormals flushed by the matrix cores.
  const float rel = 2.0f * (0x1p-17f + (float)(2 * 32 * ksteps + dim) * 0x1p-23f);
  const float abs_t = (float)(4 * 32 * ksteps + 16) * 0x1p-120f;
  float bound[4];
  bool fin[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float a = __shfl(ax, (lane >> 4) * 4 + q);
    bound[q] = a * 1.01f * rel + abs_t;
    fin[q] = a < 1e37f;   // also false for inf / NaN
  }
  __syncthreads();
  for (int g0 = 0; g0 < ntiles; g0 += kHmGroup) {
    kh_f32x4 c[kHmGroup];
#pragma unroll
    for (int t = 0; t < kHmGroup; ++t) c[t] = kh_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // operands of step st + 1 are requested before the products of step st
    float4 xa0, xb0;
    uint4 w0[kHmGroup];
    auto load = [&](int st, float4& a, float4& b, uint4 (&w)[kHmGroup]) {
      hm_load8<VEC>(xa, st * 32 + kq, dim, a, b);
      const uint4* __restrict__ bp = bt + ((size_t)st * ntiles + g0) * 64 + lane;
#pragma unroll
      for (int t = 0; t < kHmGroup; ++t) w[t] = bp[(size_t)min(t, ntiles - 1 - g0) * 64];
    };
    load(0, xa0, xb0, w0);
    for (int st = 0; st < ksteps; ++st) {
      float4 xa1, xb1;
      uint4 w1[kHmGroup];
      load(min(st + 1, ksteps - 1), xa1, xb1, w1);
      uint4 hi, lo;
      split_bf16x8(xa0, xb0, hi, lo);
#pragma unroll
      for (int t = 0; t < kHmGroup; ++t) {
        c[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(hi), as_bf16x8(w0[t]), c[t], 0, 0, 0);
        c[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(lo), as_bf16x8(w0[t]), c[t], 0, 0, 0);
      }
      xa0 = xa1;
      xb0 = xb1;
#pragma unroll
      for (int t = 0; t < kHmGroup; ++t) w0[t] = w1[t];
    }
#pragma unroll
    for (int t = 0; t < kHmGroup; ++t) {
      const int tile = g0 + t;
      if (tile >= ntiles) break;
      const int pl = tile * 16 + (lane & 15);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = wave * 16 + (lane >> 4) * 4 + q;  // row within the block
        const float sv = c[t][q];
        bool bit = sv > 0.0f;
        if (!(fin[q] && fabsf(sv) > bound[q]) && pl < P && rb + rr < batch) {
          const int slot = atomicAdd(&nq, 1);
          if (slot < kHmQueue) {
            queue[slot] = ((uint32_t)rr << 16) | (uint32_t)pl;
            bit = false;   // set by the replay below
          } else {
            bit = hm_replay(x + (rb + rr) * ldx, nnz, ent_t, P, pl);
          }
        }
        const uint64_t m = __ballot(bit && pl < P);
        if (lane < 4 && (m >> (16 * lane)) & 0xffffull)
          atomicOr(&pm[wave * 16 + lane * 4 + q][tile >> 1], (uint32_t)((m >> (16 * lane)) & 0xffffull) << (16 * (tile & 1)));
      }
    }
  }
  __syncthreads();
  const int nrep = min(nq, kHmQueue);
  for (int i = threadIdx.x; i < nrep; i += blockDim.x) {
    const uint32_t e = queue[i];
    const int rr = (int)(e >> 16), pl = (int)(e & 0xffffu);
    if (hm_replay(x + (rb + rr) * ldx, nnz, ent_t, P, pl)) atomicOr(&pm[rr][pl >> 5], 1u << (pl & 31));
  }
  __syncthreads();
  // codes: table t takes planes t*k .. t*k+k-1 of its row
  for (int i = threadIdx.x; i < kHmRows * L; i += blockDim.x) {
    const int r = i / L, t = i % L;
    if (rb + r >= batch) continue;
    const int p0 = t * k, w0 = p0 >> 5;
    const uint64_t win = (uint64_t)pm[r][w0] | ((uint64_t)pm[r][w0 + 1] << 32);
    codes[(rb + r) * L + t] = (uint32_t)((win >> (p0 & 31)) & ((1ull << k) - 1ull));
  }
}

// One block per (row, group of whole tables): each thread owns one plane of
// the group and walks the row's entries in stored order, kHashSparseBatch at
// a time (the entries' loads are the same for every lane; the plane bytes of
// a batch are all in flight), adding +-x in order: the sum stays sequential.
constexpr int kHashSparseBatch = 16;
__global__ __launch_bounds__(kHashThreads) void hash_sparse_kernel(
    const int8_t* __restrict__ planes, int k, int L, int dim, const int64_t* __restrict__ xoff,
    const uint32_t* __restrict__ xidx, const float* __restrict__ xval,
    uint32_t* __restrict__ codes) {
  __shared__ uint32_t cw[kHashThreads];
  const int64_t row = blockIdx.x;
  const int tpb = kHashThreads / k;           // tables per block
  const int t0 = blockIdx.y * tpb, t1 = min(L, t0 + tpb);
  const int64_t a = xoff[row], b = xoff[row + 1];
  for (int t = threadIdx.x; t < t1 - t0; t += blockDim.x) cw[t] = 0u;
  __syncthreads();
  const int p = t0 * k + threadIdx.x;
  if (p < t1 * k) {
    const int8_t* pl = planes + (size_t)p * dim;
    float s = 0.0f;
    for (int64_t e0 = a; e0 < b; e0 += kHashSparseBatch) {
      int8_t r[kHashSparseBatch];
      float xv[kHashSparseBatch];
#pragma unroll
      for (int j = 0; j < kHashSparseBatch; ++j) {
        const int64_t e = min(e0 + j, b - 1);
        xv[j] = xval[e];
        r[j] = pl[xidx[e]];
      }
#pragma unroll
      for (int j = 0; j < kHashSparseBatch; ++j) {
        if (e0 + j < b) {
          if (r[j] == 1) s = __fadd_rn(s, xv[j]);
          else if (r[j] == -1) s = __fsub_rn(s, xv[j]);
        }
      }
    }
    if (s >= 0.0f) atomicOr(&cw[p / k - t0], 1u << (p % k));
  }
  __syncthreads();
  for (int t = threadIdx.x; t < t1 - t0; t += blockDim.x) codes[row * L + t0 + t] = cw[t];
}

// (bucket key, insertion position) pairs: key = t * 2^k + (code_t & mask).
__global__ void build_keys_kernel(const uint32_t* __restrict__ codes, int64_t n, int L, int k,
                                  uint32_t* __restrict__ keys, uint32_t* __restrict__ pos) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n * L) return;
  const int t = (int)(q % L);
  const uint32_t mask = (1u << k) - 1u;
  keys[q] = ((uint32_t)t << k) | (codes[q] & mask);
  pos[q] = (uint32_t)(q / L);
}

__global__ void seg_bounds_kernel(const uint32_t* __restrict__ skeys, int64_t m,
                                  uint32_t* __restrict__ start, uint32_t* __restrict__ end) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= m) return;
  const uint32_t key = skeys[j];
  if (j == 0 || skeys[j - 1] != key) start[key] = (uint32_t)j;
  if (j == m - 1 || skeys[j + 1] != key) end[key] = (uint32_t)(j + 1);
}

__device__ __forceinline__ uint64_t splitmix_mod(uint64_t seed, uint64_t bound) {
  uint64_t z = seed + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z = z ^ (z >> 31);
  return z % bound;
}

__global__ void fifo_apply_kernel(int nbuckets, int cap, const uint32_t* __restrict__ start,
                                  const uint32_t* __restrict__ end,
                                  const uint32_t* __restrict__ spos,
                                  const uint32_t* __restrict__ ids, uint32_t* __restrict__ data,
                                  uint32_t* __restrict__ len) {
  const int key = blockIdx.x * blockDim.x + threadIdx.x;
  if (key >= nbuckets) return;
  const uint32_t s = start[key], e = end[key];
  if (e <= s) return;
  uint32_t* d = data + (size_t)key * cap;
  const uint32_t l = len[key];
  const uint32_t m = e - s;
  const uint32_t total = l + m;
  const uint32_t keep = min(total, (uint32_t)cap);
  const uint32_t drop = total - keep;
  uint32_t o = 0;
  for (uint32_t q = drop; q < l; ++q) d[o++] = d[q];
  const uint32_t skip = drop > l ? drop - l : 0u;
  for (uint32_t j = s + skip; j < e; ++j) d[o++] = ids[spos[j]];
  len[key] = keep;
}

// Reservoir inserts in parallel (ReservoirBucket::insert, bucket/reservoir.rs:
// 50-67).  Insert j of a bucket's run happens at count c0 + j + 1; it pushes
// into slot len0 + j while the bucket is not full, and otherwise replaces the
// slot the reference's two draws pick, or nothing.  The draws depend only on
// (count, id), so every insert's target is known up front and a slot ends up
// holding the last insert that targeted it: each insert records j + 1 with
// atomicMax, then one thread per slot copies the winner's id.
__global__ void reservoir_targets_kernel(int64_t m, int cap, const uint32_t* __restrict__ skeys,
                                         const uint32_t* __restrict__ start,
                                         const uint32_t* __restrict__ spos,
                                         const uint32_t* __restrict__ ids,
                                         const uint32_t* __restrict__ len,
                                         const uint64_t* __restrict__ count,
                                         uint32_t* __restrict__ last) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const uint32_t key = skeys[i];
  const uint32_t j = (uint32_t)(i - start[key]);
  const uint32_t l0 = len[key];
  const uint32_t id = ids[spos[i]];
  uint32_t slot = 0xffffffffu;
  if (l0 < (uint32_t)cap && j < (uint32_t)cap - l0) {
    slot = l0 + j;
  } else {
    const uint64_t c = count[key] + j + 1;
    const uint64_t seed = c * 0x517cc1b727220a95ull + (uint64_t)id;
    if (splitmix_mod(seed, c) < (uint64_t)cap) slot = (uint32_t)splitmix_mod(seed + 1, (uint64_t)cap);
  }
  if (slot != 0xffffffffu) atomicMax(&last[(size_t)key * cap + slot], j + 1u);
}

__global__ void reservoir_apply_kernel(int64_t nslots, int cap, const uint32_t* __restrict__ start,
                                       const uint32_t* __restrict__ end,
                                       const uint32_t* __restrict__ spos,
                                       const uint32_t* __restrict__ ids,
                                       const uint32_t* __restrict__ last, uint32_t* __restrict__ data,
                                       uint32_t* __restrict__ len, uint64_t* __restrict__ count) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nslots) return;
  const int64_t key = q / cap;
  const uint32_t s = start[key], e = end[key];
  if (e <= s) return;
  const uint32_t w = last[q];
  if (w) data[q] = ids[spos[s + w - 1]];
  if (q % cap == 0) {
    len[key] = min((uint32_t)cap, len[key] + (e - s));
    count[key] += e - s;
  }
}

// Bucket::remove (bucket/fifo.rs:35-42, bucket/reservoir.rs:69-76) of the ids
// routed to each bucket, in call order: the first entry equal to the id is
// replaced by the bucket's last entry (swap_remove); insertion counts stay.
__global__ void remove_buckets_kernel(int nbuckets, int cap, const uint32_t* __restrict__ start,
                                      const uint32_t* __restrict__ end,
                                      const uint32_t* __restrict__ spos,
                                      const uint32_t* __restrict__ ids, uint32_t* __restrict__ data,
                                      uint32_t* __restrict__ len) {
  const int key = blockIdx.x * blockDim.x + threadIdx.x;
  if (key >= nbuckets) return;
  const uint32_t s = start[key], e = end[key];
  if (e <= s) return;
  uint32_t* d = data + (size_t)key * cap;
  uint32_t l = len[key];
  for (uint32_t j = s; j < e; ++j) {
    const uint32_t id = ids[spos[j]];
    for (uint32_t q = 0; q < l; ++q)
      if (d[q] == id) {
        d[q] = d[l - 1];
        --l;
        break;
      }
  }
  len[key] = l;
}

// LshIndexTrait::remove (lsh/index.rs:279-281 -> BucketStorage::remove_all,
// :146-164): every bucket removes each listed id (its first occurrence) in
// list order.  A bucket holding no listed id (bitmap over [0, bound)) is left
// untouched; the others replay the list.
__global__ void remove_all_kernel(int nbuckets, int cap, const uint32_t* __restrict__ ids,
                                  int64_t n, const uint32_t* __restrict__ bits, uint32_t bound,
                                  uint32_t* __restrict__ data, uint32_t* __restrict__ len) {
  const int key = blockIdx.x * blockDim.x + threadIdx.x;
  if (key >= nbuckets) return;
  uint32_t* d = data + (size_t)key * cap;
  uint32_t l = len[key];
  bool any = false;
  for (uint32_t q = 0; q < l && !any; ++q) {
    const uint32_t v = d[q];
    any = v < bound && ((bits[v >> 5] >> (v & 31)) & 1u);
  }
  if (!any) return;
  for (int64_t i = 0; i < n && l > 0; ++i) {
    const uint32_t id = ids[i];
    for (uint32_t q = 0; q < l; ++q)
      if (d[q] == id) {
        d[q] = d[l - 1];
        --l;
        break;
      }
  }
  len[key] = l;
}

__global__ void id_bits_kernel(const uint32_t* __restrict__ ids, int64_t n, uint32_t bound,
                               uint32_t* __restrict__ bits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n && ids[i] < bound) atomicOr(&bits[ids[i] >> 5], 1u << (ids[i] & 31));
}

// Largest id of the list (ids are below 2^31 for an index, checked by the
// caller from this value).
// One atomic per block: every atomic on the single result word is serialised.
__global__ __launch_bounds__(256) void max_id_kernel(const uint32_t* __restrict__ ids, int64_t n,
                                                     uint32_t* __restrict__ mx) {
  __shared__ uint32_t wm[4];
  uint32_t m = 0u;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    m = max(m, ids[i]);
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
    if (m) atomicMax(mx, m);
  }
}

__global__ void index_clear_kernel(uint32_t* __restrict__ len, uint64_t* __restrict__ count, int nb) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nb) {
    len[i] = 0u;
    count[i] = 0ull;
  }
}

// Threads of a hash_dense_kernel block for `planes` planes (whole waves).
__host__ __device__ constexpr int hash_threads(int planes) {
  return planes >= kHashDenseMax ? kHashDenseMax : (planes <= 64 ? 64 : (planes + 63) / 64 * 64);
}

// Offset in `data` of entry i of the concatenated buckets (bstart: exclusive
// scan of the L bucket lengths, bstart[L] = total; i < total).
__device__ __forceinline__ size_t bucket_entry(const uint32_t* bstart, const uint32_t* bslot,
                                               int L, int cap, uint32_t i) {
  int lo = 0, hi = L;  // bstart[lo] <= i < bstart[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (bstart[mid] <= i) lo = mid;
    else hi = mid;
  }
  return (size_t)bslot[lo] * cap + (i - bstart[lo]);
}

// Bucket of each table (one per thread: L <= kMaxTables <= blockDim) and the
// exclusive scan of the bucket lengths; returns the number of bucket entries.
__device__ __forceinline__ uint32_t query_buckets(const uint32_t* __restrict__ qcodes, int64_t row,
                                                  int L, int k, const uint32_t* __restrict__ len,
                                                  uint32_t* bstart, uint32_t* bslot, int* wsum,
                                                  int* s_total) {
  const uint32_t mask = (1u << k) - 1u;
  const int t = threadIdx.x, tc = min(t, L - 1);
  const uint32_t slot = ((uint32_t)tc << k) | (qcodes[row * L + tc] & mask);
  const uint32_t n = len[slot];  // every thread reads a valid slot (table tc); used for t < L
  const int excl = block_excl_scan(t < L ? (int)n : 0, wsum, s_total);
  if (t < L) {
    bslot[t] = slot;
    bstart[t] = (uint32_t)excl;
  }
  if (t == 0) bstart[L] = (uint32_t)*s_total;
  __syncthreads();
  return bstart[L];
}

// One block per query row: unique bucket ids in ascending order with counts.
// Direct path (ids < kDirectIds): a count per id in LDS, then a scan.
__global__ __launch_bounds__(kQueryThreads) void query_direct_kernel(
    const uint32_t* __restrict__ qcodes, int L, int k, int cap, const uint32_t* __restrict__ data,
    const uint32_t* __restrict__ len, uint32_t id_bound, int stride, uint32_t* __restrict__ out_ids,
    uint32_t* __restrict__ out_cnt, int32_t* __restrict__ out_len) {
  extern __shared__ uint32_t sm[];
  __shared__ int wsum[kQueryThreads / 64];
  __shared__ int s_total;
  __shared__ uint32_t bstart[kMaxTables + 1], bslot[kMaxTables];
  const int64_t row = blockIdx.x;
  uint32_t* oids = out_ids + row * (int64_t)stride;
  uint32_t* ocnt = out_cnt ? out_cnt + row * (int64_t)stride : nullptr;
  for (uint32_t i = threadIdx.x; i < id_bound; i += blockDim.x) sm[i] = 0u;
  const uint32_t m = query_buckets(qcodes, row, L, k, len, bstart, bslot, wsum, &s_total);
  // every bucket entry of every table, kQueryBatch per thread in flight
  for (uint32_t i0 = threadIdx.x; i0 < m; i0 += blockDim.x * kQueryBatch) {
    uint32_t id[kQueryBatch];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q) id[q] = data[bucket_entry(bstart, bslot, L, cap, min(i0 + q * blockDim.x, m - 1))];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q)
      if (i0 + q * blockDim.x < m) atomicAdd(&sm[id[q]], 1u);
  }
  __syncthreads();
  // One scan: thread t owns the ids [t*R, t*R + R) in order, R = ceil(id_bound / threads).
  const uint32_t R = (id_bound + blockDim.x - 1) / blockDim.x;
  const uint32_t i0 = threadIdx.x * R, i1 = min(i0 + R, id_bound);
  int c = 0;
  for (uint32_t i = i0; i < i1; ++i) c += sm[i] != 0u;
  int pos = block_excl_scan(c, wsum, &s_total);
  for (uint32_t i = i0; i < i1; ++i) {
    const uint32_t v = sm[i];
    if (v) {
      oids[pos] = i;
      if (ocnt) ocnt[pos] = v;
      ++pos;
    }
  }
  if (threadIdx.x == 0) out_len[row] = s_total;
}

// Bitmap path (when the LDS below fits in kMaxDynLds): one presence bit per id.  The
// ids come out in ascending order from a scan of popcounts over groups of
// kGroupWords words; an entry's output position (its rank) is its group's
// offset plus the bits below it, so the counts are LDS increments at the rank.
// LDS: bitmap [W] | group offsets [ceil(W / kGroupWords)] | counts [L * cap].
__global__ __launch_bounds__(kQueryBigThreads) void query_bitmap_kernel(
    const uint32_t* __restrict__ qcodes, int L, int k, int cap, const uint32_t* __restrict__ data,
    const uint32_t* __restrict__ len, uint32_t id_bound, int stride, uint32_t* __restrict__ out_ids,
    uint32_t* __restrict__ out_cnt, int32_t* __restrict__ out_len) {
  extern __shared__ uint32_t sm[];
  __shared__ int wsum[kQueryBigThreads / 64];
  __shared__ int s_total;
  __shared__ uint32_t bstart[kMaxTables + 1], bslot[kMaxTables];
  const int64_t row = blockIdx.x;
  uint32_t* oids = out_ids + row * (int64_t)stride;
  uint32_t* ocnt = out_cnt ? out_cnt + row * (int64_t)stride : nullptr;
  const int W = (int)((id_bound + 31u) >> 5);
  const int G = (W + kGroupWords - 1) / kGroupWords;
  uint32_t* bm = sm;
  uint32_t* goff = sm + W;
  uint32_t* cnt = goff + G;
  for (int i = threadIdx.x; i < W; i += blockDim.x) bm[i] = 0u;
  if (ocnt)
    for (int i = threadIdx.x; i < L * cap; i += blockDim.x) cnt[i] = 0u;
  const uint32_t m = query_buckets(qcodes, row, L, k, len, bstart, bslot, wsum, &s_total);
  for (uint32_t i0 = threadIdx.x; i0 < m; i0 += blockDim.x * kQueryBatch) {
    uint32_t id[kQueryBatch];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q) id[q] = data[bucket_entry(bstart, bslot, L, cap, min(i0 + q * blockDim.x, m - 1))];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q)
      if (i0 + q * blockDim.x < m) atomicOr(&bm[id[q] >> 5], 1u << (id[q] & 31u));
  }
  __syncthreads();
  int base = 0;
  for (int g0 = 0; g0 < G; g0 += blockDim.x) {
    const int g = g0 + threadIdx.x;
    const int w0 = g * kGroupWords, w1 = min(w0 + kGroupWords, W);
    int c = 0;
    for (int w = w0; w < w1; ++w) c += __popc(bm[w]);
    int pos = block_excl_scan(c, wsum, &s_total) + base;
    if (g < G) {
      goff[g] = (uint32_t)pos;
      for (int w = w0; w < w1; ++w) {
        uint32_t bits = bm[w];
        while (bits) {
          oids[pos++] = ((uint32_t)w << 5) | (uint32_t)(__ffs(bits) - 1);
          bits &= bits - 1u;
        }
      }
    }
    base += s_total;
  }
  if (threadIdx.x == 0) out_len[row] = base;
  if (!ocnt) return;
  __syncthreads();
  for (uint32_t i0 = threadIdx.x; i0 < m; i0 += blockDim.x * kQueryBatch) {
    uint32_t id[kQueryBatch];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q) id[q] = data[bucket_entry(bstart, bslot, L, cap, min(i0 + q * blockDim.x, m - 1))];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q) {
      if (i0 + q * blockDim.x < m) {
        const int w = (int)(id[q] >> 5);
        const int g = w / kGroupWords;
        uint32_t r = goff[g];
        for (int j = g * kGroupWords; j < w; ++j) r += __popc(bm[j]);
        r += __popc(bm[w] & ((1u << (id[q] & 31u)) - 1u));
        atomicAdd(&cnt[r], 1u);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < base; i += blockDim.x) ocnt[i] = cnt[i];
}

// Sort path (any id): gather, bitonic sort ascending, count runs.
__global__ __launch_bounds__(kQueryBigThreads) void query_sort_kernel(
    const uint32_t* __restrict__ qcodes, int L, int k, int cap, const uint32_t* __restrict__ data,
    const uint32_t* __restrict__ len, int stride, uint32_t* __restrict__ out_ids,
    uint32_t* __restrict__ out_cnt, int32_t* __restrict__ out_len) {
  extern __shared__ uint32_t sm[];
  __shared__ int wsum[kQueryBigThreads / 64];
  __shared__ int s_total;
  __shared__ uint32_t bstart[kMaxTables + 1], bslot[kMaxTables];
  const int64_t row = blockIdx.x;
  uint32_t* oids = out_ids + row * (int64_t)stride;
  uint32_t* ocnt = out_cnt ? out_cnt + row * (int64_t)stride : nullptr;
  const uint32_t m = query_buckets(qcodes, row, L, k, len, bstart, bslot, wsum, &s_total);
  int P = 1;
  while (P < (int)m) P <<= 1;
  for (uint32_t i0 = threadIdx.x; i0 < m; i0 += blockDim.x * kQueryBatch) {
    uint32_t id[kQueryBatch];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q) id[q] = data[bucket_entry(bstart, bslot, L, cap, min(i0 + q * blockDim.x, m - 1))];
#pragma unroll
    for (int q = 0; q < kQueryBatch; ++q)
      if (i0 + q * blockDim.x < m) sm[i0 + q * blockDim.x] = id[q];
  }
  for (int i = (int)m + threadIdx.x; i < P; i += blockDim.x) sm[i] = 0xffffffffu;
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int st = size >> 1; st > 0; st >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        const int j = i ^ st;
        if (j > i) {
          const bool up = (i & size) == 0;
          const uint32_t a = sm[i], c = sm[j];
          if (up ? (a > c) : (a < c)) {
            sm[i] = c;
            sm[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  int base = 0;
  for (int c0 = 0; c0 < (int)m; c0 += blockDim.x) {
    const int i = c0 + threadIdx.x;
    const bool head = i < (int)m && (i == 0 || sm[i] != sm[i - 1]);
    const int pos = block_excl_scan(head ? 1 : 0, wsum, &s_total) + base;
    if (head) {
      int e = i + 1;
      while (e < (int)m && sm[e] == sm[i]) ++e;
      oids[pos] = sm[i];
      if (ocnt) ocnt[pos] = (uint32_t)(e - i);
    }
    base += s_total;
  }
  if (threadIdx.x == 0) out_len[row] = base;
}

__global__ __launch_bounds__(1024) void csr_offsets_kernel(const int32_t* __restrict__ lens,
                                                           int64_t batch, int64_t* __restrict__ off) {
  __shared__ int wsum[16];
  __shared__ int s_total;
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < batch; c0 += blockDim.x) {
    const int64_t i = c0 + threadIdx.x;
    const int v = i < batch ? lens[i] : 0;
    const int p = block_excl_scan(v, wsum, &s_total);
    if (i < batch) off[i] = base + p;
    base += s_total;
  }
  if (threadIdx.x == 0) off[batch] = base;
}

__global__ void csr_copy_u32_kernel(const uint32_t* __restrict__ src, int stride,
                                    const int32_t* __restrict__ lens,
                                    const int64_t* __restrict__ off, int64_t capacity,
                                    uint32_t* __restrict__ dst) {
  const int64_t row = blockIdx.y;
  const int n = lens[row];
  const int64_t o = off[row];
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x)
    if (o + j < capacity) dst[o + j] = src[row * (int64_t)stride + j];
}

__global__ void csr_copy_f32_kernel(const float* __restrict__ src, int stride,
                                    const int32_t* __restrict__ lens,
                                    const int64_t* __restrict__ off, int64_t capacity,
                                    float* __restrict__ dst) {
  const int64_t row = blockIdx.y;
  const int n = lens[row];
  const int64_t o = off[row];
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x)
    if (o + j < capacity) dst[o + j] = src[row * (int64_t)stride + j];
}

// The row offsets and up to three 32-bit arrays' rows in one launch, for
// batches of at most kCsrPackMax rows: block (x, row) sums lens[0..row) itself
// (a block reduction, so no block waits for another), block (0, row) writes
// off[row] (and the last row off[batch]), and every block copies its share of
// the row into each destination given.  The same result as csr_offsets_kernel
// followed by one csr_copy kernel per array.
constexpr int kCsrPackMax = 4096;
__global__ __launch_bounds__(256) void csr_pack_kernel(
    const int32_t* __restrict__ lens, int64_t batch, int stride, int64_t capacity,
    int64_t* __restrict__ off, const uint32_t* __restrict__ s0, uint32_t* __restrict__ d0,
    const uint32_t* __restrict__ s1, uint32_t* __restrict__ d1, const uint32_t* __restrict__ s2,
    uint32_t* __restrict__ d2) {
  __shared__ long long wpart[4];
  const int64_t row = blockIdx.y;
  long long part = 0;
  for (int64_t r = threadIdx.x; r < row; r += blockDim.x) part += lens[r];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m);
  if ((threadIdx.x & 63) == 0) wpart[threadIdx.x >> 6] = part;
  __syncthreads();
  const int64_t o = wpart[0] + wpart[1] + wpart[2] + wpart[3];
  const int n = lens[row];
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    off[row] = o;
    if (row == batch - 1) off[batch] = o + n;
  }
  const int64_t src = row * (int64_t)stride;
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
    if (o + j >= capacity) break;
    if (d0) d0[o + j] = s0[src + j];
    if (d1) d1[o + j] = s1[src + j];
    if (d2) d2[o + j] = s2[src + j];
  }
}

// ------------------------------------------------------------------ host helpers
int hash_dense_launch(const kh_hash_family* h, const float* x, int64_t ldx, int64_t batch,
                      uint32_t* codes, hipStream_t st) {
  if (batch == 0) return KH_OK;
  if (h->kind != KH_FAMILY_TERNARY) return rank_hash_dense_launch(h, x, ldx, batch, codes, st);
  if (h->bt_dev && batch >= kHmMinBatch) {
    for (int64_t b0 = 0; b0 < batch; b0 += (int64_t)65535 * kHmRows) {
      const int64_t nb = std::min<int64_t>(batch - b0, (int64_t)65535 * kHmRows);
      const bool vec = h->dim % 32 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
      hipLaunchKernelGGL(vec ? hash_dense_mfma_kernel<true> : hash_dense_mfma_kernel<false>,
                         dim3((unsigned)ceil_div(nb, kHmRows)), dim3(256), 0, st, h->bt_dev, h->bt_ksteps,
                         h->bt_tiles, h->nnz, h->ent_t, h->k, h->L, h->dim, x + b0 * ldx, ldx, nb,
                         codes + b0 * h->L);
      KH_LAUNCHED();
    }
    return KH_OK;
  }
  if (h->sg_dev) {
    const size_t lds = sizeof(uint4) * h->sg_n4 + sizeof(uint2) * hl_pad(h->dim) + sizeof(uint32_t) * h->sg_tpb;
    if (lds <= (size_t)kMaxDynLds) {
      static std::once_flag once;
      std::call_once(once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hash_dense_lds_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
      });
      for (int64_t b0 = 0; b0 < batch; b0 += INT32_MAX) {
        const int64_t nb = std::min<int64_t>(batch - b0, INT32_MAX);
        hipLaunchKernelGGL(hash_dense_lds_kernel, dim3((unsigned)nb, (unsigned)h->sg_groups), dim3(kHlThreads),
                           lds, st, h->sg_dev, h->sg_n4, h->sg_words, h->k, h->L, h->sg_tpb, h->dim,
                           x + b0 * ldx, ldx, codes + b0 * h->L);
        KH_LAUNCHED();
      }
      return KH_OK;
    }
  }
  const int in_lds = h->dim <= 12288 ? 1 : 0;
  const size_t lds = sizeof(float) * (in_lds ? h->dim : 0) + sizeof(uint32_t) * h->L;
  for (int64_t b0 = 0; b0 < batch; b0 += 65535 * 16) {
    const int64_t nb = std::min<int64_t>(batch - b0, 65535 * 16);
    hipLaunchKernelGGL(hash_dense_kernel, dim3((unsigned)nb), dim3(hash_threads(h->L * h->k)), lds, st,
                       h->nnz, h->ent_t, h->k, h->L, h->dim, x + b0 * ldx, ldx, nb,
                       codes + b0 * h->L, in_lds);
    KH_LAUNCHED();
  }
  return KH_OK;
}

int hash_sparse_launch(const kh_hash_family* h, const int64_t* xoff, const uint32_t* xidx,
                       const float* xval, int64_t batch, uint32_t* codes, hipStream_t st) {
  if (batch == 0) return KH_OK;
  if (h->kind != KH_FAMILY_TERNARY) return rank_hash_sparse_launch(h, xoff, xidx, xval, batch, codes, st);
  KH_CHECK_ARG(h->L <= 256, "hash_sparse supports at most 256 tables");
  const int tpb = kHashThreads / h->k;
  hipLaunchKernelGGL(hash_sparse_kernel, dim3((unsigned)batch, ceil_div(h->L, tpb)), dim3(kHashThreads),
                     0, st, h->planes_dev, h->k, h->L, h->dim, xoff, xidx, xval, codes);
  KH_LAUNCHED();
  return KH_OK;
}

// LDS bytes of query_bitmap_kernel for ids < bound over L * cap entries.
static size_t bitmap_lds(uint32_t bound, int gather) {
  const size_t W = (bound + 31u) / 32u;
  return sizeof(uint32_t) * (W + (W + kGroupWords - 1) / kGroupWords + (size_t)gather);
}

int query_launch(const kh_lsh_index* idx, const uint32_t* qcodes, int64_t batch, uint32_t* qids,
                 uint32_t* qcnt, int stride, int32_t* ulen, hipStream_t st) {
  if (batch == 0) return KH_OK;
  const uint32_t bound = idx->id_bound;
  if (bound <= (uint32_t)kDirectIds) {
    const size_t lds = sizeof(uint32_t) * std::max<uint32_t>(bound, 1);
    hipLaunchKernelGGL(query_direct_kernel, dim3((unsigned)batch), dim3(kQueryThreads), lds, st,
                       qcodes, idx->L, idx->k, idx->cap, idx->data, idx->len, bound, stride, qids,
                       qcnt, ulen);
    KH_LAUNCHED();
    return KH_OK;
  }
  const int gather = idx->L * idx->cap;
  KH_CHECK_ARG(gather <= kMaxGather, "query over ids >= %d needs L*cap <= %d (got %d)", kDirectIds,
               kMaxGather, gather);
  const size_t blds = bitmap_lds(bound, gather);
  if (blds <= (size_t)kMaxDynLds) {
    static bool attr_set = false;
    if (!attr_set) {
      KH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&query_bitmap_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds));
      attr_set = true;
    }
    hipLaunchKernelGGL(query_bitmap_kernel, dim3((unsigned)batch), dim3(kQueryBigThreads), blds, st,
                       qcodes, idx->L, idx->k, idx->cap, idx->data, idx->len, bound, stride, qids,
                       qcnt, ulen);
    KH_LAUNCHED();
    return KH_OK;
  }
  int P = 1;
  while (P < gather) P <<= 1;
  hipLaunchKernelGGL(query_sort_kernel, dim3((unsigned)batch), dim3(kQueryBigThreads),
                     sizeof(uint32_t) * P, st, qcodes, idx->L, idx->k, idx->cap, idx->data,
                     idx->len, stride, qids, qcnt, ulen);
  KH_LAUNCHED();
  return KH_OK;
}

int query_stride(const kh_lsh_index* idx) {
  const int64_t g = (int64_t)idx->L * idx->cap;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, std::max<uint32_t>(idx->id_bound, 1)));
}

int csr_finish(const uint32_t* qids, const uint32_t* qcnt, const float* f1, const float* f2,
               int stride, const int32_t* ulen, int64_t batch, int64_t* off, uint32_t* ids,
               uint32_t* cnts, float* o1, float* o2, int64_t capacity, hipStream_t st) {
  if (batch <= 0) {
    KH_HIP(hipMemsetAsync(off, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  dim3 g(std::max(1, std::min(64, ceil_div(stride, 256))), (unsigned)batch);
  // one launch for the offsets and (up to three) arrays; a fourth array or a
  // longer batch takes the separate kernels
  const int narr = (ids ? 1 : 0) + (cnts && qcnt ? 1 : 0) + (o1 && f1 ? 1 : 0) + (o2 && f2 ? 1 : 0);
  if (batch <= kCsrPackMax && narr <= 3) {
    const uint32_t* src[3] = {nullptr, nullptr, nullptr};
    uint32_t* dst[3] = {nullptr, nullptr, nullptr};
    int a = 0;
    if (ids) { src[a] = qids; dst[a++] = ids; }
    if (cnts && qcnt) { src[a] = qcnt; dst[a++] = cnts; }
    if (o1 && f1) { src[a] = reinterpret_cast<const uint32_t*>(f1); dst[a++] = reinterpret_cast<uint32_t*>(o1); }
    if (o2 && f2) { src[a] = reinterpret_cast<const uint32_t*>(f2); dst[a++] = reinterpret_cast<uint32_t*>(o2); }
    hipLaunchKernelGGL(csr_pack_kernel, g, dim3(256), 0, st, ulen, batch, stride, capacity, off, src[0],
                       dst[0], src[1], dst[1], src[2], dst[2]);
    KH_LAUNCHED();
  } else {
    hipLaunchKernelGGL(csr_offsets_kernel, dim3(1), dim3(1024), 0, st, ulen, batch, off);
    KH_LAUNCHED();
    if (ids) hipLaunchKernelGGL(csr_copy_u32_kernel, g, dim3(256), 0, st, qids, stride, ulen, off, capacity, ids);
    if (cnts && qcnt) hipLaunchKernelGGL(csr_copy_u32_kernel, g, dim3(256), 0, st, qcnt, stride, ulen, off, capacity, cnts);
    if (o1 && f1) hipLaunchKernelGGL(csr_copy_f32_kernel, g, dim3(256), 0, st, f1, stride, ulen, off, capacity, o1);
    if (o2 && f2) hipLaunchKernelGGL(csr_copy_f32_kernel, g, dim3(256), 0, st, f2, stride, ulen, off, capacity, o2);
    KH_LAUNCHED();
  }
  // Every row holds at most `stride` entries: with room for that many, no
  // overflow is possible and the call stays asynchronous (no host round trip;
  // capturable in a graph).  Otherwise the total is read back to report one.
  if (capacity >= batch * (int64_t)stride) return KH_OK;
  int64_t total = 0;
  KH_HIP(hipMemcpyAsync(&total, off + batch, sizeof(int64_t), hipMemcpyDeviceToHost, st));
  KH_HIP(hipStreamSynchronize(st));
  if (total > capacity) {
    set_error("output needs %lld entries, capacity is %lld", (long long)total, (long long)capacity);
    return KH_ERR_CAPACITY;
  }
  return KH_OK;
}

}  // namespace kh

using namespace kh;

// ====================================================================== families
static int family_finish(kh_hash_family* h, kh_hash_family** out) {
  const int P = h->L * h->k;
  std::vector<int32_t> nnz(P, 0);
  for (int p = 0; p < P; ++p) {
    const int8_t* pl = h->planes_host.data() + (size_t)p * h->dim;
    for (int d = 0; d < h->dim; ++d) nnz[p] += pl[d] != 0;
  }
  const int mx = P ? *std::max_element(nnz.begin(), nnz.end()) : 0;
  h->ent_rows = std::max(kHashBatch, (mx + kHashBatch - 1) / kHashBatch * kHashBatch);
  std::vector<uint32_t> ent((size_t)h->ent_rows * P, 0u);
  for (int p = 0; p < P; ++p) {
    const int8_t* pl = h->planes_host.data() + (size_t)p * h->dim;
    size_t j = 0;
    for (int d = 0; d < h->dim; ++d) {
      if (pl[d] == 1) ent[j++ * P + p] = (uint32_t)d << 1;
      else if (pl[d] == -1) ent[j++ * P + p] = ((uint32_t)d << 1) | 1u;
    }
  }
  // BF16 copy of the planes in the matrix-core operand order (hashing large
  // dense batches): entry (step, tile, lane) holds 8 k values of one plane
  std::vector<uint16_t> bt;
  if (P <= kHmMaxPlanes && h->dim <= kHmMaxDim) {
    h->bt_ksteps = (h->dim + 31) / 32;
    h->bt_tiles = (P + 15) / 16;
    bt.assign((size_t)h->bt_ksteps * h->bt_tiles * 64 * 8, 0);
    for (int st = 0; st < h->bt_ksteps; ++st)
      for (int tile = 0; tile < h->bt_tiles; ++tile)
        for (int l = 0; l < 64; ++l) {
          const int p = tile * 16 + (l & 15);
          for (int i = 0; i < 8; ++i) {
            const int d = st * 32 + (l >> 4) * 8 + i;
            const int8_t v = p < P && d < h->dim ? h->planes_host[(size_t)p * h->dim + d] : 0;
            bt[(((size_t)st * h->bt_tiles + tile) * 64 + l) * 8 + i] = v == 1 ? 0x3F80 : (v == -1 ? 0xBF80 : 0);
          }
        }
    h->bt_dev = static_cast<uint4*>(dev_alloc(sizeof(uint16_t) * bt.size()));
    if (!h->bt_dev) {
      kh_hash_family_destroy(h);
      return KH_ERR_ALLOC;
    }
    if (hipMemcpy(h->bt_dev, bt.data(), sizeof(uint16_t) * bt.size(), hipMemcpyHostToDevice) != hipSuccess) {
      set_error("plane upload failed");
      kh_hash_family_destroy(h);
      return KH_ERR_HIP;
    }
  }
  // 2-bit sign copy for the per-row LDS kernel: whole tables per group, as
  // few groups as 256 planes per block allow, tables spread evenly over them.
  if (h->dim <= kHlMaxDim && h->k <= kHlThreads) {
    const int per = kHlThreads / h->k;
    h->sg_groups = (h->L + per - 1) / per;
    h->sg_tpb = (h->L + h->sg_groups - 1) / h->sg_groups;
    h->sg_words = (h->sg_tpb * h->k + 15) / 16;
    h->sg_n4 = (h->dim * h->sg_words + 3) / 4;
    std::vector<uint32_t> sg((size_t)h->sg_groups * h->sg_n4 * 4, 0u);
    for (int g = 0; g < h->sg_groups; ++g)
      for (int q = 0; q < h->sg_tpb * h->k; ++q) {
        const int p = g * h->sg_tpb * h->k + q;
        if (p >= P) break;
        const int8_t* pl = h->planes_host.data() + (size_t)p * h->dim;
        for (int d = 0; d < h->dim; ++d) {
          const uint32_t code = pl[d] == 1 ? 1u : (pl[d] == -1 ? 3u : 0u);
          sg[(size_t)g * h->sg_n4 * 4 + (size_t)d * h->sg_words + q / 16] |= code << (2 * (q % 16));
        }
      }
    h->sg_dev = static_cast<uint4*>(dev_alloc(sizeof(uint32_t) * sg.size()));
    if (!h->sg_dev) {
      kh_hash_family_destroy(h);
      return KH_ERR_ALLOC;
    }
    if (hipMemcpy(h->sg_dev, sg.data(), sizeof(uint32_t) * sg.size(), hipMemcpyHostToDevice) != hipSuccess) {
      set_error("plane upload failed");
      kh_hash_family_destroy(h);
      return KH_ERR_HIP;
    }
  }
  h->planes_dev = static_cast<int8_t*>(dev_alloc(h->planes_host.size()));
  h->nnz = static_cast<int32_t*>(dev_alloc(sizeof(int32_t) * std::max(P, 1)));
  h->ent_t = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * ent.size()));
  if (!h->planes_dev || !h->nnz || !h->ent_t) {
    kh_hash_family_destroy(h);
    return KH_ERR_ALLOC;
  }
  if (hipMemcpy(h->planes_dev, h->planes_host.data(), h->planes_host.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(h->nnz, nnz.data(), sizeof(int32_t) * P, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(h->ent_t, ent.data(), sizeof(uint32_t) * ent.size(), hipMemcpyHostToDevice) != hipSuccess) {
    set_error("plane upload failed");
    kh_hash_family_destroy(h);
    return KH_ERR_HIP;
  }
  *out = h;
  return KH_OK;
}

static int family_check(int input_dim, int k, int num_tables, kh_hash_family** out) {
  KH_CHECK_ARG(out != nullptr, "null out");
  KH_CHECK_ARG(input_dim > 0 && num_tables > 0 && num_tables <= 256,
               "input_dim must be positive and num_tables in [1,256]");
  KH_CHECK_ARG(k >= 1 && k <= 24, "k (%d) must be in [1,24] (2^k buckets per table)", k);
  return KH_OK;
}

extern "C" int kh_simhash_create(int input_dim, int k, int num_tables, uint64_t seed,
                                 kh_hash_family** out) {
  int rc = family_check(input_dim, k, num_tables, out);
  if (rc != KH_OK) return rc;
  auto* h = new kh_hash_family();
  h->dim = input_dim;
  h->k = k;
  h->L = num_tables;
  h->planes_host.resize((size_t)num_tables * k * input_dim);
  simhash_planes(input_dim, k, num_tables, seed, h->planes_host.data());
  return family_finish(h, out);
}

extern "C" int kh_srp_create(int input_dim, int k, int num_tables, float sparsity, uint64_t seed,
                             kh_hash_family** out) {
  int rc = family_check(input_dim, k, num_tables, out);
  if (rc != KH_OK) return rc;
  KH_CHECK_ARG(sparsity >= 0.0f && sparsity <= 1.0f, "sparsity must be in [0, 1]");
  auto* h = new kh_hash_family();
  h->dim = input_dim;
  h->k = k;
  h->L = num_tables;
  h->planes_host.resize((size_t)num_tables * k * input_dim);
  srp_planes(input_dim, k, num_tables, sparsity, seed, h->planes_host.data());
  return family_finish(h, out);
}

extern "C" int kh_hash_family_from_planes(int input_dim, int k, int num_tables,
                                          const int8_t* planes_host, kh_hash_family** out) {
  int rc = family_check(input_dim, k, num_tables, out);
  if (rc != KH_OK) return rc;
  KH_CHECK_ARG(planes_host != nullptr, "null planes");
  const size_t n = (size_t)num_tables * k * input_dim;
  for (size_t i = 0; i < n; ++i)
    KH_CHECK_ARG(planes_host[i] >= -1 && planes_host[i] <= 1, "plane entry %zu not in {-1,0,1}", i);
  auto* h = new kh_hash_family();
  h->dim = input_dim;
  h->k = k;
  h->L = num_tables;
  h->planes_host.assign(planes_host, planes_host + n);
  return family_finish(h, out);
}

extern "C" int kh_hash_family_destroy(kh_hash_family* h) {
  if (!h) return KH_OK;
  dev_free(h->planes_dev);
  dev_free(h->nnz);
  dev_free(h->ent_t);
  dev_free(h->bt_dev);
  dev_free(h->sg_dev);
  dev_free(h->windows_dev);
  dev_free(h->fallback_dev);
  dev_free(h->perms_dev);
  delete h;
  return KH_OK;
}

extern "C" int kh_hash_family_dims(const kh_hash_family* h, int* k, int* input_dim,
                                   int* num_tables) {
  KH_CHECK_ARG(h != nullptr, "null family");
  if (k) *k = h->k;
  if (input_dim) *input_dim = h->dim;
  if (num_tables) *num_tables = h->L;
  return KH_OK;
}

extern "C" int kh_hash_family_planes(const kh_hash_family* h, int8_t* planes_host) {
  KH_CHECK_ARG(h && planes_host, "null argument");
  if (h->kind != KH_FAMILY_TERNARY) {
    set_error("the family has no hyperplanes (WTA, DWTA or MinHash)");
    return KH_ERR_UNSUPPORTED;
  }
  memcpy(planes_host, h->planes_host.data(), h->planes_host.size());
  return KH_OK;
}

extern "C" int kh_hash_dense(const kh_hash_family* h, const float* x_dev, int64_t batch,
                             uint32_t* codes_dev, void* stream) {
  KH_CHECK_ARG(h && codes_dev && (x_dev || batch == 0), "null argument");
  KH_CHECK_ARG(batch >= 0, "bad batch");
  return hash_dense_launch(h, x_dev, h->dim, batch, codes_dev, as_stream(stream));
}

extern "C" int kh_hash_sparse(const kh_hash_family* h, const int64_t* off_dev,
                              const uint32_t* idx_dev, const float* val_dev, int64_t batch,
                              uint32_t* codes_dev, void* stream) {
  KH_CHECK_ARG(h && off_dev && codes_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff, "bad batch");
  return hash_sparse_launch(h, off_dev, idx_dev, val_dev, batch, codes_dev, as_stream(stream));
}

// ====================================================================== index
extern "C" int kh_lsh_index_create(const kh_hash_family* h, int bucket_type, int capacity,
                                   kh_lsh_index** out) {
  KH_CHECK_ARG(h && out, "null argument");
  KH_CHECK_ARG(capacity > 0, "bucket capacity must be positive");
  KH_CHECK_ARG(bucket_type == KH_BUCKET_FIFO || bucket_type == KH_BUCKET_RESERVOIR,
               "bad bucket type %d", bucket_type);
  *out = nullptr;
  auto* idx = new kh_lsh_index();
  idx->h = h;
  idx->type = bucket_type;
  idx->cap = capacity;
  idx->L = h->L;
  idx->k = h->k;
  idx->nb = 1 << h->k;
  const size_t nbk = (size_t)idx->L * idx->nb;
  idx->data = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * nbk * capacity));
  idx->len = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * nbk));
  idx->count = static_cast<uint64_t*>(dev_alloc(sizeof(uint64_t) * nbk));
  if (!idx->data || !idx->len || !idx->count) {
    kh_lsh_index_destroy(idx);
    return KH_ERR_ALLOC;
  }
  if (hipMemset(idx->len, 0, sizeof(uint32_t) * nbk) != hipSuccess ||
      hipMemset(idx->count, 0, sizeof(uint64_t) * nbk) != hipSuccess ||
      hipMemset(idx->data, 0, sizeof(uint32_t) * nbk * capacity) != hipSuccess) {
    set_error("index init failed");
    kh_lsh_index_destroy(idx);
    return KH_ERR_HIP;
  }
  *out = idx;
  return KH_OK;
}

extern "C" int kh_lsh_index_destroy(kh_lsh_index* idx) {
  if (!idx) return KH_OK;
  dev_free(idx->data);
  dev_free(idx->len);
  dev_free(idx->count);
  delete idx;
  return KH_OK;
}

extern "C" int kh_lsh_index_clear(kh_lsh_index* idx, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  const int nbk = idx->L * idx->nb;
  hipLaunchKernelGGL(index_clear_kernel, dim3(ceil_div(nbk, 256)), dim3(256), 0,
                     as_stream(stream), idx->len, idx->count, nbk);
  KH_LAUNCHED();
  idx->id_bound = 0;
  return KH_OK;
}

namespace {

// Device scratch of one mutation call (mutations are `&mut self` calls and
// synchronise before they return).  The buffers come from the index's arena,
// a stack of grow-only slots: a call takes the next slots and gives them back
// on return, so repeated inserts and rebuilds allocate nothing once the
// largest call has run.
struct CallBufs {
  kh::ScratchArena& a;
  size_t mark;
  explicit CallBufs(kh::ScratchArena& arena) : a(arena), mark(arena.cursor) {}
  ~CallBufs() { a.cursor = mark; }
  template <typename T>
  T* get(size_t n) {
    const size_t bytes = sizeof(T) * (n ? n : 1);
    if (a.cursor == a.slots.size()) a.slots.push_back({nullptr, 0});
    auto& sl = a.slots[a.cursor];
    if (sl.second < bytes) {
      dev_free(sl.first);
      sl.first = dev_alloc(bytes);
      sl.second = sl.first ? bytes : 0;
    }
    if (!sl.first) return nullptr;
    ++a.cursor;
    return static_cast<T*>(sl.first);
  }
};

// Largest id of ids_dev[0..n) (synchronises): ids of an index are below
// 2^31, so that id + 1 bounds and bitmap word counts cannot wrap.
int checked_max_id(const uint32_t* ids_dev, int64_t n, hipStream_t st, CallBufs& cb,
                   uint32_t* out) {
  uint32_t* mx = cb.get<uint32_t>(1);
  if (!mx) return KH_ERR_ALLOC;
  KH_HIP(hipMemsetAsync(mx, 0, sizeof(uint32_t), st));
  hipLaunchKernelGGL(max_id_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 256)), dim3(256), 0, st,
                     ids_dev, n, mx);
  KH_LAUNCHED();
  uint32_t v = 0;
  KH_HIP(hipMemcpyAsync(&v, mx, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  KH_HIP(hipStreamSynchronize(st));
  KH_CHECK_ARG(v < 0x80000000u, "neuron id %u out of range (ids must be below 2^31)", v);
  *out = v;
  return KH_OK;
}

// The (table, bucket) of every (vector, table) pair, grouped by bucket with
// the vectors' order kept inside each group (stable radix sort): spos lists
// vector positions, start/end delimit each bucket's run.
struct Groups {
  uint32_t *spos = nullptr, *start = nullptr, *end = nullptr, *skeys = nullptr;
};
int group_by_bucket(const kh_lsh_index* idx, const uint32_t* codes_dev, int64_t n, hipStream_t st,
                    CallBufs& cb, Groups* g) {
  KH_CHECK_ARG(n * idx->L < (int64_t)0x7fffffff, "too many vectors in one call");
  const int64_t m = n * idx->L;
  const int nbk = idx->L * idx->nb;
  unsigned end_bit = 1;
  while ((1ull << end_bit) < (unsigned long long)nbk) ++end_bit;
  uint32_t* keys = cb.get<uint32_t>(m);
  uint32_t* pos = cb.get<uint32_t>(m);
  uint32_t* skeys = cb.get<uint32_t>(m);
  g->skeys = skeys;
  g->spos = cb.get<uint32_t>(m);
  g->start = cb.get<uint32_t>(nbk);
  g->end = cb.get<uint32_t>(nbk);
  if (!keys || !pos || !skeys || !g->spos || !g->start || !g->end) return KH_ERR_ALLOC;
  size_t tmp_bytes = 0;
  if (rocprim::radix_sort_pairs(nullptr, tmp_bytes, keys, skeys, pos, g->spos, (unsigned)m, 0u,
                                end_bit, st) != hipSuccess) {
    set_error("radix sort sizing failed");
    return KH_ERR_HIP;
  }
  void* tmp = cb.get<uint8_t>(tmp_bytes);
  if (!tmp) return KH_ERR_ALLOC;
  hipLaunchKernelGGL(build_keys_kernel, dim3(ceil_div(m, 256)), dim3(256), 0, st, codes_dev, n,
                     idx->L, idx->k, keys, pos);
  KH_LAUNCHED();
  if (rocprim::radix_sort_pairs(tmp, tmp_bytes, keys, skeys, pos, g->spos, (unsigned)m, 0u,
                                end_bit, st) != hipSuccess) {
    set_error("radix sort failed");
    return KH_ERR_HIP;
  }
  KH_HIP(hipMemsetAsync(g->start, 0, sizeof(uint32_t) * nbk, st));
  KH_HIP(hipMemsetAsync(g->end, 0, sizeof(uint32_t) * nbk, st));
  hipLaunchKernelGGL(seg_bounds_kernel, dim3(ceil_div(m, 256)), dim3(256), 0, st, skeys, m,
                     g->start, g->end);
  KH_LAUNCHED();
  return KH_OK;
}

}  // namespace

extern "C" int kh_lsh_index_insert_codes(kh_lsh_index* idx, const uint32_t* ids_dev,
                                         const uint32_t* codes_dev, int64_t n, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0, "bad n");
  if (n == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev && codes_dev, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  uint32_t mx = 0;
  int rc = checked_max_id(ids_dev, n, st, cb, &mx);  // before anything is inserted
  if (rc != KH_OK) return rc;
  Groups g;
  rc = group_by_bucket(idx, codes_dev, n, st, cb, &g);
  if (rc != KH_OK) return rc;
  const int nbk = idx->L * idx->nb;
  if (idx->type == KH_BUCKET_RESERVOIR) {
    const int64_t m = n * idx->L, nslots = (int64_t)nbk * idx->cap;
    uint32_t* last = cb.get<uint32_t>(nslots);
    if (!last) return KH_ERR_ALLOC;
    KH_HIP(hipMemsetAsync(last, 0, sizeof(uint32_t) * nslots, st));
    hipLaunchKernelGGL(reservoir_targets_kernel, dim3((unsigned)ceil_div(m, 256)), dim3(256), 0, st, m,
                       idx->cap, g.skeys, g.start, g.spos, ids_dev, idx->len, idx->count, last);
    KH_LAUNCHED();
    hipLaunchKernelGGL(reservoir_apply_kernel, dim3((unsigned)ceil_div(nslots, 256)), dim3(256), 0, st,
                       nslots, idx->cap, g.start, g.end, g.spos, ids_dev, last, idx->data, idx->len,
                       idx->count);
    KH_LAUNCHED();
  } else {
    hipLaunchKernelGGL(fifo_apply_kernel, dim3(ceil_div(nbk, 64)), dim3(64), 0, st, nbk, idx->cap,
                       g.start, g.end, g.spos, ids_dev, idx->data, idx->len);
    KH_LAUNCHED();
  }
  KH_HIP(hipStreamSynchronize(st));  // the call's scratch is freed on return
  idx->id_bound = std::max(idx->id_bound, mx + 1u);
  return KH_OK;
}

extern "C" int kh_lsh_index_insert(kh_lsh_index* idx, const uint32_t* ids_dev, const float* w_dev,
                                   int64_t n, int64_t ldw, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0 && ldw >= idx->h->dim, "bad n/ldw");
  if (n == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev && w_dev, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  uint32_t* codes = cb.get<uint32_t>(n * idx->L);
  if (!codes) return KH_ERR_ALLOC;
  int rc = hash_dense_launch(idx->h, w_dev, ldw, n, codes, st);
  if (rc == KH_OK) rc = kh_lsh_index_insert_codes(idx, ids_dev, codes, n, stream);
  return rc;
}

extern "C" int kh_lsh_index_insert_sparse(kh_lsh_index* idx, const uint32_t* ids_dev,
                                          const int64_t* xoff_dev, const uint32_t* xidx_dev,
                                          const float* xval_dev, int64_t n, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0 && n <= 0x7fffffff, "bad n");
  if (n == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev && xoff_dev, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  uint32_t* codes = cb.get<uint32_t>(n * idx->L);
  if (!codes) return KH_ERR_ALLOC;
  int rc = hash_sparse_launch(idx->h, xoff_dev, xidx_dev, xval_dev, n, codes, st);
  if (rc == KH_OK) rc = kh_lsh_index_insert_codes(idx, ids_dev, codes, n, stream);
  return rc;
}

extern "C" int kh_lsh_index_remove_codes(kh_lsh_index* idx, const uint32_t* ids_dev,
                                         const uint32_t* codes_dev, int64_t n, void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0, "bad n");
  if (n == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev && codes_dev, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  Groups g;
  int rc = group_by_bucket(idx, codes_dev, n, st, cb, &g);
  if (rc != KH_OK) return rc;
  const int nbk = idx->L * idx->nb;
  hipLaunchKernelGGL(remove_buckets_kernel, dim3(ceil_div(nbk, 64)), dim3(64), 0, st, nbk,
                     idx->cap, g.start, g.end, g.spos, ids_dev, idx->data, idx->len);
  KH_LAUNCHED();
  KH_HIP(hipStreamSynchronize(st));
  return KH_OK;
}

extern "C" int kh_lsh_index_remove_with_weights(kh_lsh_index* idx, const uint32_t* ids_dev,
                                                const float* w_dev, int64_t n, int64_t ldw,
                                                void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0 && ldw >= idx->h->dim, "bad n/ldw");
  if (n == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev && w_dev, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  uint32_t* codes = cb.get<uint32_t>(n * idx->L);
  if (!codes) return KH_ERR_ALLOC;
  int rc = hash_dense_launch(idx->h, w_dev, ldw, n, codes, st);
  if (rc == KH_OK) rc = kh_lsh_index_remove_codes(idx, ids_dev, codes, n, stream);
  return rc;
}

extern "C" int kh_lsh_index_remove(kh_lsh_index* idx, const uint32_t* ids_dev, int64_t n,
                                   void* stream) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  KH_CHECK_ARG(n >= 0, "bad n");
  if (n == 0 || idx->id_bound == 0) return KH_OK;
  KH_CHECK_ARG(ids_dev != nullptr, "null argument");
  hipStream_t st = as_stream(stream);
  CallBufs cb(idx->arena);
  const uint32_t words = (idx->id_bound + 31u) >> 5;  // id_bound <= 2^31
  uint32_t* bits = cb.get<uint32_t>(words);
  if (!bits) return KH_ERR_ALLOC;
  KH_HIP(hipMemsetAsync(bits, 0, sizeof(uint32_t) * words, st));
  hipLaunchKernelGGL(id_bits_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, st, ids_dev, n,
                     idx->id_bound, bits);
  KH_LAUNCHED();
  const int nbk = idx->L * idx->nb;
  hipLaunchKernelGGL(remove_all_kernel, dim3(ceil_div(nbk, 64)), dim3(64), 0, st, nbk, idx->cap,
                     ids_dev, n, bits, idx->id_bound, idx->data, idx->len);
  KH_LAUNCHED();
  KH_HIP(hipStreamSynchronize(st));
  return KH_OK;
}

enum { kQwCodes, kQwIds, kQwCnt, kQwLen };

static int query_common(const kh_lsh_index* idx, const uint32_t* qcodes, int64_t batch,
                        int64_t* off, uint32_t* ids, uint32_t* counts, int64_t capacity,
                        hipStream_t st) {
  WsSet* w = idx->ws.get(st);
  const int stride = query_stride(idx);
  uint32_t* qids = static_cast<uint32_t*>(w->get(kQwIds, sizeof(uint32_t) * batch * stride));
  uint32_t* qcnt = static_cast<uint32_t*>(w->get(kQwCnt, sizeof(uint32_t) * batch * stride));
  int32_t* ulen = static_cast<int32_t*>(w->get(kQwLen, sizeof(int32_t) * batch));
  if (!qids || !qcnt || !ulen) return KH_ERR_ALLOC;
  int rc = query_launch(idx, qcodes, batch, qids, counts ? qcnt : nullptr, stride, ulen, st);
  if (rc != KH_OK) return rc;
  return csr_finish(qids, qcnt, nullptr, nullptr, stride, ulen, batch, off, ids, counts, nullptr,
                    nullptr, capacity, st);
}

extern "C" int kh_lsh_index_query(const kh_lsh_index* idx, const float* x_dev, int64_t batch,
                                  int64_t* off_dev, uint32_t* ids_dev, uint32_t* counts_dev,
                                  int64_t capacity, void* stream) {
  KH_CHECK_ARG(idx && off_dev && ids_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && capacity >= 0, "bad batch/capacity");
  hipStream_t st = as_stream(stream);
  if (batch == 0) {
    KH_HIP(hipMemsetAsync(off_dev, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  KH_CHECK_ARG(x_dev != nullptr, "null input");
  uint32_t* qcodes = static_cast<uint32_t*>(idx->ws.get(st)->get(kQwCodes, sizeof(uint32_t) * batch * idx->L));
  if (!qcodes) return KH_ERR_ALLOC;
  int rc = hash_dense_launch(idx->h, x_dev, idx->h->dim, batch, qcodes, st);
  if (rc != KH_OK) return rc;
  return query_common(idx, qcodes, batch, off_dev, ids_dev, counts_dev, capacity, st);
}

extern "C" int kh_lsh_index_query_sparse(const kh_lsh_index* idx, const int64_t* xoff_dev,
                                         const uint32_t* xidx_dev, const float* xval_dev,
                                         int64_t batch, int64_t* off_dev, uint32_t* ids_dev,
                                         uint32_t* counts_dev, int64_t capacity, void* stream) {
  KH_CHECK_ARG(idx && off_dev && ids_dev && xoff_dev, "null argument");
  KH_CHECK_ARG(batch >= 0 && batch <= 0x7fffffff && capacity >= 0, "bad batch/capacity");
  hipStream_t st = as_stream(stream);
  if (batch == 0) {
    KH_HIP(hipMemsetAsync(off_dev, 0, sizeof(int64_t), st));
    return KH_OK;
  }
  uint32_t* qcodes = static_cast<uint32_t*>(idx->ws.get(st)->get(kQwCodes, sizeof(uint32_t) * batch * idx->L));
  if (!qcodes) return KH_ERR_ALLOC;
  int rc = hash_sparse_launch(idx->h, xoff_dev, xidx_dev, xval_dev, batch, qcodes, st);
  if (rc != KH_OK) return rc;
  return query_common(idx, qcodes, batch, off_dev, ids_dev, counts_dev, capacity, st);
}

extern "C" int kh_lsh_index_buckets(const kh_lsh_index* idx, uint32_t* data_host,
                                    uint32_t* len_host, uint64_t* count_host) {
  KH_CHECK_ARG(idx != nullptr, "null index");
  const size_t nbk = (size_t)idx->L * idx->nb;
  KH_HIP(hipDeviceSynchronize());
  if (data_host)
    KH_HIP(hipMemcpy(data_host, idx->data, sizeof(uint32_t) * nbk * idx->cap, hipMemcpyDeviceToHost));
  if (len_host) KH_HIP(hipMemcpy(len_host, idx->len, sizeof(uint32_t) * nbk, hipMemcpyDeviceToHost));
  if (count_host)
    KH_HIP(hipMemcpy(count_host, idx->count, sizeof(uint64_t) * nbk, hipMemcpyDeviceToHost));
  return KH_OK;
}
