// hash_rank.hip -- the rank-based LSH families on the GPU (gfx950):
// WtaHash (crates/klearu-core/src/hash/wta.rs), DwtaHash (hash/dwta.rs) and
// MinHash / densified one-permutation hashing (hash/minhash.rs).
//
// WTA and DWTA: one thread per (row, table).  WTA packs the k window argmax positions
// (first strict maximum from -inf) from bit 0 up, bits_per_window each;
// DWTA's sparse form takes the argmax over the window dimensions that are
// stored in the row and, for a window with none, a position fixed per
// (table, window) by std's DefaultHasher (precomputed on the host); MinHash
// takes per-bin minima of the permuted nonzero dimensions, fills empty bins
// from the next non-empty bin (circularly) and combines them as
// sum(h_i * P^i) in wrapping u64 arithmetic (one block per row).  Codes are returned as their
// low 32 bits (an index keeps the low k <= 24 bits).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "lsh_internal.hpp"
#include "rng.hpp"

namespace kh {

constexpr int kRankThreads = 128;
constexpr int kMaxMinHashBins = 24;  // k of an index (2^k buckets)
constexpr uint64_t kMinHashPrime = 0x517cc1b727220a95ull;  // minhash.rs:117

// Value of dimension d in a CSR row as SparseVector::to_dense gives it (the
// last stored entry at d wins; absent = 0).
__device__ __forceinline__ float csr_value(const uint32_t* idx, const float* val, int64_t a,
                                           int64_t b, uint32_t d) {
  float v = 0.0f;
  for (int64_t e = a; e < b; ++e)
    if (idx[e] == d) v = val[e];
  return v;
}

// Position of dimension d among the row's sorted indices, or -1 (the
// reference's binary_search on SparseVector::indices).
__device__ __forceinline__ int64_t csr_find(const uint32_t* idx, int64_t a, int64_t b, uint32_t d) {
  int64_t lo = a, hi = b;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (idx[mid] < d) lo = mid + 1;
    else hi = mid;
  }
  return (lo < b && idx[lo] == d) ? lo : -1;
}

// WTA / DWTA over dense rows, or WTA over CSR rows (to_dense values).
template <bool SPARSE>
__global__ __launch_bounds__(kRankThreads) void wta_hash_kernel(
    const uint32_t* __restrict__ windows, int k, int L, int ws, int bits,
    const float* __restrict__ x, int64_t ldx, const int64_t* __restrict__ xoff,
    const uint32_t* __restrict__ xidx, const float* __restrict__ xval, int64_t batch,
    uint32_t* __restrict__ codes) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= batch * L) return;
  const int64_t row = q / L;
  const int t = static_cast<int>(q % L);
  uint64_t h = 0;
  for (int f = 0; f < k; ++f) {
    const uint32_t* win = windows + (static_cast<size_t>(t) * k + f) * ws;
    int best = 0;
    float bv = -INFINITY;
    for (int p = 0; p < ws; ++p) {
      const float v = SPARSE ? csr_value(xidx, xval, xoff[row], xoff[row + 1], win[p])
                             : x[row * ldx + win[p]];
      if (v > bv) {
        bv = v;
        best = p;
      }
    }
    h |= static_cast<uint64_t>(best) << (bits * f);
  }
  codes[q] = static_cast<uint32_t>(h);
}

// DWTA over CSR rows (dwta.rs:108-166).
__global__ __launch_bounds__(kRankThreads) void dwta_sparse_kernel(
    const uint32_t* __restrict__ windows, const uint32_t* __restrict__ fallback, int k, int L,
    int ws, int bits, const int64_t* __restrict__ xoff, const uint32_t* __restrict__ xidx,
    const float* __restrict__ xval, int64_t batch, uint32_t* __restrict__ codes) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= batch * L) return;
  const int64_t row = q / L;
  const int t = static_cast<int>(q % L);
  const int64_t a = xoff[row], b = xoff[row + 1];
  uint64_t h = 0;
  for (int f = 0; f < k; ++f) {
    const uint32_t* win = windows + (static_cast<size_t>(t) * k + f) * ws;
    int best = -1;
    float bv = -INFINITY;
    for (int p = 0; p < ws; ++p) {
      const int64_t e = csr_find(xidx, a, b, win[p]);
      if (e >= 0 && xval[e] > bv) {
        bv = xval[e];
        best = p;
      }
    }
    const uint64_t pos = best >= 0 ? static_cast<uint64_t>(best) : fallback[t * k + f];
    h |= pos << (bits * f);
  }
  codes[q] = static_cast<uint32_t>(h);
}

// MinHash over dense rows (nonzero = x != 0) or CSR rows (every stored index
// below dim, minhash.rs:151-153).  One block per row: a dense row's nonzero
// dimensions are first collected in LDS (a bin minimum does not depend on the
// order they are taken in); then each wave takes one table at a time, its
// lanes striding over the nonzeros with an LDS atomicMin per (bin, value),
// and lane 0 densifies and combines the table's k bins.
constexpr int kMhThreads = 256;
constexpr int kMhWaves = kMhThreads / 64;
constexpr int kMhMaxStage = 16384;  // dense rows up to this dim stage their nonzeros in LDS
constexpr int64_t kMhMaxRows = 1 << 22;  // rows (blocks) per launch

template <bool SPARSE>
__global__ __launch_bounds__(kMhThreads) void minhash_rows_kernel(
    const uint32_t* __restrict__ perms, int dim, int k, int L, const float* __restrict__ x,
    int64_t ldx, const int64_t* __restrict__ xoff, const uint32_t* __restrict__ xidx,
    uint32_t* __restrict__ codes) {
  extern __shared__ uint32_t nzd[];  // dense: the row's nonzero dimensions (any order)
  __shared__ uint32_t wmin[kMhWaves][kMaxMinHashBins];
  __shared__ int nnz_s;
  const int64_t row = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t* list;
  int64_t nnz;
  if constexpr (SPARSE) {
    const int64_t a = xoff[row];
    list = xidx + a;
    nnz = xoff[row + 1] - a;
  } else {
    if (threadIdx.x == 0) nnz_s = 0;
    __syncthreads();
    const float* __restrict__ xr = x + row * ldx;
    for (int d0 = 0; d0 < dim; d0 += kMhThreads) {  // one LDS atomic per wave and step
      const int d = d0 + static_cast<int>(threadIdx.x);
      const float v = xr[min(d, dim - 1)];
      const bool nz = d < dim && v != 0.0f;
      const uint64_t bal = __ballot(nz);
      int base = 0;
      if (lane == 0 && bal) base = atomicAdd(&nnz_s, static_cast<int>(__popcll(bal)));
      base = __shfl(base, 0);
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0));
      if (nz) nzd[base + below] = static_cast<uint32_t>(d);
    }
    __syncthreads();
    list = nzd;
    nnz = nnz_s;
  }
  const uint32_t bin_size = static_cast<uint32_t>((dim + k - 1) / k);
  for (int t0 = 0; t0 < L; t0 += kMhWaves) {
    const int t = t0 + wave;
    if (lane < kMaxMinHashBins) wmin[wave][lane] = 0xffffffffu;
    __syncthreads();
    if (t < L) {
      const uint32_t* __restrict__ perm = perms + static_cast<size_t>(t) * dim;
      for (int64_t e = lane; e < nnz; e += 64) {
        const uint32_t d = list[e];
        if (SPARSE && d >= static_cast<uint32_t>(dim)) continue;
        const uint32_t pv = perm[d];
        atomicMin(&wmin[wave][pv / bin_size], pv);
      }
    }
    __syncthreads();
    if (t < L && lane == 0) {
      // densify (minhash.rs:76-104): an empty bin takes the next non-empty
      // bin circularly, so one backward pass seeded with the first non-empty
      // bin fills them all; with every bin empty all become 0
      uint32_t first = 0xffffffffu;
      for (int i = k - 1; i >= 0; --i)
        if (wmin[wave][i] != 0xffffffffu) first = wmin[wave][i];
      uint32_t cur = first == 0xffffffffu ? 0u : first;
      uint32_t m[kMaxMinHashBins];
      for (int i = k - 1; i >= 0; --i) {
        if (wmin[wave][i] != 0xffffffffu) cur = wmin[wave][i];
        m[i] = cur;
      }
      uint64_t h = 0, pp = 1;
      for (int i = 0; i < k; ++i) {
        h += static_cast<uint64_t>(m[i]) * pp;
        pp *= kMinHashPrime;
      }
      codes[row * L + t] = static_cast<uint32_t>(h & ((1ull << k) - 1ull));
    }
  }
}

// MinHash over dense rows too wide to stage: one thread per (row, table),
// walking the row in index order.
__global__ __launch_bounds__(kRankThreads) void minhash_kernel(
    const uint32_t* __restrict__ perms, int dim, int k, int L, const float* __restrict__ x,
    int64_t ldx, int64_t batch, uint32_t* __restrict__ codes) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= batch * L) return;
  const int64_t row = q / L;
  const int t = static_cast<int>(q % L);
  const uint32_t* perm = perms + static_cast<size_t>(t) * dim;
  const uint32_t bin_size = static_cast<uint32_t>((dim + k - 1) / k);
  uint32_t mins[kMaxMinHashBins];
#pragma unroll
  for (int i = 0; i < kMaxMinHashBins; ++i) mins[i] = 0xffffffffu;
  const float* xr = x + row * ldx;
  for (int d = 0; d < dim; ++d) {
    if (xr[d] == 0.0f) continue;
    const uint32_t pv = perm[d];
    const uint32_t bin = pv / bin_size;
#pragma unroll
    for (int i = 0; i < kMaxMinHashBins; ++i)
      if (i == static_cast<int>(bin) && pv < mins[i]) mins[i] = pv;
  }
  // densify and combine as minhash_rows_kernel does; every index below is a
  // compile-time constant, so mins stays in registers
  uint32_t first = 0xffffffffu;
#pragma unroll
  for (int i = kMaxMinHashBins - 1; i >= 0; --i)
    if (i < k && mins[i] != 0xffffffffu) first = mins[i];
  uint32_t cur = first == 0xffffffffu ? 0u : first;
#pragma unroll
  for (int i = kMaxMinHashBins - 1; i >= 0; --i) {
    if (i < k) {
      if (mins[i] != 0xffffffffu) cur = mins[i];
      mins[i] = cur;
    }
  }
  uint64_t h = 0, pp = 1;
#pragma unroll
  for (int i = 0; i < kMaxMinHashBins; ++i) {
    if (i < k) {
      h += static_cast<uint64_t>(mins[i]) * pp;
      pp *= kMinHashPrime;
    }
  }
  codes[q] = static_cast<uint32_t>(h & ((1ull << k) - 1ull));
}

int rank_hash_dense_launch(const kh_hash_family* h, const float* x, int64_t ldx, int64_t batch,
                           uint32_t* codes, hipStream_t st) {
  if (batch == 0) return KH_OK;
  const int64_t n = batch * h->L;
  const unsigned blocks = static_cast<unsigned>((n + kRankThreads - 1) / kRankThreads);
  if (h->kind == KH_FAMILY_MINHASH && h->dim <= kMhMaxStage) {
    // the staged nonzeros take up to 64 KiB of dynamic LDS next to the static
    // bins, past the default dynamic limit: raise it once per process
    static std::once_flag once;
    static hipError_t attr_rc = hipSuccess;
    std::call_once(once, [] {
      attr_rc = hipFuncSetAttribute(reinterpret_cast<const void*>(&minhash_rows_kernel<false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
      if (attr_rc == hipSuccess)
        attr_rc = hipFuncSetAttribute(reinterpret_cast<const void*>(&minhash_rows_kernel<true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
    });
    KH_HIP(attr_rc);
    for (int64_t b0 = 0; b0 < batch; b0 += kMhMaxRows) {
      hipLaunchKernelGGL(minhash_rows_kernel<false>, dim3(static_cast<unsigned>(std::min(batch - b0, kMhMaxRows))),
                         dim3(kMhThreads), sizeof(uint32_t) * h->dim, st, h->perms_dev, h->dim, h->k, h->L,
                         x + b0 * ldx, ldx, nullptr, nullptr, codes + b0 * h->L);
      KH_LAUNCHED();
    }
    return KH_OK;
  } else if (h->kind == KH_FAMILY_MINHASH)
    hipLaunchKernelGGL(minhash_kernel, dim3(blocks), dim3(kRankThreads), 0, st, h->perms_dev, h->dim,
                       h->k, h->L, x, ldx, batch, codes);
  else  // WTA and DWTA hash dense rows alike (dwta.rs:143-152)
    hipLaunchKernelGGL(wta_hash_kernel<false>, dim3(blocks), dim3(kRankThreads), 0, st,
                       h->windows_dev, h->k, h->L, h->ws, h->bits, x, ldx, nullptr, nullptr, nullptr,
                       batch, codes);
  KH_LAUNCHED();
  return KH_OK;
}

int rank_hash_sparse_launch(const kh_hash_family* h, const int64_t* xoff, const uint32_t* xidx,
                            const float* xval, int64_t batch, uint32_t* codes, hipStream_t st) {
  if (batch == 0) return KH_OK;
  const int64_t n = batch * h->L;
  const unsigned blocks = static_cast<unsigned>((n + kRankThreads - 1) / kRankThreads);
  if (h->kind == KH_FAMILY_MINHASH) {
    for (int64_t b0 = 0; b0 < batch; b0 += kMhMaxRows) {
      hipLaunchKernelGGL(minhash_rows_kernel<true>, dim3(static_cast<unsigned>(std::min(batch - b0, kMhMaxRows))),
                         dim3(kMhThreads), 0, st, h->perms_dev, h->dim, h->k, h->L, nullptr, 0, xoff + b0,
                         xidx, codes + b0 * h->L);
      KH_LAUNCHED();
    }
    return KH_OK;
  } else if (h->kind == KH_FAMILY_DWTA)
    hipLaunchKernelGGL(dwta_sparse_kernel, dim3(blocks), dim3(kRankThreads), 0, st, h->windows_dev,
                       h->fallback_dev, h->k, h->L, h->ws, h->bits, xoff, xidx, xval, batch, codes);
  else
    hipLaunchKernelGGL(wta_hash_kernel<true>, dim3(blocks), dim3(kRankThreads), 0, st, h->windows_dev,
                       h->k, h->L, h->ws, h->bits, nullptr, 0, xoff, xidx, xval, batch, codes);
  KH_LAUNCHED();
  return KH_OK;
}

}  // namespace kh

using namespace kh;

static int rank_check(int input_dim, int k, int num_tables, kh_hash_family** out) {
  KH_CHECK_ARG(out != nullptr, "null out");
  *out = nullptr;
  KH_CHECK_ARG(input_dim > 0 && num_tables > 0 && num_tables <= 256,
               "input_dim must be positive and num_tables in [1,256]");
  KH_CHECK_ARG(k >= 1 && k <= kMaxMinHashBins, "k (%d) must be in [1,24] (2^k buckets per table)", k);
  return KH_OK;
}

// Upload a family's tables; takes ownership of h.
static int rank_finish(kh_hash_family* h, const std::vector<uint32_t>& fallback, kh_hash_family** out) {
  auto up = [&](const std::vector<uint32_t>& v, uint32_t** dst) {
    *dst = static_cast<uint32_t*>(dev_alloc(sizeof(uint32_t) * std::max<size_t>(v.size(), 1)));
    return *dst && (v.empty() || hipMemcpy(*dst, v.data(), sizeof(uint32_t) * v.size(),
                                           hipMemcpyHostToDevice) == hipSuccess);
  };
  bool ok = true;
  if (h->kind == KH_FAMILY_MINHASH) ok = up(h->perms_host, &h->perms_dev);
  else ok = up(h->windows_host, &h->windows_dev) && (h->kind != KH_FAMILY_DWTA || up(fallback, &h->fallback_dev));
  if (!ok) {
    set_error("hash family upload failed");
    kh_hash_family_destroy(h);
    return KH_ERR_ALLOC;
  }
  *out = h;
  return KH_OK;
}

static int wta_make(int kind, int input_dim, int k, int num_tables, int window_size,
                    const uint32_t* windows_host, uint64_t seed, kh_hash_family** out) {
  int rc = rank_check(input_dim, k, num_tables, out);
  if (rc != KH_OK) return rc;
  KH_CHECK_ARG(window_size >= 1 && window_size <= input_dim, "window_size (%d) must be in [1, input_dim]",
               window_size);
  const int bits = window_size <= 1 ? 1 : static_cast<int>(std::ceil(std::log2(static_cast<double>(window_size))));
  KH_CHECK_ARG(k * bits <= 64, "k * bits_per_window = %d exceeds 64", k * bits);
  auto* h = new kh_hash_family();
  h->kind = kind;
  h->dim = input_dim;
  h->k = k;
  h->L = num_tables;
  h->ws = window_size;
  h->bits = bits;
  const size_t n = static_cast<size_t>(num_tables) * k * window_size;
  h->windows_host.resize(n);
  if (windows_host) {
    for (size_t i = 0; i < n; ++i)
      if (windows_host[i] >= static_cast<uint32_t>(input_dim)) {
        delete h;
        set_error("window entry %zu = %u not below input_dim %d", i, windows_host[i], input_dim);
        return KH_ERR_ARG;
      }
    std::copy(windows_host, windows_host + n, h->windows_host.begin());
  } else {
    wta_windows(input_dim, k, num_tables, window_size, seed, h->windows_host.data());
  }
  std::vector<uint32_t> fb;
  if (kind == KH_FAMILY_DWTA) {
    fb.resize(static_cast<size_t>(num_tables) * k);
    for (int t = 0; t < num_tables; ++t)
      for (int f = 0; f < k; ++f)
        fb[static_cast<size_t>(t) * k + f] =
            static_cast<uint32_t>(default_hasher_u64x2(t, f) % static_cast<uint64_t>(window_size));
  }
  return rank_finish(h, fb, out);
}

extern "C" int kh_wta_create(int input_dim, int k, int num_tables, int window_size, uint64_t seed,
                             kh_hash_family** out) {
  return wta_make(KH_FAMILY_WTA, input_dim, k, num_tables, window_size, nullptr, seed, out);
}

extern "C" int kh_dwta_create(int input_dim, int k, int num_tables, int window_size, uint64_t seed,
                              kh_hash_family** out) {
  return wta_make(KH_FAMILY_DWTA, input_dim, k, num_tables, window_size, nullptr, seed, out);
}

extern "C" int kh_wta_from_windows(int dwta, int input_dim, int k, int num_tables, int window_size,
                                   const uint32_t* windows_host, kh_hash_family** out) {
  KH_CHECK_ARG(windows_host != nullptr, "null windows");
  return wta_make(dwta ? KH_FAMILY_DWTA : KH_FAMILY_WTA, input_dim, k, num_tables, window_size,
                  windows_host, 0, out);
}

static int minhash_make(int input_dim, int k, int num_tables, const uint32_t* perms_host,
                        uint64_t seed, kh_hash_family** out) {
  int rc = rank_check(input_dim, k, num_tables, out);
  if (rc != KH_OK) return rc;
  auto* h = new kh_hash_family();
  h->kind = KH_FAMILY_MINHASH;
  h->dim = input_dim;
  h->k = k;
  h->L = num_tables;
  const size_t n = static_cast<size_t>(num_tables) * input_dim;
  h->perms_host.resize(n);
  if (perms_host) {
    for (size_t i = 0; i < n; ++i)
      if (perms_host[i] >= static_cast<uint32_t>(input_dim)) {
        delete h;
        set_error("permutation entry %zu = %u not below input_dim %d", i, perms_host[i], input_dim);
        return KH_ERR_ARG;
      }
    std::copy(perms_host, perms_host + n, h->perms_host.begin());
  } else {
    minhash_perms(input_dim, num_tables, seed, h->perms_host.data());
  }
  return rank_finish(h, {}, out);
}

extern "C" int kh_minhash_create(int input_dim, int k, int num_tables, uint64_t seed,
                                 kh_hash_family** out) {
  return minhash_make(input_dim, k, num_tables, nullptr, seed, out);
}

extern "C" int kh_minhash_from_permutations(int input_dim, int k, int num_tables,
                                            const uint32_t* perms_host, kh_hash_family** out) {
  KH_CHECK_ARG(perms_host != nullptr, "null permutations");
  return minhash_make(input_dim, k, num_tables, perms_host, 0, out);
}

extern "C" int kh_hash_family_kind(const kh_hash_family* h, int* kind, int* window_size) {
  KH_CHECK_ARG(h != nullptr, "null family");
  if (kind) *kind = h->kind;
  if (window_size) *window_size = h->ws;
  return KH_OK;
}

extern "C" int kh_hash_family_tables(const kh_hash_family* h, uint32_t* out_host) {
  KH_CHECK_ARG(h && out_host, "null argument");
  if (h->kind == KH_FAMILY_MINHASH)
    std::copy(h->perms_host.begin(), h->perms_host.end(), out_host);
  else if (h->kind == KH_FAMILY_WTA || h->kind == KH_FAMILY_DWTA)
    std::copy(h->windows_host.begin(), h->windows_host.end(), out_host);
  else {
    set_error("a hyperplane family has no windows or permutations (kh_hash_family_planes)");
    return KH_ERR_UNSUPPORTED;
  }
  return KH_OK;
}
