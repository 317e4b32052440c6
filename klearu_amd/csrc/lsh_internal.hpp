// lsh_internal.hpp -- handle layouts shared by lsh.hip and slide.hip.
#pragma once
#include <vector>

#include "common.hpp"

struct kh_hash_family {
  int dim = 0, k = 0, L = 0;
  int kind = KH_FAMILY_TERNARY;          // KH_FAMILY_*: hyperplanes or a rank-based family
  int ws = 0, bits = 0;                  // WTA / DWTA: window size, bits per window
  std::vector<uint32_t> windows_host;    // WTA / DWTA [L][k][ws]
  uint32_t* windows_dev = nullptr;
  uint32_t* fallback_dev = nullptr;      // DWTA [L][k]: empty-window position
  std::vector<uint32_t> perms_host;      // MinHash [L][dim]
  uint32_t* perms_dev = nullptr;
  std::vector<int8_t> planes_host;  // [L][k][dim]
  int8_t* planes_dev = nullptr;     // [L*k][dim]
  // Nonzero lists of the planes, transposed so that the planes handled by
  // consecutive lanes are adjacent: entry j of plane p at ent_t[j*L*k + p],
  // (dim << 1) | (sign < 0), in dimension order; rows past a plane's nnz are 0.
  int32_t* nnz = nullptr;           // [L*k]
  uint32_t* ent_t = nullptr;        // [ent_rows][L*k]
  int ent_rows = 0;                 // max nnz rounded up to the hash kernel's batch
  // Planes as BF16 matrix-core operands (L*k <= 1024, dim <= 8192):
  // [ceil(dim/32)][ceil(L*k/16)][64 lanes] x 8 values; null otherwise.
  uint4* bt_dev = nullptr;
  int bt_ksteps = 0, bt_tiles = 0;
  // 2-bit plane signs for the per-row LDS kernel (dim small enough to stage
  // them): group g holds tables g*sg_tpb.. (planes q = 0..sg_tpb*k-1 of the
  // group), as [dim][sg_words] words, plane q in bits 2(q%16), 2(q%16)+1 of
  // word q/16 (01 = +1, 11 = -1, 00 = no term); each group padded to sg_n4
  // uint4.  Null when dim or k rule it out.
  uint4* sg_dev = nullptr;
  int sg_tpb = 0, sg_groups = 0, sg_words = 0, sg_n4 = 0;
};

namespace kh {
// Grow-only device scratch slots of an index's mutation calls, used as a stack.
struct ScratchArena {
  std::vector<std::pair<void*, size_t>> slots;
  size_t cursor = 0;
  ScratchArena() = default;
  ScratchArena(const ScratchArena&) = delete;
  ScratchArena& operator=(const ScratchArena&) = delete;
  ~ScratchArena() {
    for (auto& s : slots) dev_free(s.first);
  }
};
}  // namespace kh

struct kh_lsh_index {
  const kh_hash_family* h = nullptr;
  int type = 0, cap = 0, L = 0, k = 0, nb = 0;
  uint32_t* data = nullptr;   // [L][nb][cap]
  uint32_t* len = nullptr;    // [L][nb]
  uint64_t* count = nullptr;  // [L][nb]
  uint32_t id_bound = 0;      // 1 + largest id inserted so far (ids are below 2^31)
  mutable kh::StreamWs ws;    // query scratch per stream
  kh::ScratchArena arena;     // insert / remove / rebuild scratch, kept between calls
};

namespace kh {

int hash_dense_launch(const kh_hash_family* h, const float* x, int64_t ldx, int64_t batch,
                      uint32_t* codes, hipStream_t st);
int hash_sparse_launch(const kh_hash_family* h, const int64_t* xoff, const uint32_t* xidx,
                       const float* xval, int64_t batch, uint32_t* codes, hipStream_t st);
// Per-row unique ids (ascending) and hit counts into [batch][stride] buffers.
int query_launch(const kh_lsh_index* idx, const uint32_t* qcodes, int64_t batch, uint32_t* qids,
                 uint32_t* qcnt, int stride, int32_t* ulen, hipStream_t st);
int query_stride(const kh_lsh_index* idx);
// The rank-based families (hash_rank.hip), called by the two launchers above.
int rank_hash_dense_launch(const kh_hash_family* h, const float* x, int64_t ldx, int64_t batch,
                           uint32_t* codes, hipStream_t st);
int rank_hash_sparse_launch(const kh_hash_family* h, const int64_t* xoff, const uint32_t* xidx,
                            const float* xval, int64_t batch, uint32_t* codes, hipStream_t st);
// Row lengths -> CSR offsets, copies of up to four per-row arrays, then a
// synchronising capacity check.
int csr_finish(const uint32_t* qids, const uint32_t* qcnt, const float* f1, const float* f2,
               int stride, const int32_t* ulen, int64_t batch, int64_t* off, uint32_t* ids,
               uint32_t* cnts, float* o1, float* o2, int64_t capacity, hipStream_t st);

}  // namespace kh
