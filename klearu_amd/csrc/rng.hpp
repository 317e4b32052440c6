// rng.hpp -- host-side rand 0.8 StdRng (ChaCha12) for hyperplane generation.
#pragma once
#include <cstdint>

namespace kh {

void chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]);

class StdRng {
 public:
  static StdRng seed_from_u64(uint64_t seed);
  uint32_t next_u32();
  uint64_t next_u64();
  double gen_f64();
  // rand 0.8.5 Rng::gen_range(0..n) for u32 (UniformInt::sample_single)
  uint32_t gen_range_u32(uint32_t n);
  // SliceRandom::shuffle (rand 0.8.5): Fisher-Yates from the last element
  void shuffle(uint32_t* v, int64_t n);

 private:
  void refill();
  uint32_t key_[8] = {};
  uint64_t counter_ = 0;
  uint32_t buf_[64] = {};
  int idx_ = 64;
};

// planes[num_tables][k][dim] in {-1, 0, +1}, the draw order of SimHash::new.
void simhash_planes(int dim, int k, int num_tables, uint64_t seed, int8_t* planes);
// Dense ternary form of SparseRandomProjection::new's sparse (idx, sign) lists.
void srp_planes(int dim, int k, int num_tables, float sparsity, uint64_t seed, int8_t* planes);
// WtaHash::new / DwtaHash::new windows[L][k][ws] (first ws of a fresh shuffle each).
void wta_windows(int dim, int k, int num_tables, int ws, uint64_t seed, uint32_t* windows);
// MinHash::new permutations[L][dim].
void minhash_perms(int dim, int num_tables, uint64_t seed, uint32_t* perms);
// SipHash-1-3 (keys 0, 0) of two little-endian u64 words: std's DefaultHasher
// after hashing two usize values.
uint64_t default_hasher_u64x2(uint64_t a, uint64_t b);

}  // namespace kh
