// rng.hpp -- host-side rand 0.8 StdRng (ChaCha12) for hyperplane generation.
#pragma once
#include <cstdint>

namespace kh {

void chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]);

class StdRng {
 public:
  static StdRng seed_from_u64(uint64_t seed);
  uint64_t next_u64();
  double gen_f64();

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

}  // namespace kh
