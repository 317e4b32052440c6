// rng.cpp -- host-side rand 0.8 StdRng stream used by SimHash::new and
// SparseRandomProjection::new (crates/klearu-core/src/hash/simhash.rs:37-71,
// hash/srp.rs:43-84), so that kh_simhash_create(dim, k, L, seed) draws the
// same hyperplanes as the reference constructor.
//
// StdRng in rand 0.8.5 is rand_chacha 0.3.1's ChaCha12Rng: the ChaCha block
// function (RFC 7539 section 2.3) with 12 rounds, key = 32-byte seed, 64-bit
// block counter in words 12-13 starting at 0, stream id 0 in words 14-15,
// buffered four blocks (64 words) at a time.  seed_from_u64 (rand_core 0.6.4)
// fills the seed with eight PCG32 outputs, advancing the LCG before each
// output.  gen::<f64>() takes the 53 high bits of next_u64() (low word first)
// and scales by 2^-53.
#include "rng.hpp"

#include <algorithm>
#include <vector>

namespace kh {

static inline uint32_t rotl(uint32_t v, int s) { return (v << s) | (v >> (32 - s)); }

static void quarter(uint32_t* x, int a, int b, int c, int d) {
  x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
  x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
  x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
  x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
}

void chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]) {
  uint32_t x[16];
  for (int i = 0; i < 16; ++i) x[i] = in[i];
  for (int r = 0; r < rounds; r += 2) {
    quarter(x, 0, 4, 8, 12);
    quarter(x, 1, 5, 9, 13);
    quarter(x, 2, 6, 10, 14);
    quarter(x, 3, 7, 11, 15);
    quarter(x, 0, 5, 10, 15);
    quarter(x, 1, 6, 11, 12);
    quarter(x, 2, 7, 8, 13);
    quarter(x, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
}

StdRng StdRng::seed_from_u64(uint64_t state) {
  StdRng r;
  for (int i = 0; i < 8; ++i) {
    state = state * 6364136223846793005ull + 11634580027462260723ull;
    const uint32_t xs = static_cast<uint32_t>(((state >> 18) ^ state) >> 27);
    const uint32_t rot = static_cast<uint32_t>(state >> 59);
    r.key_[i] = (xs >> rot) | (xs << ((32u - rot) & 31u));
  }
  return r;
}

void StdRng::refill() {
  uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
  for (int i = 0; i < 8; ++i) in[4 + i] = key_[i];
  in[14] = 0;
  in[15] = 0;
  for (int blk = 0; blk < 4; ++blk) {
    const uint64_t c = counter_ + static_cast<uint64_t>(blk);
    in[12] = static_cast<uint32_t>(c);
    in[13] = static_cast<uint32_t>(c >> 32);
    chacha_block(in, 12, buf_ + 16 * blk);
  }
  counter_ += 4;
  idx_ = 0;
}

uint64_t StdRng::next_u64() {
  if (idx_ < 63) {
    const uint64_t lo = buf_[idx_], hi = buf_[idx_ + 1];
    idx_ += 2;
    return (hi << 32) | lo;
  }
  if (idx_ >= 64) {
    refill();
    idx_ = 2;
    return (static_cast<uint64_t>(buf_[1]) << 32) | buf_[0];
  }
  const uint64_t lo = buf_[63];
  refill();
  idx_ = 1;
  return (static_cast<uint64_t>(buf_[0]) << 32) | lo;
}

uint32_t StdRng::next_u32() {
  if (idx_ >= 64) refill();
  return buf_[idx_++];
}

// sample_single_inclusive(0, n - 1) of rand 0.8.5's UniformInt<u32>: the high
// word of draw * n, rejecting draws whose low word exceeds the conservative
// zone (n << lzcnt(n)) - 1.
uint32_t StdRng::gen_range_u32(uint32_t n) {
  const uint32_t zone = (n << __builtin_clz(n)) - 1u;
  for (;;) {
    const uint64_t m = static_cast<uint64_t>(next_u32()) * n;
    if (static_cast<uint32_t>(m) <= zone) return static_cast<uint32_t>(m >> 32);
  }
}

void StdRng::shuffle(uint32_t* v, int64_t n) {
  for (int64_t i = n - 1; i >= 1; --i) {
    const uint32_t j = gen_range_u32(static_cast<uint32_t>(i + 1));
    const uint32_t t = v[i];
    v[i] = v[j];
    v[j] = t;
  }
}

double StdRng::gen_f64() {
  return static_cast<double>(next_u64() >> 11) * (1.0 / 9007199254740992.0);
}

void simhash_planes(int dim, int k, int num_tables, uint64_t seed, int8_t* planes) {
  StdRng r = StdRng::seed_from_u64(seed);
  const double lo = 1.0 / 6.0, hi = 1.0 / 6.0 + 2.0 / 3.0;
  const int64_t n = static_cast<int64_t>(num_tables) * k * dim;
  for (int64_t i = 0; i < n; ++i) {
    const double v = r.gen_f64();
    planes[i] = v < lo ? -1 : (v < hi ? 0 : 1);
  }
}

void srp_planes(int dim, int k, int num_tables, float sparsity, uint64_t seed, int8_t* planes) {
  StdRng r = StdRng::seed_from_u64(seed);
  const double pneg = static_cast<double>(sparsity) / 2.0;
  const double pzero_end = pneg + (1.0 - static_cast<double>(sparsity));
  const int64_t n = static_cast<int64_t>(num_tables) * k * dim;
  for (int64_t i = 0; i < n; ++i) {
    const double v = r.gen_f64();
    planes[i] = v < pneg ? -1 : (v >= pzero_end ? 1 : 0);
  }
}

void wta_windows(int dim, int k, int num_tables, int ws, uint64_t seed, uint32_t* windows) {
  StdRng r = StdRng::seed_from_u64(seed);
  std::vector<uint32_t> perm(dim);
  for (int t = 0; t < num_tables; ++t)
    for (int f = 0; f < k; ++f) {
      for (int d = 0; d < dim; ++d) perm[d] = static_cast<uint32_t>(d);
      r.shuffle(perm.data(), dim);
      std::copy(perm.begin(), perm.begin() + ws, windows + (static_cast<int64_t>(t) * k + f) * ws);
    }
}

void minhash_perms(int dim, int num_tables, uint64_t seed, uint32_t* perms) {
  StdRng r = StdRng::seed_from_u64(seed);
  for (int t = 0; t < num_tables; ++t) {
    uint32_t* p = perms + static_cast<int64_t>(t) * dim;
    for (int d = 0; d < dim; ++d) p[d] = static_cast<uint32_t>(d);
    r.shuffle(p, dim);
  }
}

// SipHash-1-3: one compression round per 8-byte word, three finalisation
// rounds (Aumasson & Bernstein's SipHash with c = 1, d = 3, as std's
// DefaultHasher), keys k0 = k1 = 0.
static inline uint64_t rotl64(uint64_t v, int s) { return (v << s) | (v >> (64 - s)); }
static void sip_round(uint64_t& v0, uint64_t& v1, uint64_t& v2, uint64_t& v3) {
  v0 += v1; v1 = rotl64(v1, 13); v1 ^= v0; v0 = rotl64(v0, 32);
  v2 += v3; v3 = rotl64(v3, 16); v3 ^= v2;
  v0 += v3; v3 = rotl64(v3, 21); v3 ^= v0;
  v2 += v1; v1 = rotl64(v1, 17); v1 ^= v2; v2 = rotl64(v2, 32);
}

uint64_t default_hasher_u64x2(uint64_t a, uint64_t b) {
  uint64_t v0 = 0x736f6d6570736575ull, v1 = 0x646f72616e646f6dull;
  uint64_t v2 = 0x6c7967656e657261ull, v3 = 0x7465646279746573ull;
  for (uint64_t m : {a, b}) {
    v3 ^= m;
    sip_round(v0, v1, v2, v3);
    v0 ^= m;
  }
  const uint64_t fin = 16ull << 56;  // length byte, no tail
  v3 ^= fin;
  sip_round(v0, v1, v2, v3);
  v0 ^= fin;
  v2 ^= 0xff;
  for (int r = 0; r < 3; ++r) sip_round(v0, v1, v2, v3);
  return v0 ^ v1 ^ v2 ^ v3;
}

}  // namespace kh
