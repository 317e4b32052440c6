/*
 * oracle.c -- CPU restatement of klearu's activation-sparse inference path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library and
 * the timed CPU port for bench.py's cpu_baseline.  Never linked by the product.
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off -fno-fast-math oracle.c -lm
 * (no -mfma: fmaf() is then glibc's correctly rounded fused multiply-add, the
 * same single rounding as _mm256_fmadd_ps).
 *
 * Citations are path:line in the reference tree (QuilibriumNetwork/klearu).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* klearu-accel: crates/klearu-accel/src/simd/mod.rs                         */
/* ======================================================================== */

/* hsum_avx2 (simd/mod.rs:128-141): [v0+v4, v1+v5, v2+v6, v3+v7] -> movehdup
 * pairs lane 1 into lane 0 and lane 3 into lane 2 -> movehl brings lane 2 down
 * -> add_ss.  Result: ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)).
 * Pinned: brute-force equality with the AVX2 intrinsic build (oracle_avx2.c)
 * in tests/test_oracle_accel.py. */
static float hsum8(const float v[8]) {
  float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
  float t0 = s0 + s1;
  float t2 = s2 + s3;
  return t0 + t2;
}

/* dense_dot_dense_avx2 (simd/mod.rs:174-207): two 8-lane FMA accumulators over
 * 16-element chunks, an optional extra 8-chunk into acc0, hsum(acc0+acc1), then
 * a scalar tail `sum += a[i]*b[i]` (product rounded, then added).
 * Pinned: KATs simd/mod.rs:428 (=32), AVX2 intrinsic build equality. */
float or_dense_dot_avx2_order(const float* a, const float* b, int64_t n) {
  float acc0[8], acc1[8];
  for (int l = 0; l < 8; ++l) acc0[l] = acc1[l] = 0.0f;
  int64_t chunks = n / 16;
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t o = c * 16;
    for (int l = 0; l < 8; ++l) acc0[l] = fmaf(a[o + l], b[o + l], acc0[l]);
    for (int l = 0; l < 8; ++l) acc1[l] = fmaf(a[o + 8 + l], b[o + 8 + l], acc1[l]);
  }
  int64_t rs = chunks * 16;
  int extra = (rs + 8 <= n);
  if (extra)
    for (int l = 0; l < 8; ++l) acc0[l] = fmaf(a[rs + l], b[rs + l], acc0[l]);
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = acc0[l] + acc1[l];
  float sum = hsum8(v);
  for (int64_t i = extra ? rs + 8 : rs; i < n; ++i) {
    float p = a[i] * b[i];
    sum = sum + p;
  }
  return sum;
}

/* dense_dot_dense_scalar (simd/mod.rs:74-76): iterator sum of products. */
float or_dense_dot_scalar(const float* a, const float* b, int64_t n) {
  float s = -0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float p = a[i] * b[i];
    s = s + p;
  }
  return s;
}

/* sparse_dot_dense_avx2 (simd/mod.rs:145-170): one 8-lane FMA accumulator over
 * chunks of 8 gathered values, hsum, then a scalar tail. */
float or_sparse_dot_dense_avx2_order(const uint32_t* idx, const float* val, int64_t nnz,
                                     const float* dense) {
  float acc[8];
  for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
  int64_t chunks = nnz / 8;
  for (int64_t c = 0; c < chunks; ++c)
    for (int l = 0; l < 8; ++l)
      acc[l] = fmaf(val[c * 8 + l], dense[idx[c * 8 + l]], acc[l]);
  float sum = hsum8(acc);
  for (int64_t i = chunks * 8; i < nnz; ++i) {
    float p = val[i] * dense[idx[i]];
    sum = sum + p;
  }
  return sum;
}

/* sparse_dot_dense_scalar (simd/mod.rs:39-45): `let mut sum = 0.0f32`. */
float or_sparse_dot_dense_scalar(const uint32_t* idx, const float* val, int64_t nnz,
                                 const float* dense) {
  float s = 0.0f;
  for (int64_t i = 0; i < nnz; ++i) {
    float p = val[i] * dense[idx[i]];
    s = s + p;
  }
  return s;
}

/* scatter_add_avx2 (simd/mod.rs:211-236): scaled = val*scale (vector multiply,
 * same rounding as scalar), then sequential `dense[idx] += scaled` in index
 * order, so duplicate indices accumulate in order.  The scalar tail
 * (`dense[idx] += values[i] * scale`) has identical arithmetic. */
void or_scatter_add(const uint32_t* idx, const float* val, int64_t n, float* dense, float scale) {
  for (int64_t i = 0; i < n; ++i) {
    float s = val[i] * scale;
    dense[idx[i]] = dense[idx[i]] + s;
  }
}

/* ======================================================================== */
/* klearu-accel: crates/klearu-accel/src/bf16/mod.rs (half 2.x bf16)         */
/* ======================================================================== */

/* bf16::from_f32 (half crate, used at bf16/mod.rs:38,57,87): round to nearest,
 * ties to even; NaN keeps its sign and top payload bits and is forced quiet.
 * Pinned: closed form + round-trip KATs in tests. */
uint16_t or_bf16_from_f32(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  uint32_t r = u + 0x7fffu + lsb;
  return (uint16_t)(r >> 16);
}

/* bf16::to_f32: the bf16 bits are the high half of the f32. */
float or_bf16_to_f32(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void or_bf16_from_f32_n(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_from_f32(x[i]);
}

/* Bf16Weights::dot_f32 (bf16/mod.rs:64-77): iterator sum of w.to_f32()*x. */
float or_bf16_dot_f32(const uint16_t* w, const float* x, int64_t n) {
  float s = -0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float p = or_bf16_to_f32(w[i]) * x[i];
    s = s + p;
  }
  return s;
}

/* Bf16FullMode::dot (bf16/mod.rs:122-134). */
float or_bf16_full_dot(const uint16_t* a, const uint16_t* b, int64_t n) {
  float s = -0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float p = or_bf16_to_f32(a[i]) * or_bf16_to_f32(b[i]);
    s = s + p;
  }
  return s;
}

/* f32::exp (Rust std -> glibc expf on x86-64 Linux) of every element; the
 * reference's sigmoid / SiLU / softmax call it (mlp_predictor.rs:121,
 * sparse_mlp.rs:41, layer.rs:295, sparse_attention.rs:88).
 * Pinned: it is the platform libm itself. */
void or_expf_n(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

/* Bf16Weights::update_from_f32 (bf16/mod.rs:85-88) applied to every element. */
void or_bf16_update_from_f32(uint16_t* w, const float* delta, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float c = or_bf16_to_f32(w[i]);
    w[i] = or_bf16_from_f32(c + delta[i]);
  }
}

/* ======================================================================== */
/* rand 0.8.5 StdRng = rand_chacha 0.3.1 ChaCha12Rng, seeded by rand_core     */
/* 0.6.4 SeedableRng::seed_from_u64.  Third-party crates, not in the reference */
/* tree; restated from their published algorithms (ChaCha: RFC 7539 block     */
/* function with djb's 64-bit counter / 64-bit stream layout; PCG32 XSH-RR).  */
/* Call sites: klearu-core/src/hash/simhash.rs:38-71, hash/srp.rs:55-75.     */
/* Parity: block function pinned by RFC 7539 vectors; PCG32 output function   */
/* pinned by the PCG reference demo vector; the composed seed->plane stream is */
/* parity unpinned (no reference test holds a drawn value).                   */
/* ======================================================================== */

#define ROTL32(v, s) (((v) << (s)) | ((v) >> (32 - (s))))
#define CHACHA_QR(a, b, c, d)                 \
  do {                                        \
    a += b; d ^= a; d = ROTL32(d, 16);        \
    c += d; b ^= c; b = ROTL32(b, 12);        \
    a += b; d ^= a; d = ROTL32(d, 8);         \
    c += d; b ^= c; b = ROTL32(b, 7);         \
  } while (0)

void or_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]) {
  uint32_t x[16];
  memcpy(x, in, sizeof(x));
  for (int r = 0; r < rounds; r += 2) {
    CHACHA_QR(x[0], x[4], x[8], x[12]);
    CHACHA_QR(x[1], x[5], x[9], x[13]);
    CHACHA_QR(x[2], x[6], x[10], x[14]);
    CHACHA_QR(x[3], x[7], x[11], x[15]);
    CHACHA_QR(x[0], x[5], x[10], x[15]);
    CHACHA_QR(x[1], x[6], x[11], x[12]);
    CHACHA_QR(x[2], x[7], x[8], x[13]);
    CHACHA_QR(x[3], x[4], x[9], x[14]);
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
}

/* PCG32 XSH-RR output permutation of a 64-bit LCG state. */
uint32_t or_pcg32_output(uint64_t s) {
  uint32_t xs = (uint32_t)(((s >> 18) ^ s) >> 27);
  uint32_t rot = (uint32_t)(s >> 59);
  return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

static void stdrng_refill(or_stdrng* r) {
  uint32_t in[16];
  in[0] = 0x61707865u; in[1] = 0x3320646eu; in[2] = 0x79622d32u; in[3] = 0x6b206574u;
  for (int i = 0; i < 8; ++i) in[4 + i] = r->key[i];
  in[14] = 0; in[15] = 0; /* stream id 0 */
  for (int blk = 0; blk < 4; ++blk) {
    uint64_t c = r->counter + (uint64_t)blk;
    in[12] = (uint32_t)c;
    in[13] = (uint32_t)(c >> 32);
    or_chacha_block(in, 12, r->buf + 16 * blk);
  }
  r->counter += 4;
  r->idx = 0;
}

void or_stdrng_from_seed(or_stdrng* r, const uint8_t seed[32]) {
  for (int i = 0; i < 8; ++i)
    r->key[i] = (uint32_t)seed[4 * i] | ((uint32_t)seed[4 * i + 1] << 8) |
                ((uint32_t)seed[4 * i + 2] << 16) | ((uint32_t)seed[4 * i + 3] << 24);
  r->counter = 0;
  r->idx = 64;
}

/* rand_core 0.6.4 seed_from_u64: advance the PCG32 LCG first, then output;
 * eight 32-bit outputs fill the 32-byte seed in little-endian order. */
void or_stdrng_seed_from_u64(or_stdrng* r, uint64_t state) {
  uint8_t seed[32];
  for (int i = 0; i < 8; ++i) {
    state = state * 6364136223846793005ull + 11634580027462260723ull;
    uint32_t x = or_pcg32_output(state);
    seed[4 * i] = (uint8_t)x;
    seed[4 * i + 1] = (uint8_t)(x >> 8);
    seed[4 * i + 2] = (uint8_t)(x >> 16);
    seed[4 * i + 3] = (uint8_t)(x >> 24);
  }
  or_stdrng_from_seed(r, seed);
}

uint32_t or_stdrng_next_u32(or_stdrng* r) {
  if (r->idx >= 64) stdrng_refill(r);
  return r->buf[r->idx++];
}

/* BlockRng::next_u64: low word first; a u64 that straddles a refill takes the
 * last word of the old buffer as its low half. */
uint64_t or_stdrng_next_u64(or_stdrng* r) {
  if (r->idx < 63) {
    uint64_t lo = r->buf[r->idx], hi = r->buf[r->idx + 1];
    r->idx += 2;
    return (hi << 32) | lo;
  }
  if (r->idx >= 64) {
    stdrng_refill(r);
    uint64_t lo = r->buf[0], hi = r->buf[1];
    r->idx = 2;
    return (hi << 32) | lo;
  }
  uint64_t lo = r->buf[63];
  stdrng_refill(r);
  uint64_t hi = r->buf[0];
  r->idx = 1;
  return (hi << 32) | lo;
}

/* Standard distribution for f64 (rand 0.8): 53 high bits times 2^-53. */
double or_stdrng_gen_f64(or_stdrng* r) {
  uint64_t v = or_stdrng_next_u64(r) >> 11;
  return (double)v * (1.0 / 9007199254740992.0);
}

/* ======================================================================== */
/* Hash families                                                             */
/* ======================================================================== */

/* SimHash::new + sample_ternary (hash/simhash.rs:37-71): table -> bit -> dim
 * order, r < 1/6 -> -1, r < 1/6 + 2/3 -> 0, else +1.  planes[L][k][dim]. */
void or_simhash_planes(int dim, int k, int num_tables, uint64_t seed, int8_t* planes) {
  or_stdrng r;
  or_stdrng_seed_from_u64(&r, seed);
  const double lo = 1.0 / 6.0, hi = 1.0 / 6.0 + 2.0 / 3.0;
  int64_t n = (int64_t)num_tables * k * dim;
  for (int64_t i = 0; i < n; ++i) {
    double v = or_stdrng_gen_f64(&r);
    planes[i] = v < lo ? -1 : (v < hi ? 0 : 1);
  }
}

/* SparseRandomProjection::new (hash/srp.rs:43-84): per projection t*k+b, per
 * dim d: r < s/2 -> -1; r >= s/2 + (1-s) -> +1; else 0 (s widened to f64).
 * Emitted as dense ternary planes[L*k][dim]; the sparse (idx, sign) list of
 * the reference is exactly the nonzero entries in ascending d. */
void or_srp_planes(int dim, int k, int num_tables, float sparsity, uint64_t seed, int8_t* planes) {
  or_stdrng r;
  or_stdrng_seed_from_u64(&r, seed);
  const double pneg = (double)sparsity / 2.0;
  const double pzero_end = pneg + (1.0 - (double)sparsity);
  int64_t n = (int64_t)num_tables * k * dim;
  for (int64_t i = 0; i < n; ++i) {
    double v = or_stdrng_gen_f64(&r);
    planes[i] = v < pneg ? -1 : (v >= pzero_end ? 1 : 0);
  }
}

/* dot_ternary_dense + hash_dense (hash/simhash.rs:75-85, :103-113); SRP's
 * dot_sparse_dense (hash/srp.rs:95-106) visits the same nonzero planes in the
 * same ascending-d order, so the same code serves both families.
 * Pinned: zero vector -> 2^k-1 (simhash.rs:232-240), dense==sparse
 * (simhash.rs:173,218), brute force in tests. */
uint64_t or_hash_dense(const int8_t* planes, int dim, int k, int table, const float* x) {
  uint64_t h = 0;
  for (int b = 0; b < k; ++b) {
    const int8_t* p = planes + ((int64_t)table * k + b) * dim;
    float s = 0.0f;
    for (int d = 0; d < dim; ++d) {
      if (p[d] == 1) s = s + x[d];
      else if (p[d] == -1) s = s - x[d];
    }
    if (s >= 0.0f) h |= 1ull << b;
  }
  return h;
}

/* dot_ternary_sparse + hash_sparse (hash/simhash.rs:89-100, :116-126). */
uint64_t or_hash_sparse(const int8_t* planes, int dim, int k, int table, const uint32_t* idx,
                        const float* val, int64_t nnz) {
  uint64_t h = 0;
  for (int b = 0; b < k; ++b) {
    const int8_t* p = planes + ((int64_t)table * k + b) * dim;
    float s = 0.0f;
    for (int64_t i = 0; i < nnz; ++i) {
      int8_t r = p[idx[i]];
      if (r == 1) s = s + val[i];
      else if (r == -1) s = s - val[i];
    }
    if (s >= 0.0f) h |= 1ull << b;
  }
  return h;
}

void or_hash_dense_batch(const int8_t* planes, int dim, int k, int num_tables, const float* x,
                         int64_t batch, uint32_t* codes) {
  for (int64_t i = 0; i < batch; ++i)
    for (int t = 0; t < num_tables; ++t)
      codes[i * num_tables + t] = (uint32_t)or_hash_dense(planes, dim, k, t, x + i * dim);
}

/* ======================================================================== */
/* WTA / DWTA / MinHash (klearu-core/src/hash/wta.rs, dwta.rs, minhash.rs)    */
/* ======================================================================== */

/* rand 0.8.5 Rng::gen_range(0..n) for u32 (UniformInt::sample_single ->
 * sample_single_inclusive): widening multiply of next_u32 by n, rejecting
 * low words above zone = (n << lzcnt(n)) - 1.  Third-party (rand 0.8.5, not in
 * the reference tree), restated from its published source; the composed
 * draws are parity unpinned (no reference test holds a drawn window). */
uint32_t or_rand_gen_range_u32(or_stdrng* r, uint32_t n) {
  const uint32_t zone = (n << __builtin_clz(n)) - 1u;
  for (;;) {
    const uint64_t m = (uint64_t)or_stdrng_next_u32(r) * n;
    if ((uint32_t)m <= zone) return (uint32_t)(m >> 32);
  }
}

/* SliceRandom::shuffle (rand 0.8.5 seq/mod.rs): for i = len-1 down to 1,
 * swap(i, gen_index(i + 1)); gen_index uses the u32 gen_range below 2^32. */
void or_rand_shuffle_u32(or_stdrng* r, uint32_t* v, int64_t n) {
  for (int64_t i = n - 1; i >= 1; --i) {
    const uint32_t j = or_rand_gen_range_u32(r, (uint32_t)(i + 1));
    const uint32_t t = v[i];
    v[i] = v[j];
    v[j] = t;
  }
}

/* WtaHash::new / DwtaHash::new window draws (wta.rs:42-90, dwta.rs:40-88):
 * per table, per hash function, shuffle a fresh 0..dim and keep the first
 * window_size entries.  windows[L][k][ws]. */
void or_wta_windows(int dim, int k, int num_tables, int ws, uint64_t seed, uint32_t* windows) {
  or_stdrng r;
  or_stdrng_seed_from_u64(&r, seed);
  uint32_t* perm = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)dim);
  for (int t = 0; t < num_tables; ++t)
    for (int f = 0; f < k; ++f) {
      for (int d = 0; d < dim; ++d) perm[d] = (uint32_t)d;
      or_rand_shuffle_u32(&r, perm, dim);
      memcpy(windows + ((int64_t)t * k + f) * ws, perm, sizeof(uint32_t) * (size_t)ws);
    }
  free(perm);
}

/* MinHash::new (minhash.rs:38-60): per table a shuffled 0..dim (u32). */
void or_minhash_perms(int dim, int num_tables, uint64_t seed, uint32_t* perms) {
  or_stdrng r;
  or_stdrng_seed_from_u64(&r, seed);
  for (int t = 0; t < num_tables; ++t) {
    uint32_t* p = perms + (int64_t)t * dim;
    for (int d = 0; d < dim; ++d) p[d] = (uint32_t)d;
    or_rand_shuffle_u32(&r, p, dim);
  }
}

/* bits_per_window (wta.rs:54-58): 1 for ws <= 1, else ceil(log2(ws)). */
int or_wta_bits(int ws) { return ws <= 1 ? 1 : (int)ceil(log2((double)ws)); }

/* argmax_dense (wta.rs:93-105): first strict maximum from -inf (NaN never
 * wins; all -inf / NaN gives 0). */
static int wta_argmax(const float* x, const uint32_t* win, int ws) {
  int best = 0;
  float bv = -INFINITY;
  for (int p = 0; p < ws; ++p) {
    const float v = x[win[p]];
    if (v > bv) { bv = v; best = p; }
  }
  return best;
}

/* WtaHash::hash_dense (wta.rs:108-119), also DwtaHash::hash_dense: the k
 * argmax positions packed from bit 0 up, bits per window each.
 * Pinned: brute-force tie / NaN / -inf KATs and the reference's positive-
 * scaling invariance (wta.rs:202-215) in tests/test_oracle_families.py. */
uint64_t or_wta_hash_dense(const uint32_t* windows, int k, int ws, int table, const float* x) {
  const int bits = or_wta_bits(ws);
  uint64_t h = 0;
  for (int f = 0; f < k; ++f)
    h |= (uint64_t)wta_argmax(x, windows + ((int64_t)table * k + f) * ws, ws) << (bits * f);
  return h;
}

/* SipHash-1-3 with keys 0, 0 over two little-endian u64 words: std's
 * DefaultHasher after `table.hash(); hash_fn.hash();` (usize writes), then
 * finish().  Pinned: the same round code with c = 2, d = 4 reproduces the
 * SipHash paper's reference vectors (tests/test_oracle_families.py). */
#define ROTL64(v, s) (((v) << (s)) | ((v) >> (64 - (s))))
static void sip_round(uint64_t* v) {
  v[0] += v[1]; v[1] = ROTL64(v[1], 13); v[1] ^= v[0]; v[0] = ROTL64(v[0], 32);
  v[2] += v[3]; v[3] = ROTL64(v[3], 16); v[3] ^= v[2];
  v[0] += v[3]; v[3] = ROTL64(v[3], 21); v[3] ^= v[0];
  v[2] += v[1]; v[1] = ROTL64(v[1], 17); v[1] ^= v[2]; v[2] = ROTL64(v[2], 32);
}
uint64_t or_siphash(int c_rounds, int d_rounds, uint64_t k0, uint64_t k1, const uint8_t* msg,
                    int64_t len) {
  uint64_t v[4] = {k0 ^ 0x736f6d6570736575ull, k1 ^ 0x646f72616e646f6dull,
                   k0 ^ 0x6c7967656e657261ull, k1 ^ 0x7465646279746573ull};
  int64_t i = 0;
  for (; i + 8 <= len; i += 8) {
    uint64_t m = 0;
    for (int b = 0; b < 8; ++b) m |= (uint64_t)msg[i + b] << (8 * b);
    v[3] ^= m;
    for (int r = 0; r < c_rounds; ++r) sip_round(v);
    v[0] ^= m;
  }
  uint64_t b = (uint64_t)(len & 0xff) << 56;
  for (int j = 0; i + j < len; ++j) b |= (uint64_t)msg[i + j] << (8 * j);
  v[3] ^= b;
  for (int r = 0; r < c_rounds; ++r) sip_round(v);
  v[0] ^= b;
  v[2] ^= 0xff;
  for (int r = 0; r < d_rounds; ++r) sip_round(v);
  return v[0] ^ v[1] ^ v[2] ^ v[3];
}

/* DwtaHash's empty-window fallback (dwta.rs:133-141): DefaultHasher of
 * (table, hash_fn) modulo window_size. */
uint32_t or_dwta_fallback(uint64_t table, uint64_t hash_fn, int ws) {
  uint8_t m[16];
  for (int b = 0; b < 8; ++b) {
    m[b] = (uint8_t)(table >> (8 * b));
    m[8 + b] = (uint8_t)(hash_fn >> (8 * b));
  }
  return (uint32_t)(or_siphash(1, 3, 0, 0, m, 16) % (uint64_t)ws);
}

/* DwtaHash::hash_sparse (dwta.rs:154-166, argmax_sparse :108-143): argmax over
 * the window positions whose dimension is stored in the (sorted) sparse
 * input, else the fallback.  WtaHash::hash_sparse is hash_dense of to_dense. */
uint64_t or_dwta_hash_sparse(const uint32_t* windows, int k, int ws, int table, const uint32_t* idx,
                             const float* val, int64_t nnz) {
  const int bits = or_wta_bits(ws);
  uint64_t h = 0;
  for (int f = 0; f < k; ++f) {
    const uint32_t* win = windows + ((int64_t)table * k + f) * ws;
    int best = -1;
    float bv = -INFINITY;
    for (int p = 0; p < ws; ++p) {
      int64_t lo = 0, hi = nnz;  /* binary search */
      while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        if (idx[mid] < win[p]) lo = mid + 1; else hi = mid;
      }
      if (lo < nnz && idx[lo] == win[p] && val[lo] > bv) { bv = val[lo]; best = p; }
    }
    const uint64_t pos = best >= 0 ? (uint64_t)best : or_dwta_fallback((uint64_t)table, (uint64_t)f, ws);
    h |= pos << (bits * f);
  }
  return h;
}

/* MinHash hash_impl (minhash.rs:64-136): per-bin minimum permuted index over
 * the nonzero dimensions (bin = permuted / ceil(dim/k), bins >= k dropped),
 * empty bins take the next non-empty bin circularly (all empty -> all 0),
 * then sum(h_i * P^i) with wrapping u64 arithmetic, P = 0x517cc1b727220a95,
 * masked to k bits.  nz: the nonzero dims (dense: x != 0 in index order;
 * sparse: every stored index).  Pinned: closed-form KATs in
 * tests/test_oracle_families.py. */
uint64_t or_minhash_hash(const uint32_t* perms, int dim, int k, int table, const uint32_t* nz,
                         int64_t n_nz) {
  const uint32_t* perm = perms + (int64_t)table * dim;
  const int64_t bin_size = (dim + k - 1) / k;
  uint32_t* mins = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)k);
  for (int b = 0; b < k; ++b) mins[b] = 0xffffffffu;
  for (int64_t i = 0; i < n_nz; ++i) {
    const uint32_t pv = perm[nz[i]];
    const int64_t bin = pv / bin_size;
    if (bin < k && pv < mins[bin]) mins[bin] = pv;
  }
  int all_empty = 1;
  for (int b = 0; b < k; ++b) if (mins[b] != 0xffffffffu) { all_empty = 0; break; }
  if (all_empty) {
    for (int b = 0; b < k; ++b) mins[b] = 0;
  } else {
    for (int b = 0; b < k; ++b)
      if (mins[b] == 0xffffffffu) {
        int j = (b + 1) % k;
        while (mins[j] == 0xffffffffu) j = (j + 1) % k;
        mins[b] = mins[j];
      }
  }
  const uint64_t mask = k >= 64 ? ~0ull : ((1ull << k) - 1ull);
  uint64_t h = 0, pp = 1;
  for (int b = 0; b < k; ++b) {
    h += (uint64_t)mins[b] * pp;
    pp *= 0x517cc1b727220a95ull;
  }
  free(mins);
  return h & mask;
}

/* ======================================================================== */
/* Buckets and the LSH index                                                 */
/* ======================================================================== */

/* ReservoirBucket::deterministic_rand (bucket/reservoir.rs:40-47): SplitMix64
 * finaliser of seed + golden gamma, reduced modulo bound. */
uint64_t or_reservoir_rand(uint64_t seed, uint64_t bound) {
  uint64_t z = seed + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z = z ^ (z >> 31);
  return z % bound;
}

/* FifoBucket::insert (bucket/fifo.rs:27-33): evict index 0 when full. */
static void fifo_insert(uint32_t* d, uint32_t* len, int cap, uint32_t id) {
  if (*len >= (uint32_t)cap) {
    memmove(d, d + 1, sizeof(uint32_t) * (*len - 1));
    *len -= 1;
  }
  d[(*len)++] = id;
}

/* ReservoirBucket::insert (bucket/reservoir.rs:51-67). */
static void reservoir_insert(uint32_t* d, uint32_t* len, uint64_t* count, int cap, uint32_t id) {
  *count += 1;
  if (*len < (uint32_t)cap) {
    d[(*len)++] = id;
    return;
  }
  uint64_t seed = *count * 0x517cc1b727220a95ull + (uint64_t)id;
  uint64_t j = or_reservoir_rand(seed, *count);
  if (j < (uint64_t)cap) {
    uint64_t slot = or_reservoir_rand(seed + 1, (uint64_t)cap);
    d[slot] = id;
  }
}

/* LshIndex::insert (lsh/index.rs:257-262) for ids in the given order, tables
 * inner; bucket = code & (2^k - 1) (index.rs:208-211).  data[L][2^k][cap],
 * len[L][2^k], count[L][2^k] (count is used by reservoir buckets only). */
void or_lsh_insert_many(int num_tables, int k, int cap, int bucket_type, uint32_t* data,
                        uint32_t* len, uint64_t* count, int64_t n, const uint32_t* ids,
                        const uint32_t* codes) {
  const int64_t nb = (int64_t)1 << k;
  for (int64_t i = 0; i < n; ++i)
    for (int t = 0; t < num_tables; ++t) {
      int64_t b = (int64_t)(codes[i * num_tables + t] & (uint32_t)(nb - 1));
      int64_t slot = (int64_t)t * nb + b;
      if (bucket_type == OR_BUCKET_FIFO)
        fifo_insert(data + slot * cap, len + slot, cap, ids[i]);
      else
        reservoir_insert(data + slot * cap, len + slot, count + slot, cap, ids[i]);
    }
}

/* Bucket::remove for FIFO and reservoir buckets (bucket/fifo.rs:35-42,
 * bucket/reservoir.rs:69-76): the first entry equal to id is replaced by the
 * last entry (Vec::swap_remove); the insertion count is unchanged.  Returns 1
 * when something was removed. */
static int bucket_remove(uint32_t* d, uint32_t* len, uint32_t id) {
  for (uint32_t q = 0; q < *len; ++q)
    if (d[q] == id) {
      d[q] = d[*len - 1];
      *len -= 1;
      return 1;
    }
  return 0;
}

/* LshIndexTrait::remove_with_weights (lsh/index.rs:271-276) for n vectors in
 * order, tables inner, from their codes[n][num_tables]. */
void or_lsh_remove_many(int num_tables, int k, int cap, uint32_t* data, uint32_t* len, int64_t n,
                        const uint32_t* ids, const uint32_t* codes) {
  const int64_t nb = (int64_t)1 << k;
  for (int64_t i = 0; i < n; ++i)
    for (int t = 0; t < num_tables; ++t) {
      int64_t b = (int64_t)(codes[i * num_tables + t] & (uint32_t)(nb - 1));
      int64_t slot = (int64_t)t * nb + b;
      bucket_remove(data + slot * cap, len + slot, ids[i]);
    }
}

/* LshIndexTrait::remove (lsh/index.rs:278-280 -> BucketStorage::remove_all,
 * :146-164) for n ids in order: every bucket of every table removes the id. */
void or_lsh_remove_all(int num_tables, int k, int cap, uint32_t* data, uint32_t* len, int64_t n,
                       const uint32_t* ids) {
  const int64_t nbk = (int64_t)num_tables << k;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t slot = 0; slot < nbk; ++slot) bucket_remove(data + slot * cap, len + slot, ids[i]);
}

static int cmp_u32(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/* collect_counts (lsh/index.rs:219-234): every occurrence of an id in the L
 * query buckets adds one to its count.  The reference returns HashMap order
 * (randomised per process); the canonical order here is ascending id.
 * Returns the number of unique ids; out arrays need L*cap entries. */
int64_t or_lsh_query(int num_tables, int k, int cap, const uint32_t* data, const uint32_t* len,
                     const uint32_t* codes, uint32_t* out_ids, uint32_t* out_counts) {
  const int64_t nb = (int64_t)1 << k;
  uint32_t* all = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)num_tables * cap + 4);
  int64_t m = 0;
  for (int t = 0; t < num_tables; ++t) {
    int64_t slot = (int64_t)t * nb + (codes[t] & (uint32_t)(nb - 1));
    for (uint32_t j = 0; j < len[slot]; ++j) all[m++] = data[slot * cap + j];
  }
  qsort(all, (size_t)m, sizeof(uint32_t), cmp_u32);
  int64_t u = 0;
  for (int64_t i = 0; i < m;) {
    int64_t j = i;
    while (j < m && all[j] == all[i]) ++j;
    out_ids[u] = all[i];
    if (out_counts) out_counts[u] = (uint32_t)(j - i);
    ++u;
    i = j;
  }
  free(all);
  return u;
}

/* ======================================================================== */
/* Sampling strategies                                                       */
/* ======================================================================== */

typedef struct { uint32_t id, count; } pair_ic;
static int cmp_topk(const void* a, const void* b) {
  const pair_ic* x = (const pair_ic*)a;
  const pair_ic* y = (const pair_ic*)b;
  if (x->count != y->count) return x->count > y->count ? -1 : 1;
  return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* TopKSampling::select (sampling/topk.rs:19-34): count desc, id asc, take k. */
int64_t or_sample_topk(const uint32_t* ids, const uint32_t* counts, int64_t n, int64_t k,
                       uint32_t* out) {
  pair_ic* p = (pair_ic*)malloc(sizeof(pair_ic) * (size_t)(n + 1));
  for (int64_t i = 0; i < n; ++i) { p[i].id = ids[i]; p[i].count = counts[i]; }
  qsort(p, (size_t)n, sizeof(pair_ic), cmp_topk);
  int64_t m = n < k ? n : k;
  for (int64_t i = 0; i < m; ++i) out[i] = p[i].id;
  free(p);
  return m;
}

/* ThresholdSampling::select (sampling/threshold.rs:20-43): count >= t in input
 * order; if none pass, the single best (highest count, then lowest id). */
int64_t or_sample_threshold(const uint32_t* ids, const uint32_t* counts, int64_t n,
                            uint32_t threshold, uint32_t* out) {
  if (n == 0) return 0;
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i)
    if (counts[i] >= threshold) out[m++] = ids[i];
  if (m > 0) return m;
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (counts[i] > counts[best] || (counts[i] == counts[best] && ids[i] < ids[best])) best = i;
  out[0] = ids[best];
  return 1;
}

/* ======================================================================== */
/* SLIDE neuron / layer                                                      */
/* ======================================================================== */

/* Neuron::forward (network/neuron.rs:47-62): iterator sum of w*x, then +bias. */
float or_neuron_forward(const float* w, float bias, const float* x, int64_t dim) {
  float s = -0.0f;
  for (int64_t d = 0; d < dim; ++d) {
    float p = w[d] * x[d];
    s = s + p;
  }
  return s + bias;
}

/* Neuron::forward_sparse (network/neuron.rs:66-68) via SparseVector::dot_dense
 * (tensor/sparse.rs:89-101): iterator sum of val*w[idx] over stored entries. */
float or_neuron_forward_sparse(const float* w, float bias, const uint32_t* idx, const float* val,
                               int64_t nnz) {
  float s = -0.0f;
  for (int64_t i = 0; i < nnz; ++i) {
    float p = val[i] * w[idx[i]];
    s = s + p;
  }
  return s + bias;
}

/* apply_activation / apply_softmax (network/layer.rs:250-261, :286-308). */
void or_layer_activate(const float* pre, int64_t n, int act, float* out) {
  if (act == OR_ACT_SOFTMAX) {
    if (n == 0) return;
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mx = fmaxf(mx, pre[i]);
    float s = -0.0f;
    for (int64_t i = 0; i < n; ++i) {
      out[i] = expf(pre[i] - mx);
      s = s + out[i];
    }
    if (s > 0.0f) {
      for (int64_t i = 0; i < n; ++i) out[i] = out[i] / s;
    } else {
      float u = 1.0f / (float)n;
      for (int64_t i = 0; i < n; ++i) out[i] = u;
    }
    return;
  }
  for (int64_t i = 0; i < n; ++i) {
    float x = pre[i];
    switch (act) {
      case OR_ACT_RELU: out[i] = fmaxf(x, 0.0f); break;
      case OR_ACT_SIGMOID: out[i] = 1.0f / (1.0f + expf(-x)); break;
      case OR_ACT_TANH: out[i] = tanhf(x); break;
      default: out[i] = x; break;
    }
  }
}

/* ======================================================================== */
/* Deja Vu predictor: crates/klearu-dejavu/src/predictor/mlp_predictor.rs     */
/* ======================================================================== */

/* 1 / (1 + exp(-z)) in f32 with glibc expf (mlp_predictor.rs:121). */
float or_sigmoid(float z) {
  float e = expf(-z);
  float d = 1.0f + e;
  return 1.0f / d;
}

/* SparsityPredictor::predict (mlp_predictor.rs:102-124): both layers are
 * iterator sums (sequential f32, product rounded before the add). */
void or_predictor_predict(const float* w1, const float* b1, const float* w2, const float* b2,
                          int in_dim, int hid, int out_dim, const float* x, float* scores,
                          float* hidden) {
  float* h = hidden ? hidden : (float*)malloc(sizeof(float) * (size_t)hid);
  for (int i = 0; i < hid; ++i) {
    float s = -0.0f;
    const float* row = w1 + (int64_t)i * in_dim;
    for (int j = 0; j < in_dim; ++j) {
      float p = row[j] * x[j];
      s = s + p;
    }
    h[i] = fmaxf(s + b1[i], 0.0f);
  }
  for (int o = 0; o < out_dim; ++o) {
    float s = -0.0f;
    const float* row = w2 + (int64_t)o * hid;
    for (int i = 0; i < hid; ++i) {
      float p = row[i] * h[i];
      s = s + p;
    }
    scores[o] = or_sigmoid(s + b2[o]);
  }
  if (!hidden) free(h);
}

/* Same, with BF16-valued weights widened exactly (bits << 16). */
void or_predictor_predict_bf16(const uint16_t* w1, const float* b1, const uint16_t* w2,
                               const float* b2, int in_dim, int hid, int out_dim, const float* x,
                               float* scores, float* hidden) {
  float* h = hidden ? hidden : (float*)malloc(sizeof(float) * (size_t)hid);
  for (int i = 0; i < hid; ++i) {
    float s = -0.0f;
    const uint16_t* row = w1 + (int64_t)i * in_dim;
    for (int j = 0; j < in_dim; ++j) {
      float p = or_bf16_to_f32(row[j]) * x[j];
      s = s + p;
    }
    h[i] = fmaxf(s + b1[i], 0.0f);
  }
  for (int o = 0; o < out_dim; ++o) {
    float s = -0.0f;
    const uint16_t* row = w2 + (int64_t)o * hid;
    for (int i = 0; i < hid; ++i) {
      float p = or_bf16_to_f32(row[i]) * h[i];
      s = s + p;
    }
    scores[o] = or_sigmoid(s + b2[o]);
  }
  if (!hidden) free(h);
}

/* Stable merge sort of indices by score descending (ties keep index order),
 * as `sort_by(|a, b| b.1.partial_cmp(&a.1))` (a stable sort) does at
 * mlp_predictor.rs:127-132.  -0.0 and +0.0 compare equal there and here. */
static void merge_desc(const float* s, int64_t* a, int64_t* tmp, int64_t n) {
  if (n < 2) return;
  int64_t m = n / 2;
  merge_desc(s, a, tmp, m);
  merge_desc(s, a + m, tmp, n - m);
  int64_t i = 0, j = m, o = 0;
  while (i < m && j < n) {
    if (s[a[j]] > s[a[i]]) tmp[o++] = a[j++];
    else tmp[o++] = a[i++];
  }
  while (i < m) tmp[o++] = a[i++];
  while (j < n) tmp[o++] = a[j++];
  memcpy(a, tmp, sizeof(int64_t) * (size_t)n);
}

void or_select_top_k(const float* scores, int64_t n, int64_t k, int64_t* out) {
  int64_t* a = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n + 1));
  int64_t* t = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n + 1));
  for (int64_t i = 0; i < n; ++i) a[i] = i;
  merge_desc(scores, a, t, n);
  int64_t m = k < n ? k : n;
  memcpy(out, a, sizeof(int64_t) * (size_t)m);
  free(a);
  free(t);
}

/* ======================================================================== */
/* klearu-llm sparse decode blocks                                           */
/* ======================================================================== */

/* silu (sparse/sparse_mlp.rs:39-42). */
float or_silu(float x) {
  float e = expf(-x);
  float d = 1.0f + e;
  return x / d;
}

static void widen_row(const uint16_t* w, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_bf16_to_f32(w[i]);
}

/* sparse_mlp::forward_sparse (sparse/sparse_mlp.rs:4-37) with
 * Linear::forward_sparse (model/linear.rs:107-114) = dense_dot_dense_simd per
 * active row.  Weights are BF16 values (the reference widens them to f32 at
 * load, weight/safetensors.rs:150-152; widening is exact).  wg, wu:
 * [inter][hidden]; wd: [hidden][inter] (reference layout).  The down
 * projection is a sequential sum in active-list order starting at +0.0. */
void or_sparse_mlp_forward_bf16(const uint16_t* wg, const uint16_t* wu, const uint16_t* wd,
                                int hidden, int inter, const float* x, const int64_t* active,
                                int64_t k, float* y, float* h_out) {
  float* row = (float*)malloc(sizeof(float) * (size_t)hidden);
  float* h = (float*)malloc(sizeof(float) * (size_t)(k + 1));
  for (int64_t i = 0; i < k; ++i) {
    widen_row(wg + active[i] * hidden, hidden, row);
    float g = or_dense_dot_avx2_order(row, x, hidden);
    widen_row(wu + active[i] * hidden, hidden, row);
    float u = or_dense_dot_avx2_order(row, x, hidden);
    h[i] = or_silu(g) * u;
  }
  for (int j = 0; j < hidden; ++j) {
    const uint16_t* w = wd + (int64_t)j * inter;
    float s = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      float p = or_bf16_to_f32(w[active[i]]) * h[i];
      s = s + p;
    }
    y[j] = s;
  }
  if (h_out) memcpy(h_out, h, sizeof(float) * (size_t)k);
  free(row);
  free(h);
}

/* RmsNorm's scale 1/rms (model/rms_norm.rs:48-52): the sequential f32 sum of
 * the rounded squares from 0.0, then sqrt(sum/n + eps) and its reciprocal. */
float or_rms_inv(const float* x, int64_t n, float eps) {
  float ss = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float p = x[i] * x[i];
    ss = ss + p;
  }
  float rms = sqrtf(ss / (float)n + eps);
  return 1.0f / rms;
}

/* RmsNorm::forward (model/rms_norm.rs:43-64), plain-weight variant. */
void or_rmsnorm(float* x, const float* w, int64_t n, float eps) {
  float inv = or_rms_inv(x, n, eps);
  for (int64_t i = 0; i < n; ++i) {
    float t = x[i] * inv;
    x[i] = t * w[i];
  }
}

/* RotaryEmbedding::new_partial with rotary_dim == head_dim (model/rope.rs:17-46):
 * freq = 1 / theta^(2i/d), angle = pos*freq, tables [max_seq][d/2]. */
void or_rope_tables(int head_dim, int max_seq, float theta, float* cos_t, float* sin_t) {
  int half = head_dim / 2;
  for (int p = 0; p < max_seq; ++p)
    for (int i = 0; i < half; ++i) {
      float e = (2.0f * (float)i) / (float)head_dim;
      float freq = 1.0f / powf(theta, e);
      float ang = (float)p * freq;
      cos_t[(int64_t)p * half + i] = cosf(ang);
      sin_t[(int64_t)p * half + i] = sinf(ang);
    }
}

/* RotaryEmbedding::apply (model/rope.rs:75-87): NeoX half-split rotation. */
void or_rope_apply(float* x, int half, const float* cos_t, const float* sin_t, int64_t pos) {
  for (int i = 0; i < half; ++i) {
    float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
    float x0 = x[i], x1 = x[half + i];
    float a = x0 * c, b = x1 * s;
    float e = x1 * c, f = x0 * s;
    x[i] = a - b;
    x[half + i] = e + f;
  }
}

/* Linear::forward (model/linear.rs:79-104): one AVX2-order dot per row. */
void or_linear_forward_bf16(const uint16_t* w, int out_f, int in_f, const float* x, float* y) {
  float* row = (float*)malloc(sizeof(float) * (size_t)in_f);
  for (int o = 0; o < out_f; ++o) {
    widen_row(w + (int64_t)o * in_f, in_f, row);
    y[o] = or_dense_dot_avx2_order(row, x, in_f);
  }
  free(row);
}

/* sparse_attention::forward_sparse (sparse/sparse_attention.rs:7-79) with
 * softmax_inplace (:81-95) and KvCache::append (model/kv_cache.rs:33-48).
 * Caches are [num_kv_heads][max_seq][head_dim] f32 holding pos valid rows on
 * entry; this call appends row pos.  Weights are BF16 values in the reference
 * [out][in] layout. */
void or_sparse_attention_forward_bf16(const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                                      const uint16_t* wo, int hidden, int num_heads,
                                      int num_kv_heads, int head_dim, const float* x, int64_t pos,
                                      const float* cos_t, const float* sin_t, float* k_cache,
                                      float* v_cache, int64_t max_seq, const int64_t* heads,
                                      int64_t n_heads, float* out) {
  const int group = num_heads / num_kv_heads;
  const int qd = num_heads * head_dim, kvd = num_kv_heads * head_dim;
  const int half = head_dim / 2;
  float* q = (float*)malloc(sizeof(float) * (size_t)qd);
  float* kk = (float*)malloc(sizeof(float) * (size_t)kvd);
  float* vv = (float*)malloc(sizeof(float) * (size_t)kvd);
  or_linear_forward_bf16(wq, qd, hidden, x, q);
  or_linear_forward_bf16(wk, kvd, hidden, x, kk);
  or_linear_forward_bf16(wv, kvd, hidden, x, vv);
  for (int h = 0; h < num_heads; ++h) or_rope_apply(q + h * head_dim, half, cos_t, sin_t, pos);
  for (int h = 0; h < num_kv_heads; ++h) or_rope_apply(kk + h * head_dim, half, cos_t, sin_t, pos);
  for (int h = 0; h < num_kv_heads; ++h) {
    memcpy(k_cache + ((int64_t)h * max_seq + pos) * head_dim, kk + h * head_dim,
           sizeof(float) * (size_t)head_dim);
    memcpy(v_cache + ((int64_t)h * max_seq + pos) * head_dim, vv + h * head_dim,
           sizeof(float) * (size_t)head_dim);
  }
  const int64_t seq = pos + 1;
  const float inv_sqrt = 1.0f / sqrtf((float)head_dim);
  float* concat = (float*)calloc((size_t)qd, sizeof(float));
  float* sc = (float*)malloc(sizeof(float) * (size_t)seq);
  for (int64_t a = 0; a < n_heads; ++a) {
    int64_t h = heads[a];
    if (h >= num_heads) continue;
    int64_t kvh = h / group;
    const float* qh = q + h * head_dim;
    for (int64_t j = 0; j < seq; ++j)
      sc[j] = or_dense_dot_avx2_order(qh, k_cache + (kvh * max_seq + j) * head_dim, head_dim) *
              inv_sqrt;
    float mx = -INFINITY;
    for (int64_t j = 0; j < seq; ++j) mx = fmaxf(mx, sc[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j < seq; ++j) {
      sc[j] = expf(sc[j] - mx);
      sum = sum + sc[j];
    }
    float inv = 1.0f / sum;
    for (int64_t j = 0; j < seq; ++j) sc[j] = sc[j] * inv;
    float* ho = concat + h * head_dim;
    for (int64_t j = 0; j < seq; ++j) {
      const float* vj = v_cache + (kvh * max_seq + j) * head_dim;
      for (int d = 0; d < head_dim; ++d) {
        float p = sc[j] * vj[d];
        ho[d] = ho[d] + p;
      }
    }
  }
  or_linear_forward_bf16(wo, hidden, qd, concat, out);
  free(q); free(kk); free(vv); free(concat); free(sc);
}

/* ======================================================================== */
/* klearu-dejavu toy layer (f32 weights with bias)                           */
/* ======================================================================== */

/* dejavu Linear::forward_sparse (klearu-dejavu/src/transformer/mod.rs:126-134). */
void or_dejavu_linear_forward_sparse(const float* w, const float* bias, int in_f,
                                     const float* x, const int64_t* idx, int64_t n, float* out) {
  for (int64_t a = 0; a < n; ++a) {
    const float* row = w + idx[a] * in_f;
    float s = -0.0f;
    for (int j = 0; j < in_f; ++j) {
      float p = row[j] * x[j];
      s = s + p;
    }
    out[a] = s + bias[idx[a]];
  }
}

/* dejavu Linear::forward (klearu-dejavu/src/transformer/mod.rs:114-123): every
 * row, a sequential sum from -0.0 of the rounded products, plus the bias.
 * Pinned: float64 bound and equality with forward_sparse over every row
 * (tests/test_oracle_dejavu.py). */
void or_dejavu_linear_forward(const float* w, const float* bias, int in_f, int out_f,
                              const float* x, float* out) {
  for (int r = 0; r < out_f; ++r) {
    const float* row = w + (int64_t)r * in_f;
    float s = -0.0f;
    for (int j = 0; j < in_f; ++j) {
      float p = row[j] * x[j];
      s = s + p;
    }
    out[r] = s + bias[r];
  }
}

/* SparseAttention::forward (klearu-dejavu/src/attention.rs:18-74): q/k/v rows
 * of the selected heads only (zeros elsewhere), per selected head the score
 * sigmoid(dot(q_h, k_h) / sqrt(head_dim)) scales v_h, then o_proj runs dense
 * over the whole concatenation.  Heads are taken in list order; a repeated
 * head recomputes the same values.
 * Pinned: all heads selected equals the reference's dense restatement
 * (attention.rs:119-160) and a float64 bound (tests/test_oracle_dejavu.py). */
void or_dejavu_sparse_attention_forward(const float* wq, const float* bq, const float* wk,
                                        const float* bk, const float* wv, const float* bv,
                                        const float* wo, const float* bo, int hidden,
                                        int num_heads, int head_dim, const float* x,
                                        const int64_t* heads, int64_t n_heads, float* y) {
  const int64_t qd = (int64_t)num_heads * head_dim;
  float* q = (float*)calloc((size_t)qd, sizeof(float));
  float* k = (float*)calloc((size_t)qd, sizeof(float));
  float* v = (float*)calloc((size_t)qd, sizeof(float));
  float* att = (float*)calloc((size_t)qd, sizeof(float));
  int64_t* idx = (int64_t*)malloc(sizeof(int64_t) * (size_t)head_dim);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
  for (int64_t a = 0; a < n_heads; ++a) {
    const int64_t st = heads[a] * head_dim;
    for (int d = 0; d < head_dim; ++d) idx[d] = st + d;
    or_dejavu_linear_forward_sparse(wq, bq, hidden, x, idx, head_dim, tmp);
    for (int d = 0; d < head_dim; ++d) q[st + d] = tmp[d];
    or_dejavu_linear_forward_sparse(wk, bk, hidden, x, idx, head_dim, tmp);
    for (int d = 0; d < head_dim; ++d) k[st + d] = tmp[d];
    or_dejavu_linear_forward_sparse(wv, bv, hidden, x, idx, head_dim, tmp);
    for (int d = 0; d < head_dim; ++d) v[st + d] = tmp[d];
  }
  const float scale = sqrtf((float)head_dim);
  for (int64_t a = 0; a < n_heads; ++a) {
    const int64_t st = heads[a] * head_dim;
    float s = -0.0f;
    for (int d = 0; d < head_dim; ++d) {
      float p = q[st + d] * k[st + d];
      s = s + p;
    }
    s = s / scale;
    float e = expf(-s);
    float den = 1.0f + e;
    float sc = 1.0f / den;
    for (int d = 0; d < head_dim; ++d) att[st + d] = v[st + d] * sc;
  }
  or_dejavu_linear_forward(wo, bo, (int)qd, hidden, att, y);
  free(q); free(k); free(v); free(att); free(idx); free(tmp);
}

/* SparseMlp::forward (klearu-dejavu/src/mlp.rs:23-58): SwiGLU over selected
 * neurons; the down projection adds column idx of wd [hidden][inter] times the
 * activation into every output, in selection order, then adds the bias. */
void or_dejavu_sparse_mlp_forward(const float* wg, const float* bg, const float* wu,
                                  const float* bu, const float* wd, const float* bd, int hidden,
                                  int inter, const float* x, const int64_t* sel, int64_t n,
                                  float* y) {
  float* g = (float*)malloc(sizeof(float) * (size_t)(n + 1));
  float* u = (float*)malloc(sizeof(float) * (size_t)(n + 1));
  float* sh = (float*)calloc((size_t)inter, sizeof(float));
  or_dejavu_linear_forward_sparse(wg, bg, hidden, x, sel, n, g);
  or_dejavu_linear_forward_sparse(wu, bu, hidden, x, sel, n, u);
  for (int64_t a = 0; a < n; ++a) {
    float e = expf(-g[a]);
    float d = 1.0f + e;
    float si = g[a] / d;
    sh[sel[a]] = si * u[a];
  }
  for (int j = 0; j < hidden; ++j) y[j] = 0.0f;
  for (int64_t a = 0; a < n; ++a) {
    float v = sh[sel[a]];
    if (v != 0.0f)
      for (int j = 0; j < hidden; ++j) {
        float p = wd[(int64_t)j * inter + sel[a]] * v;
        y[j] = y[j] + p;
      }
  }
  for (int j = 0; j < hidden; ++j) y[j] = y[j] + bd[j];
  free(g); free(u); free(sh);
}

/* ======================================================================== */
/* SLIDE Layer::forward for one dense input (network/layer.rs:65-120)        */
/* ======================================================================== */

static int cmp_u32_asc(const void* a, const void* b) { return cmp_u32(a, b); }

/* Query (lsh/index.rs:282-284) -> sampling (layer.rs:78; sampling 0 vanilla,
 * 1 top-k, 2 threshold) -> empty set falls back to every neuron (:82-84) ->
 * ids < n (:87) -> Neuron::forward per active id (:90-93) -> activation
 * (:96-107).  Active ids are returned ascending (the reference's order is
 * HashMap order for vanilla/threshold).  Returns the number of active ids;
 * out arrays need max(n, L*cap) entries. */
static int64_t slide_forward_impl(const int8_t* planes, int dim, int k, int num_tables, int cap,
                                  const uint32_t* data, const uint32_t* len, const float* W,
                                  const float* bias, int n, const float* x, int sampling,
                                  int top_k, int threshold, int act, uint32_t* out_ids,
                                  float* out_pre, float* out_act, int sampler_order) {
  uint32_t* codes = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)num_tables);
  or_hash_dense_batch(planes, dim, k, num_tables, x, 1, codes);
  const int64_t m = (int64_t)num_tables * cap + 1;
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  uint32_t* cnt = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  int64_t u = or_lsh_query(num_tables, k, cap, data, len, codes, ids, cnt);
  int64_t a = 0;
  if (sampling == 1) {
    a = or_sample_topk(ids, cnt, u, top_k, out_ids);
  } else if (sampling == 2) {
    a = or_sample_threshold(ids, cnt, u, (uint32_t)threshold, out_ids);
  } else {
    memcpy(out_ids, ids, sizeof(uint32_t) * (size_t)u);
    a = u;
  }
  if (a == 0) {
    for (int i = 0; i < n; ++i) out_ids[i] = (uint32_t)i;
    a = n;
  }
  int64_t r = 0;
  for (int64_t i = 0; i < a; ++i)
    if (out_ids[i] < (uint32_t)n) out_ids[r++] = out_ids[i];
  a = r;
  if (!sampler_order) qsort(out_ids, (size_t)a, sizeof(uint32_t), cmp_u32_asc);
  for (int64_t i = 0; i < a; ++i)
    out_pre[i] = or_neuron_forward(W + (int64_t)out_ids[i] * dim, bias[out_ids[i]], x, dim);
  or_layer_activate(out_pre, a, act, out_act);
  free(codes);
  free(ids);
  free(cnt);
  return a;
}

int64_t or_slide_forward(const int8_t* planes, int dim, int k, int num_tables, int cap,
                         const uint32_t* data, const uint32_t* len, const float* W,
                         const float* bias, int n, const float* x, int sampling, int top_k,
                         int threshold, int act, uint32_t* out_ids, float* out_pre,
                         float* out_act) {
  return slide_forward_impl(planes, dim, k, num_tables, cap, data, len, W, bias, n, x, sampling,
                            top_k, threshold, act, out_ids, out_pre, out_act, 0);
}

/* Layer::forward with the active list in the sampler's order, which the
 * backward pass's sums follow: TopKSampling::select sorts by count descending,
 * then id (sampling/topk.rs:19-34); the query's candidates come in ascending id
 * order here (or_lsh_query), which vanilla and threshold sampling keep (the
 * reference's HashMap order is not reproducible: its RandomState differs
 * from run to run).  The softmax sum (layer.rs:298) follows the same order.
 * Pinned: the count-order KAT in tests/test_oracle_train.py. */
int64_t or_slide_forward_ordered(const int8_t* planes, int dim, int k, int num_tables, int cap,
                                 const uint32_t* data, const uint32_t* len, const float* W,
                                 const float* bias, int n, const float* x, int sampling,
                                 int top_k, int threshold, int act, uint32_t* out_ids,
                                 float* out_pre, float* out_act) {
  return slide_forward_impl(planes, dim, k, num_tables, cap, data, len, W, bias, n, x, sampling,
                            top_k, threshold, act, out_ids, out_pre, out_act, 1);
}

/* ======================================================================== */
/* SLIDE training: network/layer.rs:124-226, network/net.rs:176-230, optim/   */
/* ======================================================================== */

/* f32::powi: llvm.powi with a run-time exponent is the __powisf2 libcall of
 * Rust's compiler-builtins (src/float/pow.rs): square-and-multiply in f32 from
 * the low exponent bit up, reciprocal for negative exponents.
 * Pinned: closed forms (b^0 = 1, b^1 = b, b^2 = b*b, b^4 = (b*b)*(b*b),
 * b^3 = b*(b*b)) in tests/test_oracle_train.py. */
float or_powi_f32(float a, int32_t b) {
  const int recip = b < 0;
  uint32_t p = recip ? 0u - (uint32_t)b : (uint32_t)b;
  float mul = 1.0f;
  for (;;) {
    if (p & 1u) mul = mul * a;
    p >>= 1;
    if (p == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / mul : mul;
}

/* Sgd::update (optim/sgd.rs:18-57): lr rounded to f32; with momentum
 * v = momentum*m - lr*g, m = v, w += v; without, w -= lr*g.  mw/mb are
 * ignored when momentum <= 0.
 * Pinned: the reference's own expected values (sgd.rs:77-117) in
 * tests/test_oracle_train.py. */
void or_sgd_update(float* w, const float* gw, int64_t n, float* bias, float gb, double lr_d,
                   float momentum, float* mw, float* mb) {
  const float lr = (float)lr_d;
  if (momentum > 0.0f) {
    for (int64_t i = 0; i < n; ++i) {
      float a = momentum * mw[i];
      float b = lr * gw[i];
      float v = a - b;
      mw[i] = v;
      w[i] = w[i] + v;
    }
    float a = momentum * *mb;
    float b = lr * gb;
    float vb = a - b;
    *mb = vb;
    *bias = *bias + vb;
  } else {
    for (int64_t i = 0; i < n; ++i) {
      float b = lr * gw[i];
      w[i] = w[i] - b;
    }
    float b = lr * gb;
    *bias = *bias - b;
  }
}

/* Adam::update (optim/adam.rs:28-77): corrections 1 - beta^step with
 * f32::powi (or_powi_f32; step 0 counts as 1, `step as i32` wraps), then per
 * weight m = b1*m + (1-b1)*g, v = b2*v + ((1-b2)*g)*g,
 * w -= (lr*(m/c1)) / (sqrt(v/c2) + eps); the bias likewise.
 * Pinned: hand-computed first steps (m = (1-b1) g, v = (1-b2) g^2) and the
 * reference's sign / zero-gradient tests (adam.rs:131-254) in
 * tests/test_oracle_train.py. */
static float adam_one(float w, float g, float* m, float* v, float lr, float b1, float b2,
                      float eps, float c1, float c2) {
  float a = b1 * *m;
  float b = (1.0f - b1) * g;
  *m = a + b;
  float c = b2 * *v;
  float d = (1.0f - b2) * g;
  d = d * g;
  *v = c + d;
  float mh = *m / c1;
  float vh = *v / c2;
  float num = lr * mh;
  float den = sqrtf(vh) + eps;
  return w - num / den;
}

void or_adam_update(float* w, const float* gw, int64_t n, float* bias, float gb, double lr_d,
                    uint64_t step, float beta1, float beta2, float eps, float* m_w, float* v_w,
                    float* m_b, float* v_b) {
  const float lr = (float)lr_d;
  const uint64_t st = step < 1 ? 1 : step;
  const int32_t si = (int32_t)(uint32_t)st;
  const float c1 = 1.0f - or_powi_f32(beta1, si);
  const float c2 = 1.0f - or_powi_f32(beta2, si);
  for (int64_t i = 0; i < n; ++i) w[i] = adam_one(w[i], gw[i], m_w + i, v_w + i, lr, beta1, beta2, eps, c1, c2);
  *bias = adam_one(*bias, gb, m_b, v_b, lr, beta1, beta2, eps, c1, c2);
}

/* activation_derivative (layer.rs:266-283). */
float or_activation_derivative(float pre, float post, int act) {
  switch (act) {
    case OR_ACT_RELU: return pre > 0.0f ? 1.0f : 0.0f;
    case OR_ACT_SIGMOID: return post * (1.0f - post);
    case OR_ACT_TANH: return 1.0f - post * post;
    default: return 1.0f;
  }
}

/* The softmax branch of Layer::backward (layer.rs:141-175): for each i, a
 * sequential sum from +0.0 over j of go_j*s_j*(1-s_j) (i == j) or
 * go_j*(-s_i*s_j), each product rounded left to right.
 * Pinned: a cancellation KAT only the sequential order reproduces and the
 * identity sum_j J_ij go_j = s_i (go_i - sum_j s_j go_j) within rounding, in
 * tests/test_oracle_train.py. */
void or_softmax_local_grads(const float* s, const float* go, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    float r = 0.0f;
    for (int64_t j = 0; j < n; ++j) {
      float t;
      if (i == j) {
        t = go[j] * s[j];
        t = t * (1.0f - s[j]);
      } else {
        float q = -s[i] * s[j];
        t = go[j] * q;
      }
      r = r + t;
    }
    out[i] = r;
  }
}

/* compute_loss (net.rs:180-201): -ln(max(p, 1e-7)) per label (1e-7 when the
 * label is not active), summed in label order, divided by the label count.
 * Pinned: the reference's expected values (net.rs:404-465). */
float or_compute_loss(const float* act_dense, const uint32_t* active, int64_t n_act,
                      const uint32_t* labels, int64_t n_labels) {
  if (n_labels == 0) return 0.0f;
  const float eps = 1e-7f;
  float loss = 0.0f;
  for (int64_t l = 0; l < n_labels; ++l) {
    int found = 0;
    for (int64_t a = 0; a < n_act; ++a)
      if (active[a] == labels[l]) { found = 1; break; }
    float prob = found ? fmaxf(act_dense[labels[l]], eps) : eps;
    loss = loss - logf(prob);
  }
  return loss / (float)n_labels;
}

/* compute_loss_gradient (net.rs:205-230): grad = activations at active ids,
 * then 1/|labels| subtracted once per label occurrence; all zero without labels.
 * Pinned: the reference's expected values (net.rs:479-494). */
void or_compute_loss_gradient(const float* act_dense, const uint32_t* active, int64_t n_act,
                              const uint32_t* labels, int64_t n_labels, int64_t num_output,
                              float* grad) {
  for (int64_t i = 0; i < num_output; ++i) grad[i] = 0.0f;
  if (n_labels == 0) return;
  for (int64_t a = 0; a < n_act; ++a)
    if ((int64_t)active[a] < num_output) grad[active[a]] = act_dense[active[a]];
  const float w = 1.0f / (float)n_labels;
  for (int64_t l = 0; l < n_labels; ++l)
    if ((int64_t)labels[l] < num_output) grad[labels[l]] = grad[labels[l]] - w;
}

/* Layer::backward (layer.rs:124-226) for one sample: local gradients (softmax
 * Jacobian or go * activation_derivative), then per active neuron in list
 * order grad_in[j] += lg * w[j] (weights before the update; sequential from
 * +0.0) and the optimizer update with grad_weights[j] = lg * input[j] and
 * grad_bias = lg.  opt 0: SGD (st_w1/st_b1 = momentum buffers), 1: Adam
 * (st_w1/st_b1 = first moments, st_w2/st_b2 = second).  grad_in may be NULL.
 * Pinned: the pieces above, and a cancellation KAT for the grad_in order in
 * tests/test_oracle_train.py. */
void or_layer_backward(float* W, float* bias, int dim, int n, int act, const float* input,
                       const uint32_t* active, int64_t n_act, const float* pre,
                       const float* act_dense, const float* grad_out, int64_t grad_out_len,
                       int opt, float momentum, float beta1, float beta2, float eps,
                       float* st_w1, float* st_w2, float* st_b1, float* st_b2, double lr,
                       uint64_t step, float* grad_in) {
  if (grad_in)
    for (int j = 0; j < dim; ++j) grad_in[j] = 0.0f;
  if (n_act == 0) return;
  float* lg = (float*)malloc(sizeof(float) * (size_t)n_act);
  if (act == OR_ACT_SOFTMAX) {
    float* sm = (float*)malloc(sizeof(float) * (size_t)n_act);
    float* go = (float*)malloc(sizeof(float) * (size_t)n_act);
    or_layer_activate(pre, n_act, OR_ACT_SOFTMAX, sm);
    for (int64_t a = 0; a < n_act; ++a)
      go[a] = (int64_t)active[a] < grad_out_len ? grad_out[active[a]] : 0.0f;
    or_softmax_local_grads(sm, go, n_act, lg);
    free(sm);
    free(go);
  } else {
    for (int64_t a = 0; a < n_act; ++a) {
      const uint32_t id = active[a];
      const float go = (int64_t)id < grad_out_len ? grad_out[id] : 0.0f;
      lg[a] = go * or_activation_derivative(pre[a], act_dense[id], act);
    }
  }
  float* gw = (float*)malloc(sizeof(float) * (size_t)dim);
  for (int64_t a = 0; a < n_act; ++a) {
    const int64_t id = active[a];
    float* w = W + id * dim;
    for (int j = 0; j < dim; ++j) gw[j] = lg[a] * input[j];
    if (grad_in)
      for (int j = 0; j < dim; ++j) {
        float p = lg[a] * w[j];
        grad_in[j] = grad_in[j] + p;
      }
    (void)n;
    if (opt == 1)
      or_adam_update(w, gw, dim, bias + id, lg[a], lr, step, beta1, beta2, eps, st_w1 + id * dim,
                     st_w2 + id * dim, st_b1 + id, st_b2 + id);
    else
      or_sgd_update(w, gw, dim, bias + id, lg[a], lr, momentum, st_w1 + id * dim, st_b1 + id);
  }
  free(gw);
  free(lg);
}

/* ======================================================================== */
/* CPU baseline drivers (bench.py's cpu legs).  One call runs a whole batch, */
/* so a timed call holds no per-row interpreter overhead.  Each is a loop   */
/* over the pinned functions above; tests/test_oracle_families.py checks    */
/* them against those functions row by row.                                 */
/* ======================================================================== */

/* The compiler that built this library (recorded with the CPU timings). */
const char* or_compiler_version(void) { return __VERSION__; }

/* codes[r*num_tables + t] for rows X[rows][dim]: kind 0 WTA / DWTA on dense
 * rows (dwta.rs:143-152 hashes a dense row as WTA does, wta.rs:83-118), kind 2
 * MinHash over the row's nonzero dimensions (minhash.rs:55-103). */
void or_cpu_rank_hash_batch(int kind, const uint32_t* tabs, int dim, int k, int ws, int num_tables,
                            const float* X, int64_t rows, uint64_t* codes) {
  uint32_t* nz = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(dim > 0 ? dim : 1));
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = X + r * dim;
    if (kind == 2) {
      int64_t m = 0;
      for (int d = 0; d < dim; ++d)
        if (x[d] != 0.0f) nz[m++] = (uint32_t)d;
      for (int t = 0; t < num_tables; ++t) codes[r * num_tables + t] = or_minhash_hash(tabs, dim, k, t, nz, m);
    } else {
      for (int t = 0; t < num_tables; ++t) codes[r * num_tables + t] = or_wta_hash_dense(tabs, k, ws, t, x);
    }
  }
  free(nz);
}

/* SparseInferenceEngine::infer over rows (klearu-bolt/src/sparse_inference.rs:36-74):
 * hash, query, the top_k candidates by (count desc, id asc), dot + bias
 * (+ ReLU when relu); no fallback to all neurons.  Returns the total number of
 * outputs; out_n[r] holds each row's count, out_act the activations row after
 * row (room for rows * top_k). */
int64_t or_cpu_bolt_batch(const int8_t* planes, int dim, int k, int num_tables, int cap,
                          const uint32_t* data, const uint32_t* len, const float* W, const float* bias,
                          const float* X, int64_t rows, int top_k, int relu, int64_t* out_n,
                          float* out_act) {
  uint32_t* codes = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)num_tables);
  const int64_t m = (int64_t)num_tables * cap + 1;
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  uint32_t* cnt = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  uint32_t* sel = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  int64_t tot = 0;
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = X + r * dim;
    or_hash_dense_batch(planes, dim, k, num_tables, x, 1, codes);
    const int64_t u = or_lsh_query(num_tables, k, cap, data, len, codes, ids, cnt);
    const int64_t a = or_sample_topk(ids, cnt, u, top_k, sel);
    for (int64_t i = 0; i < a; ++i) {
      const float z = or_neuron_forward(W + (int64_t)sel[i] * dim, bias[sel[i]], x, dim);
      out_act[tot + i] = relu ? (z > 0.0f ? z : 0.0f) : z;
    }
    out_n[r] = a;
    tot += a;
  }
  free(codes);
  free(ids);
  free(cnt);
  free(sel);
  return tot;
}

/* LshSparsityPredictor::predict over rows (klearu-dejavu/src/predictor/lsh_predictor.rs:15-43):
 * hash, query with counts, the top_k ids by (count desc, id asc), written to
 * out_ids[r*top_k ...] with out_n[r] of them. */
void or_cpu_lsh_topk_batch(const int8_t* planes, int dim, int k, int num_tables, int cap,
                           const uint32_t* data, const uint32_t* len, const float* X, int64_t rows,
                           int top_k, int64_t* out_n, uint32_t* out_ids) {
  uint32_t* codes = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)num_tables);
  const int64_t m = (int64_t)num_tables * cap + 1;
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  uint32_t* cnt = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  uint32_t* sel = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)m);
  for (int64_t r = 0; r < rows; ++r) {
    or_hash_dense_batch(planes, dim, k, num_tables, X + r * dim, 1, codes);
    const int64_t u = or_lsh_query(num_tables, k, cap, data, len, codes, ids, cnt);
    const int64_t a = or_sample_topk(ids, cnt, u, top_k, sel);
    for (int64_t i = 0; i < a; ++i) out_ids[r * top_k + i] = sel[i];
    out_n[r] = a;
  }
  free(codes);
  free(ids);
  free(cnt);
  free(sel);
}
