/*
 * oracle_avx2.c -- AVX2/FMA restatement of klearu-accel's x86_64 kernels and the
 * timed CPU port of the reference's sparse decode path (bench.py cpu_baseline).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with
 *   gcc -O3 -mavx2 -mfma -ffp-contract=off
 * so that the only fused operations are the explicit _mm256_fmadd_ps the
 * reference issues.  tests/test_oracle_accel.py checks that these produce the
 * same bits as the portable emulation in oracle.c.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* hsum_avx2 (crates/klearu-accel/src/simd/mod.rs:128-141). */
static inline float hsum_avx2(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 s = _mm_add_ps(lo, hi);
  __m128 sh = _mm_movehdup_ps(s);
  __m128 sums = _mm_add_ps(s, sh);
  __m128 sh2 = _mm_movehl_ps(sums, sums);
  return _mm_cvtss_f32(_mm_add_ss(sums, sh2));
}

/* dense_dot_dense_avx2 (simd/mod.rs:174-207). */
float or_avx2_dense_dot(const float* a, const float* b, int64_t n) {
  int64_t chunks = n / 16;
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t o = c * 16;
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o), _mm256_loadu_ps(b + o), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 8), _mm256_loadu_ps(b + o + 8), acc1);
  }
  int64_t rs = chunks * 16;
  int extra = (rs + 8 <= n);
  if (extra) acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + rs), _mm256_loadu_ps(b + rs), acc0);
  float sum = hsum_avx2(_mm256_add_ps(acc0, acc1));
  for (int64_t i = extra ? rs + 8 : rs; i < n; ++i) {
    float p = a[i] * b[i];
    sum = sum + p;
  }
  return sum;
}

/* sparse_dot_dense_avx2 (simd/mod.rs:145-170). */
float or_avx2_sparse_dot_dense(const uint32_t* idx, const float* val, int64_t nnz,
                               const float* dense) {
  int64_t chunks = nnz / 8;
  __m256 acc = _mm256_setzero_ps();
  for (int64_t c = 0; c < chunks; ++c) {
    __m256i ix = _mm256_loadu_si256((const __m256i*)(idx + c * 8));
    __m256 g = _mm256_i32gather_ps(dense, ix, 4);
    acc = _mm256_fmadd_ps(_mm256_loadu_ps(val + c * 8), g, acc);
  }
  float sum = hsum_avx2(acc);
  for (int64_t i = chunks * 8; i < nnz; ++i) {
    float p = val[i] * dense[idx[i]];
    sum = sum + p;
  }
  return sum;
}

/*
 * One token of the reference's Deja Vu FFN block for one layer, as
 * SparseModel::forward_decode_sparse runs it (crates/klearu-llm/src/sparse/mod.rs:115-142):
 *   norm = RmsNorm(hidden) (model/rms_norm.rs:43-64, weight w_norm)
 *   active = predictor.select_top_k(norm, k) (klearu-dejavu/.../mlp_predictor.rs:102-132)
 *   y = sparse_mlp::forward_sparse(norm, active) (sparse/sparse_mlp.rs:4-37)
 *   hidden += y
 * Weights are f32 (the reference's in-memory type), gate/up [inter][hidden],
 * down [hidden][inter].  The predictor is sequential scalar code, the gate/up
 * dots are AVX2 (Linear::forward_sparse, model/linear.rs:107-114), the down
 * projection is the sequential gather of sparse_mlp.rs:27-34.
 */
void or_cpu_dejavu_ffn_layer(const float* wg, const float* wu, const float* wd,
                             const float* w_norm, float eps, const float* pw1, const float* pb1,
                             const float* pw2, const float* pb2, int hid_p, int hidden, int inter,
                             int64_t k, float* hstate, float* scratch, int64_t* active_out) {
  float* norm = scratch;                  /* hidden */
  float* scores = norm + hidden;          /* inter */
  float* ph = scores + inter;             /* hid_p */
  float* hv = ph + hid_p;                 /* k */
  float* y = hv + k;                      /* hidden */
  memcpy(norm, hstate, sizeof(float) * (size_t)hidden);
  or_rmsnorm(norm, w_norm, hidden, eps);
  or_predictor_predict(pw1, pb1, pw2, pb2, hidden, hid_p, inter, norm, scores, ph);
  or_select_top_k(scores, inter, k, active_out);
  for (int64_t i = 0; i < k; ++i) {
    float g = or_avx2_dense_dot(wg + active_out[i] * hidden, norm, hidden);
    float u = or_avx2_dense_dot(wu + active_out[i] * hidden, norm, hidden);
    hv[i] = or_silu(g) * u;
  }
  for (int j = 0; j < hidden; ++j) {
    const float* w = wd + (int64_t)j * inter;
    float s = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      float p = w[active_out[i]] * hv[i];
      s = s + p;
    }
    y[j] = s;
  }
  for (int j = 0; j < hidden; ++j) hstate[j] = hstate[j] + y[j];
}

/* Linear::forward (model/linear.rs:79-104): one AVX2 dot per output row. */
static void avx2_linear(const float* w, int out_f, int in_f, const float* x, float* y) {
  for (int o = 0; o < out_f; ++o) y[o] = or_avx2_dense_dot(w + (int64_t)o * in_f, x, in_f);
}

/*
 * One token of the reference's head-sparse attention block for one layer
 * (crates/klearu-llm/src/sparse/mod.rs:76-113 decode path):
 *   norm = RmsNorm(hidden); heads = predictor.select_top_k(norm, k)
 *   out = sparse_attention::forward_sparse(norm, pos, heads) (sparse_attention.rs:7-79)
 *   hidden += out
 * f32 weights wq[nh*d][H], wk/wv[nkv*d][H], wo[H][nh*d]; caches [nkv][max_seq][d]
 * with pos valid rows (row pos is written).  Projections use the AVX2 dot, the
 * rest is the reference's sequential scalar code.  scratch: 2*H + nh*d*2 + 2*nkv*d
 * + n_out + hid_p + max_seq floats.
 */
void or_cpu_sparse_attention_layer(const float* wq, const float* wk, const float* wv,
                                   const float* wo, const float* w_norm, float eps,
                                   const float* pw1, const float* pb1, const float* pw2,
                                   const float* pb2, int hid_p, int hidden, int nh, int nkv,
                                   int d, int64_t k, const float* cos_t, const float* sin_t,
                                   float* k_cache, float* v_cache, int64_t max_seq, int64_t pos,
                                   float* hstate, float* scratch, int64_t* heads_out) {
  const int qd = nh * d, kvd = nkv * d, half = d / 2, group = nh / nkv;
  float* norm = scratch;
  float* q = norm + hidden;
  float* kk = q + qd;
  float* vv = kk + kvd;
  float* concat = vv + kvd;
  float* out = concat + qd;
  float* scores = out + hidden;
  float* ph = scores + nh;
  float* sc = ph + hid_p;
  memcpy(norm, hstate, sizeof(float) * (size_t)hidden);
  or_rmsnorm(norm, w_norm, hidden, eps);
  or_predictor_predict(pw1, pb1, pw2, pb2, hidden, hid_p, nh, norm, scores, ph);
  or_select_top_k(scores, nh, k, heads_out);
  avx2_linear(wq, qd, hidden, norm, q);
  avx2_linear(wk, kvd, hidden, norm, kk);
  avx2_linear(wv, kvd, hidden, norm, vv);
  for (int h = 0; h < nh; ++h) or_rope_apply(q + h * d, half, cos_t, sin_t, pos);
  for (int h = 0; h < nkv; ++h) or_rope_apply(kk + h * d, half, cos_t, sin_t, pos);
  for (int h = 0; h < nkv; ++h) {
    memcpy(k_cache + ((int64_t)h * max_seq + pos) * d, kk + h * d, sizeof(float) * (size_t)d);
    memcpy(v_cache + ((int64_t)h * max_seq + pos) * d, vv + h * d, sizeof(float) * (size_t)d);
  }
  const int64_t seq = pos + 1;
  const float inv_sqrt = 1.0f / sqrtf((float)d);
  memset(concat, 0, sizeof(float) * (size_t)qd);
  for (int64_t a = 0; a < k && a < nh; ++a) {
    const int64_t h = heads_out[a];
    const int64_t kvh = h / group;
    const float* qh = q + h * d;
    for (int64_t j = 0; j < seq; ++j)
      sc[j] = or_avx2_dense_dot(qh, k_cache + (kvh * max_seq + j) * d, d) * inv_sqrt;
    float mx = -INFINITY;
    for (int64_t j = 0; j < seq; ++j) mx = fmaxf(mx, sc[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j < seq; ++j) {
      sc[j] = expf(sc[j] - mx);
      sum = sum + sc[j];
    }
    const float inv = 1.0f / sum;
    for (int64_t j = 0; j < seq; ++j) sc[j] = sc[j] * inv;
    float* ho = concat + h * d;
    for (int64_t j = 0; j < seq; ++j) {
      const float* vj = v_cache + (kvh * max_seq + j) * d;
      for (int e = 0; e < d; ++e) {
        float p = sc[j] * vj[e];
        ho[e] = ho[e] + p;
      }
    }
  }
  avx2_linear(wo, hidden, qd, concat, out);
  for (int j = 0; j < hidden; ++j) hstate[j] = hstate[j] + out[j];
}
