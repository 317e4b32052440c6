/*
 * oracle.h -- CPU restatement of klearu's activation-sparse inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for the baseline, as the timed CPU port of the reference).  The product
 * path (klearu_amd/, libklearu_hip.so) never links or calls it.
 *
 * Every function restates the arithmetic of a reference function, in the same
 * operation order, and cites it as path:line relative to the reference tree
 * (QuilibriumNetwork/klearu, crates/...).  The reference is Rust; Rust never
 * contracts a*b+c into an FMA, so this file is compiled with
 * -ffp-contract=off and FMAs appear only where the reference issues them
 * explicitly (_mm256_fmadd_ps), written here as fmaf().
 *
 * Iterator `.sum()` over f32 starts from -0.0 in current Rust (it started from
 * +0.0 before 1.81); the two differ only in the sign of an all-zero sum.  The
 * oracle uses -0.0 at those call sites and +0.0 where the reference writes
 * `let mut sum = 0.0f32`.
 *
 * Parity status of each function (how it is pinned) is listed in the header
 * comment of the function in oracle.c.
 */
#ifndef KLEARU_ORACLE_H
#define KLEARU_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- klearu-accel: simd/mod.rs ---- */
float or_dense_dot_avx2_order(const float* a, const float* b, int64_t n);
float or_dense_dot_scalar(const float* a, const float* b, int64_t n);
float or_sparse_dot_dense_avx2_order(const uint32_t* idx, const float* val, int64_t nnz,
                                     const float* dense);
float or_sparse_dot_dense_scalar(const uint32_t* idx, const float* val, int64_t nnz,
                                 const float* dense);
void or_scatter_add(const uint32_t* idx, const float* val, int64_t n, float* dense, float scale);

/* ---- klearu-accel: bf16/mod.rs (half 2.x bf16 semantics) ---- */
uint16_t or_bf16_from_f32(float x);
float or_bf16_to_f32(uint16_t b);
void or_bf16_from_f32_n(const float* x, uint16_t* out, int64_t n);
float or_bf16_dot_f32(const uint16_t* w, const float* x, int64_t n);
float or_bf16_full_dot(const uint16_t* a, const uint16_t* b, int64_t n);
void or_bf16_update_from_f32(uint16_t* w, const float* delta, int64_t n);
void or_expf_n(const float* x, float* y, int64_t n);

/* ---- rand 0.8.5 StdRng (ChaCha12) as used by SimHash::new / SRP::new ---- */
void or_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]);
uint32_t or_pcg32_output(uint64_t state);
typedef struct {
  uint32_t key[8];
  uint64_t counter; /* next block counter */
  uint32_t buf[64]; /* four blocks of keystream */
  int idx;          /* next unread word in buf; 64 = empty */
} or_stdrng;
void or_stdrng_seed_from_u64(or_stdrng* r, uint64_t seed);
void or_stdrng_from_seed(or_stdrng* r, const uint8_t seed[32]);
uint32_t or_stdrng_next_u32(or_stdrng* r);
uint64_t or_stdrng_next_u64(or_stdrng* r);
double or_stdrng_gen_f64(or_stdrng* r);
/* ---- hash/wta.rs, dwta.rs, minhash.rs (+ rand 0.8.5 shuffle, SipHash-1-3) ---- */
uint32_t or_rand_gen_range_u32(or_stdrng* r, uint32_t n);
void or_rand_shuffle_u32(or_stdrng* r, uint32_t* v, int64_t n);
void or_wta_windows(int dim, int k, int num_tables, int ws, uint64_t seed, uint32_t* windows);
void or_minhash_perms(int dim, int num_tables, uint64_t seed, uint32_t* perms);
int or_wta_bits(int ws);
uint64_t or_wta_hash_dense(const uint32_t* windows, int k, int ws, int table, const float* x);
uint64_t or_siphash(int c_rounds, int d_rounds, uint64_t k0, uint64_t k1, const uint8_t* msg,
                    int64_t len);
uint32_t or_dwta_fallback(uint64_t table, uint64_t hash_fn, int ws);
uint64_t or_dwta_hash_sparse(const uint32_t* windows, int k, int ws, int table, const uint32_t* idx,
                             const float* val, int64_t nnz);
uint64_t or_minhash_hash(const uint32_t* perms, int dim, int k, int table, const uint32_t* nz,
                         int64_t n_nz);

/* ---- hash families: hash/simhash.rs, hash/srp.rs ---- */
void or_simhash_planes(int dim, int k, int num_tables, uint64_t seed, int8_t* planes);
void or_srp_planes(int dim, int k, int num_tables, float sparsity, uint64_t seed, int8_t* planes);
uint64_t or_hash_dense(const int8_t* planes, int dim, int k, int table, const float* x);
uint64_t or_hash_sparse(const int8_t* planes, int dim, int k, int table, const uint32_t* idx,
                        const float* val, int64_t nnz);
void or_hash_dense_batch(const int8_t* planes, int dim, int k, int num_tables, const float* x,
                         int64_t batch, uint32_t* codes);

/* ---- buckets + index: bucket/fifo.rs, bucket/reservoir.rs, lsh/index.rs ---- */
enum { OR_BUCKET_FIFO = 0, OR_BUCKET_RESERVOIR = 1 };
uint64_t or_reservoir_rand(uint64_t seed, uint64_t bound);
void or_lsh_insert_many(int num_tables, int k, int cap, int bucket_type, uint32_t* data,
                        uint32_t* len, uint64_t* count, int64_t n, const uint32_t* ids,
                        const uint32_t* codes);
void or_lsh_remove_many(int num_tables, int k, int cap, uint32_t* data, uint32_t* len, int64_t n,
                        const uint32_t* ids, const uint32_t* codes);
void or_lsh_remove_all(int num_tables, int k, int cap, uint32_t* data, uint32_t* len, int64_t n,
                       const uint32_t* ids);
int64_t or_lsh_query(int num_tables, int k, int cap, const uint32_t* data, const uint32_t* len,
                     const uint32_t* codes, uint32_t* out_ids, uint32_t* out_counts);

/* ---- sampling/{topk,threshold}.rs ---- */
int64_t or_sample_topk(const uint32_t* ids, const uint32_t* counts, int64_t n, int64_t k,
                       uint32_t* out);
int64_t or_sample_threshold(const uint32_t* ids, const uint32_t* counts, int64_t n,
                            uint32_t threshold, uint32_t* out);

/* ---- network/neuron.rs, network/layer.rs ---- */
enum { OR_ACT_RELU = 0, OR_ACT_SIGMOID = 1, OR_ACT_TANH = 2, OR_ACT_SOFTMAX = 3, OR_ACT_IDENTITY = 4 };
float or_neuron_forward(const float* w, float bias, const float* x, int64_t dim);
float or_neuron_forward_sparse(const float* w, float bias, const uint32_t* idx, const float* val,
                               int64_t nnz);
void or_layer_activate(const float* pre, int64_t n, int act, float* out);

int64_t or_slide_forward(const int8_t* planes, int dim, int k, int num_tables, int cap,
                         const uint32_t* data, const uint32_t* len, const float* W,
                         const float* bias, int n, const float* x, int sampling, int top_k,
                         int threshold, int act, uint32_t* out_ids, float* out_pre,
                         float* out_act);
int64_t or_slide_forward_ordered(const int8_t* planes, int dim, int k, int num_tables, int cap,
                                 const uint32_t* data, const uint32_t* len, const float* W,
                                 const float* bias, int n, const float* x, int sampling,
                                 int top_k, int threshold, int act, uint32_t* out_ids,
                                 float* out_pre, float* out_act);

/* ---- SLIDE training: network/layer.rs, network/net.rs, optim/ ---- */
float or_powi_f32(float a, int32_t b);
void or_sgd_update(float* w, const float* gw, int64_t n, float* bias, float gb, double lr,
                   float momentum, float* mw, float* mb);
void or_adam_update(float* w, const float* gw, int64_t n, float* bias, float gb, double lr,
                    uint64_t step, float beta1, float beta2, float eps, float* m_w, float* v_w,
                    float* m_b, float* v_b);
float or_activation_derivative(float pre, float post, int act);
void or_softmax_local_grads(const float* s, const float* go, int64_t n, float* out);
float or_compute_loss(const float* act_dense, const uint32_t* active, int64_t n_act,
                      const uint32_t* labels, int64_t n_labels);
void or_compute_loss_gradient(const float* act_dense, const uint32_t* active, int64_t n_act,
                              const uint32_t* labels, int64_t n_labels, int64_t num_output,
                              float* grad);
void or_layer_backward(float* W, float* bias, int dim, int n, int act, const float* input,
                       const uint32_t* active, int64_t n_act, const float* pre,
                       const float* act_dense, const float* grad_out, int64_t grad_out_len,
                       int opt, float momentum, float beta1, float beta2, float eps,
                       float* st_w1, float* st_w2, float* st_b1, float* st_b2, double lr,
                       uint64_t step, float* grad_in);

/* ---- klearu-dejavu predictor/mlp_predictor.rs ---- */
void or_predictor_predict(const float* w1, const float* b1, const float* w2, const float* b2,
                          int in_dim, int hid, int out_dim, const float* x, float* scores,
                          float* hidden);
void or_predictor_predict_bf16(const uint16_t* w1, const float* b1, const uint16_t* w2,
                               const float* b2, int in_dim, int hid, int out_dim, const float* x,
                               float* scores, float* hidden);
void or_select_top_k(const float* scores, int64_t n, int64_t k, int64_t* out);
float or_sigmoid(float z);

/* ---- klearu-llm sparse/sparse_mlp.rs, model/{rms_norm,rope}.rs, sparse/sparse_attention.rs ---- */
void or_sparse_mlp_forward_bf16(const uint16_t* wg, const uint16_t* wu, const uint16_t* wd,
                                int hidden, int inter, const float* x, const int64_t* active,
                                int64_t k, float* y, float* h);
float or_silu(float x);
float or_rms_inv(const float* x, int64_t n, float eps);
void or_rmsnorm(float* x, const float* w, int64_t n, float eps);
void or_rope_tables(int head_dim, int max_seq, float theta, float* cos_t, float* sin_t);
void or_rope_apply(float* x, int half, const float* cos_t, const float* sin_t, int64_t pos);
void or_linear_forward_bf16(const uint16_t* w, int out_f, int in_f, const float* x, float* y);
void or_sparse_attention_forward_bf16(const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                                      const uint16_t* wo, int hidden, int num_heads,
                                      int num_kv_heads, int head_dim, const float* x, int64_t pos,
                                      const float* cos_t, const float* sin_t, float* k_cache,
                                      float* v_cache, int64_t max_seq, const int64_t* heads,
                                      int64_t n_heads, float* out);

/* ---- timed CPU ports (oracle_avx2.c) ---- */
float or_avx2_dense_dot(const float* a, const float* b, int64_t n);
float or_avx2_sparse_dot_dense(const uint32_t* idx, const float* val, int64_t nnz,
                               const float* dense);
void or_cpu_dejavu_ffn_layer(const float* wg, const float* wu, const float* wd,
                             const float* w_norm, float eps, const float* pw1, const float* pb1,
                             const float* pw2, const float* pb2, int hid_p, int hidden, int inter,
                             int64_t k, float* hstate, float* scratch, int64_t* active_out);
void or_cpu_sparse_attention_layer(const float* wq, const float* wk, const float* wv,
                                   const float* wo, const float* w_norm, float eps,
                                   const float* pw1, const float* pb1, const float* pw2,
                                   const float* pb2, int hid_p, int hidden, int nh, int nkv,
                                   int d, int64_t k, const float* cos_t, const float* sin_t,
                                   float* k_cache, float* v_cache, int64_t max_seq, int64_t pos,
                                   float* hstate, float* scratch, int64_t* heads_out);

/* ---- klearu-dejavu mlp.rs / attention.rs / transformer Linear (toy layer, f32 + bias) ---- */
void or_dejavu_linear_forward_sparse(const float* w, const float* bias, int in_f,
                                     const float* x, const int64_t* idx, int64_t n, float* out);
void or_dejavu_sparse_mlp_forward(const float* wg, const float* bg, const float* wu,
                                  const float* bu, const float* wd, const float* bd, int hidden,
                                  int inter, const float* x, const int64_t* sel, int64_t n,
                                  float* y);
void or_dejavu_linear_forward(const float* w, const float* bias, int in_f, int out_f,
                              const float* x, float* out);
void or_dejavu_sparse_attention_forward(const float* wq, const float* bq, const float* wk,
                                        const float* bk, const float* wv, const float* bv,
                                        const float* wo, const float* bo, int hidden,
                                        int num_heads, int head_dim, const float* x,
                                        const int64_t* heads, int64_t n_heads, float* y);

/* ---- CPU baseline drivers (bench.py): loops over the functions above ---- */
const char* or_compiler_version(void);
void or_cpu_rank_hash_batch(int kind, const uint32_t* tabs, int dim, int k, int ws, int num_tables,
                            const float* X, int64_t rows, uint64_t* codes);
int64_t or_cpu_bolt_batch(const int8_t* planes, int dim, int k, int num_tables, int cap,
                          const uint32_t* data, const uint32_t* len, const float* W, const float* bias,
                          const float* X, int64_t rows, int top_k, int relu, int64_t* out_n,
                          float* out_act);
void or_cpu_lsh_topk_batch(const int8_t* planes, int dim, int k, int num_tables, int cap,
                           const uint32_t* data, const uint32_t* len, const float* X, int64_t rows,
                           int top_k, int64_t* out_n, uint32_t* out_ids);

#ifdef __cplusplus
}
#endif
#endif

