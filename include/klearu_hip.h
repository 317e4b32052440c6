/*
 * klearu_hip.h -- C ABI of libklearu_hip.so, the MI355X (gfx950) implementation
 * of klearu's activation-sparse inference path.
 *
 * Each entry point names the reference interface it replaces (path:line in
 * QuilibriumNetwork/klearu).  Conventions:
 *   - Every function returns int: KH_OK (0) or a negative KH_ERR_* code; the
 *     message of the last failure on the calling thread is kh_last_error().
 *     Nothing aborts: the reference's panics on length mismatch become
 *     KH_ERR_ARG.
 *   - Pointers named *_dev are device pointers (hipMalloc'd or torch tensors);
 *     pointers named *_host are host pointers.  `stream` is a hipStream_t
 *     (NULL = the legacy default stream).  Compute calls are asynchronous on
 *     that stream unless stated otherwise.
 *   - Handles are device-resident and immutable after creation except where a
 *     function says it mutates the handle (the reference's `&mut self`, which
 *     needs exclusive access).  Non-mutating calls (the reference's `&self`
 *     methods of Send + Sync types) may run concurrently on one handle from
 *     different streams and host threads: a handle keeps one scratch set per
 *     stream, and calls on one stream are ordered by it.  Scratch is sized by
 *     the first calls on a stream; warm a stream up before capturing it in a
 *     HIP graph (buffers that are outgrown stay allocated until the handle is
 *     destroyed, so earlier graphs stay valid).
 *   - Selections (hash codes, active sets, top-k) are bit-exact with the
 *     reference's sequential f32 arithmetic.  Sets whose reference order is a
 *     HashMap iteration order are returned in ascending id order.
 */
#ifndef KLEARU_HIP_H
#define KLEARU_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KH_OK 0
#define KH_ERR_ARG (-1)         /* bad shape / argument (reference: assert panic) */
#define KH_ERR_HIP (-2)         /* HIP runtime error */
#define KH_ERR_CAPACITY (-3)    /* output capacity too small */
#define KH_ERR_ALLOC (-4)       /* device allocation failed */
#define KH_ERR_UNSUPPORTED (-5) /* shape outside what the kernels support */

const char* kh_last_error(void);
int kh_version(void);

/* ======================================================================== */
/* klearu-accel entry points (crates/klearu-accel/src/simd/mod.rs,          */
/* crates/klearu-accel/src/bf16/mod.rs)                                     */
/* ======================================================================== */

/* dense_dot_dense_simd (simd/mod.rs:54-72), batched over rows:
 * out[r] = dot(a[r*lda .. r*lda+n], b[0..n]) in the AVX2 order of
 * simd/mod.rs:174-207 (bit-exact). */
int kh_dense_dot_dense(const float* a_dev, int64_t rows, int64_t lda, const float* b_dev,
                       int64_t n, float* out_dev, void* stream);

/* sparse_dot_dense_simd (simd/mod.rs:19-36): out[0] = sum_i val[i]*dense[idx[i]]
 * in the AVX2 gather order of simd/mod.rs:145-170 (bit-exact). */
int kh_sparse_dot_dense(const uint32_t* idx_dev, const float* val_dev, int64_t nnz,
                        const float* dense_dev, int64_t dense_len, float* out_dev,
                        void* stream);

/* scatter_add_simd (simd/mod.rs:86-109): dense[idx[i]] += val[i]*scale, with
 * duplicate indices applied in index order (bit-exact, atomic-free). */
int kh_scatter_add(const uint32_t* idx_dev, const float* val_dev, int64_t n, float* dense_dev,
                   int64_t dense_len, float scale, void* stream);

/* Bf16Weights::from_f32 (bf16/mod.rs:37-41): round to nearest even. */
int kh_bf16_from_f32(const float* x_dev, uint16_t* out_dev, int64_t n, void* stream);
/* Bf16Weights::to_f32 (bf16/mod.rs:44-46). */
int kh_bf16_to_f32(const uint16_t* x_dev, float* out_dev, int64_t n, void* stream);
/* Bf16Weights::dot_f32 (bf16/mod.rs:64-77), rows batched like kh_dense_dot_dense;
 * sequential f32 sum (bit-exact). */
int kh_bf16_dot_f32(const uint16_t* w_dev, int64_t rows, int64_t ldw, const float* x_dev,
                    int64_t n, float* out_dev, void* stream);
/* Bf16FullMode::dot (bf16/mod.rs:122-134), sequential f32 sum (bit-exact). */
int kh_bf16_full_dot(const uint16_t* a_dev, const uint16_t* b_dev, int64_t n, float* out_dev,
                     void* stream);
/* Bf16Weights::update_from_f32 (bf16/mod.rs:85-88) for every element:
 * w[i] = bf16(f32(w[i]) + delta[i]). */
int kh_bf16_update_from_f32(uint16_t* w_dev, const float* delta_dev, int64_t n, void* stream);

/* f32::exp as Rust evaluates it on x86-64 Linux (glibc expf), elementwise:
 * the exponential inside the predictor's sigmoid (mlp_predictor.rs:121),
 * SiLU (sparse_mlp.rs:41), the SLIDE activations (layer.rs:253, :295) and the
 * attention softmax (sparse_attention.rs:88).  Bit-identical to glibc expf. */
int kh_expf(const float* x_dev, float* y_dev, int64_t n, void* stream);

/* ======================================================================== */
/* LSH hash families (crates/klearu-core/src/hash/)                         */
/* ======================================================================== */

typedef struct kh_hash_family kh_hash_family;

/* SimHash::new(input_dim, k, num_tables, seed) (hash/simhash.rs:37-58):
 * ternary planes drawn from a restatement of rand 0.8 StdRng (ChaCha12) in
 * table->bit->dim order.  No reference test holds a drawn value, so the
 * seed -> plane stream is unpinned; a caller that needs the reference's exact
 * planes draws them with SimHash::new and passes them to
 * kh_hash_family_from_planes. */
int kh_simhash_create(int input_dim, int k, int num_tables, uint64_t seed, kh_hash_family** out);
/* SparseRandomProjection::new (hash/srp.rs:43-84); same StdRng caveat. */
int kh_srp_create(int input_dim, int k, int num_tables, float sparsity, uint64_t seed,
                  kh_hash_family** out);
/* A family from explicit ternary planes planes_host[num_tables][k][input_dim]
 * with entries in {-1, 0, +1}. */
int kh_hash_family_from_planes(int input_dim, int k, int num_tables, const int8_t* planes_host,
                               kh_hash_family** out);
int kh_hash_family_destroy(kh_hash_family* h);
/* HashFamily::k / input_dim / num_tables (hash/mod.rs:31-38). */
int kh_hash_family_dims(const kh_hash_family* h, int* k, int* input_dim, int* num_tables);
/* Copies the planes back as planes_host[num_tables][k][input_dim]. */
int kh_hash_family_planes(const kh_hash_family* h, int8_t* planes_host);
/* The rank-based families (crates/klearu-core/src/hash/wta.rs, dwta.rs,
 * minhash.rs).  Their codes, as kh_hash_dense / kh_hash_sparse return them,
 * are the low 32 bits of the reference's u64 code (an index keeps the low k).
 * WtaHash::new(input_dim, k, num_tables, window_size, seed) (wta.rs:42-90):
 * per table and hash function, the first window_size entries of a shuffle
 * of 0..input_dim (rand 0.8.5 SliceRandom::shuffle on StdRng); k *
 * ceil(log2(window_size)) <= 64.  The composed seed -> window stream is
 * restated, not pinned by a reference value; kh_wta_from_windows takes
 * windows drawn by the reference itself. */
int kh_wta_create(int input_dim, int k, int num_tables, int window_size, uint64_t seed,
                  kh_hash_family** out);
/* DwtaHash::new (dwta.rs:40-88): WTA's windows; sparse inputs (sorted,
 * distinct indices, as SparseVector holds them) hash over stored dimensions
 * only, an empty window taking DefaultHasher((table, hash_fn)) % window_size. */
int kh_dwta_create(int input_dim, int k, int num_tables, int window_size, uint64_t seed,
                   kh_hash_family** out);
/* WTA (dwta = 0) or DWTA (dwta = 1) from windows_host[num_tables][k][window_size]. */
int kh_wta_from_windows(int dwta, int input_dim, int k, int num_tables, int window_size,
                        const uint32_t* windows_host, kh_hash_family** out);
/* MinHash::new (minhash.rs:38-60): one shuffled 0..input_dim per table; k bins. */
int kh_minhash_create(int input_dim, int k, int num_tables, uint64_t seed, kh_hash_family** out);
/* MinHash from perms_host[num_tables][input_dim] (permutations[table][dim]). */
int kh_minhash_from_permutations(int input_dim, int k, int num_tables, const uint32_t* perms_host,
                                 kh_hash_family** out);
#define KH_FAMILY_TERNARY 0 /* SimHash / SparseRandomProjection hyperplanes */
#define KH_FAMILY_WTA 1
#define KH_FAMILY_DWTA 2
#define KH_FAMILY_MINHASH 3
/* The family's kind and window size (0 unless WTA / DWTA). */
int kh_hash_family_kind(const kh_hash_family* h, int* kind, int* window_size);
/* Copy WTA / DWTA windows [L][k][window_size] or MinHash permutations
 * [L][input_dim] (KH_ERR_UNSUPPORTED for hyperplane families). */
int kh_hash_family_tables(const kh_hash_family* h, uint32_t* out_host);
/* HashFamily::hash_dense (hash/mod.rs:26) for every table and a batch:
 * codes[b][t] = hash_dense(x[b], t), x_dev [batch][input_dim]. */
int kh_hash_dense(const kh_hash_family* h, const float* x_dev, int64_t batch, uint32_t* codes_dev,
                  void* stream);
/* HashFamily::hash_sparse (hash/mod.rs:29) for a CSR batch: row b is
 * (idx[off[b]..off[b+1]], val[...]) with ascending idx (SparseVector). */
int kh_hash_sparse(const kh_hash_family* h, const int64_t* off_dev, const uint32_t* idx_dev,
                   const float* val_dev, int64_t batch, uint32_t* codes_dev, void* stream);

/* ======================================================================== */
/* LSH index (crates/klearu-core/src/lsh/index.rs, bucket/)                 */
/* ======================================================================== */

#define KH_BUCKET_FIFO 0      /* FifoBucket (bucket/fifo.rs:26-55) */
#define KH_BUCKET_RESERVOIR 1 /* ReservoirBucket (bucket/reservoir.rs:50-90) */

typedef struct kh_lsh_index kh_lsh_index;

/* LshIndex::new(hash_family, bucket_type, capacity) (lsh/index.rs:193-204).
 * The index keeps a reference to `h`, which must outlive it. */
int kh_lsh_index_create(const kh_hash_family* h, int bucket_type, int capacity,
                        kh_lsh_index** out);
int kh_lsh_index_destroy(kh_lsh_index* idx);
/* LshIndexTrait::insert (lsh/index.rs:257-262) for n vectors in order:
 * ids[i] with dense weights w[i*ldw .. i*ldw+input_dim] (tables inner). Mutates.
 * Batches of 1024 or more vectors hash on the matrix cores with an exact
 * sequential replay wherever the sign is not certain (same codes).  The
 * mutation calls keep their device scratch in the index (about 20 bytes per
 * vector and table of the largest call) until it is destroyed. */
int kh_lsh_index_insert(kh_lsh_index* idx, const uint32_t* ids_dev, const float* w_dev,
                        int64_t n, int64_t ldw, void* stream);
/* Same from precomputed codes[n][num_tables] (e.g. from kh_hash_dense). */
int kh_lsh_index_insert_codes(kh_lsh_index* idx, const uint32_t* ids_dev,
                              const uint32_t* codes_dev, int64_t n, void* stream);
/* LshIndexTrait::insert_sparse (lsh/index.rs:264-269) for n SparseVectors in
 * order (CSR: vector i is xidx/xval[xoff[i]..xoff[i+1]], ascending indices),
 * hashed with hash_sparse.  Mutates. */
int kh_lsh_index_insert_sparse(kh_lsh_index* idx, const uint32_t* ids_dev, const int64_t* xoff_dev,
                               const uint32_t* xidx_dev, const float* xval_dev, int64_t n,
                               void* stream);
/* LshIndexTrait::remove_with_weights (lsh/index.rs:271-276) for n vectors in
 * order: in each table, the bucket the weights hash to drops the id's first
 * entry by swap_remove (bucket/fifo.rs:35-42, bucket/reservoir.rs:69-76);
 * reservoir insertion counts are unchanged.  Mutates; synchronises. */
int kh_lsh_index_remove_with_weights(kh_lsh_index* idx, const uint32_t* ids_dev,
                                     const float* w_dev, int64_t n, int64_t ldw, void* stream);
/* Same from precomputed codes[n][num_tables]. */
int kh_lsh_index_remove_codes(kh_lsh_index* idx, const uint32_t* ids_dev,
                              const uint32_t* codes_dev, int64_t n, void* stream);
/* LshIndexTrait::remove (lsh/index.rs:278-280, BucketStorage::remove_all
 * :146-164): each id in order is removed (first entry, swap_remove) from every
 * bucket of every table.  Mutates; synchronises. */
int kh_lsh_index_remove(kh_lsh_index* idx, const uint32_t* ids_dev, int64_t n, void* stream);
/* LshIndexTrait::clear (lsh/index.rs:313-315). Mutates. */
int kh_lsh_index_clear(kh_lsh_index* idx, void* stream);
/* LshIndexTrait::rebuild (lsh/index.rs:302-307): clear, then insert ids_dev[i]
 * with weights w_dev + i*ldw in order.  Mutates; synchronises. */
int kh_lsh_index_rebuild(kh_lsh_index* idx, const uint32_t* ids_dev, const float* w_dev,
                         int64_t n, int64_t ldw, void* stream);
/* LshIndexTrait::query / query_with_counts (lsh/index.rs:282-284, :294-296)
 * for a batch of dense inputs.  Output is CSR: the unique ids of sample b are
 * ids_dev[off[b]..off[b+1]] in ascending order with counts_dev (number of
 * table hits; may be NULL for query_union, index.rs:286-288).  off_dev has
 * batch+1 entries; off[batch] is the total even when it exceeds capacity, in
 * which case nothing past capacity is written and the call returns
 * KH_ERR_CAPACITY (this check synchronises the stream). */
int kh_lsh_index_query(const kh_lsh_index* idx, const float* x_dev, int64_t batch,
                       int64_t* off_dev, uint32_t* ids_dev, uint32_t* counts_dev,
                       int64_t capacity, void* stream);
/* query_sparse_union / query_sparse_with_counts (lsh/index.rs:290-299), CSR input. */
int kh_lsh_index_query_sparse(const kh_lsh_index* idx, const int64_t* xoff_dev,
                              const uint32_t* xidx_dev, const float* xval_dev, int64_t batch,
                              int64_t* off_dev, uint32_t* ids_dev, uint32_t* counts_dev,
                              int64_t capacity, void* stream);
/* LshSparsityPredictor::predict (crates/klearu-dejavu/src/predictor/
 * lsh_predictor.rs:33-43) for a batch of dense inputs: the query's candidates
 * sorted by hit count descending (ties: ascending id; the reference's follow
 * HashMap order), the first top_k: ids_dev[batch][top_k] with n_dev[b] of them
 * valid.  (build_from_observations, :22-30, is kh_lsh_index_clear then
 * kh_lsh_index_insert of each observation's input once per important id.) */
int kh_lsh_index_query_top_k(const kh_lsh_index* idx, const float* x_dev, int64_t batch,
                             int64_t top_k, uint32_t* ids_dev, int32_t* n_dev, void* stream);
/* Bucket contents for parity checks (synchronous): data_host[L][2^k][cap],
 * len_host[L][2^k], count_host[L][2^k] (reservoir insertion counters). */
int kh_lsh_index_buckets(const kh_lsh_index* idx, uint32_t* data_host, uint32_t* len_host,
                         uint64_t* count_host);

/* ======================================================================== */
/* SLIDE sparse layer (crates/klearu-core/src/network/layer.rs)             */
/* ======================================================================== */

#define KH_SAMPLING_VANILLA 0   /* sampling/vanilla.rs:8-12 */
#define KH_SAMPLING_TOPK 1      /* sampling/topk.rs:19-34 */
#define KH_SAMPLING_THRESHOLD 2 /* sampling/threshold.rs:20-43 */

#define KH_ACT_RELU 0     /* layer.rs:252 */
#define KH_ACT_SIGMOID 1  /* layer.rs:253 */
#define KH_ACT_TANH 2     /* layer.rs:254 */
#define KH_ACT_SOFTMAX 3  /* layer.rs:286-308 */
#define KH_ACT_IDENTITY 4 /* layer.rs:255 */

typedef struct kh_slide_layer kh_slide_layer;

/* Layer{neurons, lsh_index, sampling, config} (layer.rs:10-15) built from
 * explicit weights: w_host[num_neurons][input_dim] f32, bias_host[num_neurons].
 * The index is built by inserting neurons 0..n-1 in order (layer.rs:42-44).
 * `index` must have been created over a family with this input_dim and stay
 * alive; the layer inserts into it. */
int kh_slide_layer_create(int input_dim, int num_neurons, const float* w_host,
                          const float* bias_host, kh_lsh_index* index, int sampling, int top_k,
                          int threshold, int activation, kh_slide_layer** out);
int kh_slide_layer_destroy(kh_slide_layer* l);
/* Layer::forward (layer.rs:65-120) for a batch of dense inputs x_dev[batch][input_dim].
 * Active neurons of sample b: act_ids[off[b]..off[b+1]] (ascending id), with
 * pre-activations and activations in the same order (either may be NULL).
 * Same capacity rules as kh_lsh_index_query. */
int kh_slide_layer_forward(const kh_slide_layer* l, const float* x_dev, int64_t batch,
                           int64_t* off_dev, uint32_t* act_ids_dev, float* pre_dev,
                           float* act_dev, int64_t capacity, void* stream);
/* Same for CSR sparse inputs (Neuron::forward_sparse, neuron.rs:66-68; the
 * hash uses hash_sparse). */
int kh_slide_layer_forward_sparse(const kh_slide_layer* l, const int64_t* xoff_dev,
                                  const uint32_t* xidx_dev, const float* xval_dev, int64_t batch,
                                  int64_t* off_dev, uint32_t* act_ids_dev, float* pre_dev,
                                  float* act_dev, int64_t capacity, void* stream);
/* SparseInferenceEngine::infer (relu = 1) / infer_linear (relu = 0)
 * (crates/klearu-bolt/src/sparse_inference.rs:36-111) over the layer's index
 * and weights: effective_k = (base_top_k as f32 * sparsity_multiplier) as
 * usize; the query's candidates sorted by hit count (descending; the
 * reference's ties follow HashMap order, here ascending id), the first
 * effective_k of them with id < num_neurons, each the sequential dot of x and
 * its weights plus bias, then max(0) for infer.  No all-neurons fallback:
 * an empty candidate set gives an empty row.  Output CSR as
 * kh_slide_layer_forward (ids in that order; act_dev may be NULL). */
int kh_sparse_inference(const kh_slide_layer* l, const float* x_dev, int64_t batch,
                        int64_t base_top_k, float sparsity_multiplier, int relu, int64_t* off_dev,
                        uint32_t* ids_dev, float* act_dev, int64_t capacity, void* stream);

/* Dense layer over sparse inputs: y[b][o] = act(Neuron::forward_sparse) for all
 * neurons (the 128-d hidden layer of the extreme-classification net).
 * w_host[num_neurons][input_dim]. */
typedef struct kh_dense_layer kh_dense_layer;
int kh_dense_layer_create(int input_dim, int num_neurons, const float* w_host,
                          const float* bias_host, int activation, kh_dense_layer** out);
int kh_dense_layer_destroy(kh_dense_layer* l);
int kh_dense_layer_forward_sparse(const kh_dense_layer* l, const int64_t* xoff_dev,
                                  const uint32_t* xidx_dev, const float* xval_dev, int64_t batch,
                                  float* y_dev, void* stream);

/* ======================================================================== */
/* SLIDE training: backward, optimizers, rebuild scheduling                 */
/* (network/layer.rs:124-233, network/net.rs:81-230, optim/, lsh/maintenance.rs) */
/* ======================================================================== */

/* RebuildScheduler (lsh/maintenance.rs:20-98): host-side state.  The interval
 * after the i-th rebuild is (usize)(base * exp(decay * i)) (f64 exp, truncated,
 * saturating), at least 1; the step arithmetic wraps as Rust's release build. */
typedef struct kh_rebuild_scheduler {
  uint64_t base_interval;
  double decay;
  uint64_t rebuild_count;
  uint64_t next_rebuild_step;
  uint64_t current_step;
} kh_rebuild_scheduler;
/* RebuildScheduler::new (maintenance.rs:36-44). */
void kh_rebuild_scheduler_init(kh_rebuild_scheduler* s, uint64_t base_interval, double decay);
/* RebuildScheduler::step (:48-62): 1 when a rebuild is due at the new step. */
int kh_rebuild_scheduler_step(kh_rebuild_scheduler* s);
/* RebuildScheduler::should_rebuild (:70-81): jump to `step`, 1 when due. */
int kh_rebuild_scheduler_should_rebuild(kh_rebuild_scheduler* s, uint64_t step);

#define KH_OPT_SGD 0  /* optim/sgd.rs:3-69 (momentum 0 = vanilla) */
#define KH_OPT_ADAM 1 /* optim/adam.rs:3-90 */

/* Layer::rebuild_index (layer.rs:228-233): clear the layer's index and insert
 * neurons 0..n-1 from the current weights.  Mutates; synchronises. */
int kh_slide_layer_rebuild_index(kh_slide_layer* l, void* stream);
/* Optimizer::create_state for every neuron (net.rs:40-55): zeroed SGD momentum
 * (momentum > 0) or Adam moments.  Replaces any earlier state.  Synchronous. */
int kh_slide_layer_init_optimizer(kh_slide_layer* l, int optimizer, float momentum, float beta1,
                                  float beta2, float eps);
/* Copy the current weights [n][dim] and biases [n] back.  Synchronous. */
int kh_slide_layer_weights(const kh_slide_layer* l, float* w_host, float* bias_host);
/* Layer::backward (layer.rs:124-226) for one sample.  The LayerOutput is given
 * on the device: act_ids_dev[0..*n_act_dev) in the order the forward produced
 * them (the sums over active neurons follow it), pre_dev in the same order,
 * act_dense_dev[n] the layer's dense activations; x_dev[dim] the layer's
 * input; grad_out_dev[grad_out_len] (entries past the length read as 0).
 * Computes grad_in_dev[dim] (may be NULL when not needed) from the weights
 * before the update, then updates every active neuron's weights and bias with
 * the layer's optimizer (kh_slide_layer_init_optimizer) at learning rate
 * (f32)lr and step `step`.  Mutates the layer. */
int kh_slide_layer_backward(kh_slide_layer* l, const float* x_dev, const uint32_t* act_ids_dev,
                            const int32_t* n_act_dev, const float* pre_dev,
                            const float* act_dense_dev, const float* grad_out_dev,
                            int64_t grad_out_len, double lr, uint64_t step, float* grad_in_dev,
                            void* stream);

typedef struct kh_slide_network kh_slide_network;
/* Network (net.rs:10-58) over existing layers (not owned; they must outlive
 * the network, and layer i+1's input_dim must equal layer i's num_neurons).
 * Initialises every layer's optimizer state (momentum / beta1 / beta2 / eps as
 * Sgd::new / Adam::new take them; the reference's NetworkConfig uses
 * Sgd::new(0.9) and Adam::default() = 0.9, 0.999, 1e-8) and a
 * RebuildScheduler(rebuild_base, rebuild_decay). */
int kh_slide_network_create(kh_slide_layer* const* layers, int n_layers, int optimizer,
                            float momentum, float beta1, float beta2, float eps,
                            uint64_t rebuild_base, double rebuild_decay, kh_slide_network** out);
int kh_slide_network_destroy(kh_slide_network* n);
/* Network::train_step (net.rs:81-120, backward :122-146) over examples x_dev[batch][input_dim]
 * (Example::features.to_dense()) with labels labels_host[label_off_host[b] ..
 * label_off_host[b+1]]: per example in order, forward (Layer::forward with the
 * sampler's order: top-k sampling lists the active neurons by count
 * descending, then id; the other samplers by ascending id, where the
 * reference's HashMap order differs from run to run), compute_loss /
 * compute_loss_gradient (net.rs:180-230) and the backward pass of every
 * layer, updating weights as it goes; then step += 1 and, when the scheduler
 * says so, every layer's index is rebuilt.  *loss_out = total / batch (0 for
 * an empty batch, which changes nothing).  Mutates; synchronises. */
int kh_slide_network_train_step(kh_slide_network* n, const float* x_dev, int64_t batch,
                                const int64_t* label_off_host, const uint32_t* labels_host,
                                double lr, float* loss_out, void* stream);
/* Same with the examples' features as CSR rows (SparseVector, at most 4096
 * stored entries each): row b is xidx/xval[xoff[b]..xoff[b+1]), densified as
 * SparseVector::to_dense does (tensor/sparse.rs:77-83: a later entry at the
 * same index overwrites an earlier one); indices >= input_dim are skipped. */
int kh_slide_network_train_step_sparse(kh_slide_network* n, const int64_t* xoff_dev,
                                       const uint32_t* xidx_dev, const float* xval_dev,
                                       int64_t batch, const int64_t* label_off_host,
                                       const uint32_t* labels_host, double lr, float* loss_out,
                                       void* stream);
/* Network::predict (net.rs:151-154) for each row of x_dev[batch][input_dim]:
 * out_dev[batch][num_neurons of the last layer], the last layer's dense
 * activations. */
int kh_slide_network_predict(kh_slide_network* n, const float* x_dev, int64_t batch,
                             float* out_dev, void* stream);
/* Same for CSR rows (as kh_slide_network_train_step_sparse reads them). */
int kh_slide_network_predict_sparse(kh_slide_network* n, const int64_t* xoff_dev,
                                    const uint32_t* xidx_dev, const float* xval_dev,
                                    int64_t batch, float* out_dev, void* stream);
/* Network::step (net.rs:13) and the scheduler's state. */
int kh_slide_network_state(const kh_slide_network* n, uint64_t* step,
                           kh_rebuild_scheduler* scheduler);

/* ======================================================================== */
/* Deja Vu predictor + top-k (crates/klearu-dejavu/src/predictor/,          */
/* crates/klearu-llm/src/sparse/predictor_store.rs)                         */
/* ======================================================================== */

typedef struct kh_predictor kh_predictor;

/* SparsityPredictor::from_weights (mlp_predictor.rs:66-84): w1_host[hidden][input],
 * b1_host[hidden], w2_host[output][hidden], b2_host[output], all f32 as the
 * reference stores them. */
int kh_predictor_create(int input_dim, int hidden_dim, int output_dim, const float* w1_host,
                        const float* b1_host, const float* w2_host, const float* b2_host,
                        kh_predictor** out);
int kh_predictor_destroy(kh_predictor* p);
/* The reference's predictor cannot fail after construction, so this has no
 * counterpart there: the batched layer-1 kernel (batches of two or more rows)
 * hands products between its waves through LDS flags whose waits are bounded,
 * so a lost hand-off ends the kernel instead of hanging it, and is recorded on
 * the handle.  kh_predictor_status synchronises the device and returns
 * KH_ERR_HIP (clearing the record) if any call since the last status call
 * gave up a wait -- its scores are then not trusted -- else KH_OK. */
int kh_predictor_status(const kh_predictor* p);
/* Test hook, no counterpart in the reference: the number of sleeps (about 64
 * cycles each) after which such a wait gives up (default 4194304; at least 1).
 * A tiny limit forces the give-up path while every kernel still exits. */
int kh_predictor_set_spin_limit(kh_predictor* p, int spins);
/* SparsityPredictor::predict (mlp_predictor.rs:102-124) for x_dev[batch][input]:
 * scores_dev[batch][output] (sigmoid), bit-exact with the reference. */
int kh_predictor_predict(const kh_predictor* p, const float* x_dev, int64_t batch,
                         float* scores_dev, void* stream);

#define KH_ORDER_SCORE 0     /* reference order: score descending, ties by index */
#define KH_ORDER_ASCENDING 1 /* same set, ascending index */

/* SparsityPredictor::select_top_k (mlp_predictor.rs:127-132) /
 * PredictorStore::predict_neurons|predict_heads (predictor_store.rs:31-45):
 * ids_dev[batch][min(k, output)] (int32). */
int kh_predictor_select_top_k(const kh_predictor* p, const float* x_dev, int64_t batch, int k,
                              int order, int32_t* ids_dev, void* stream);
/* No counterpart in the reference: kh_predictor_select_top_k for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  Same arguments and results, bit-identical; every
 * buffer comes from one static 4 MiB device array per GPU, so it calls no
 * hipMalloc/hipFree.  Requests needing more than 4 MiB of scratch
 * (4*batch*(hidden + output) + 8*batch*ceil(output/64) bytes, plus
 * 8*batch*min(k, output) for KH_ORDER_SCORE, each rounded up to 256) return
 * KH_ERR_CAPACITY.  All calls on one GPU share the array: calls that overlap
 * on one GPU (other streams, other threads) race and must be ordered. */
int kh_predictor_select_top_k_noalloc(const kh_predictor* p, const float* x_dev, int64_t batch,
                                      int k, int order, int32_t* ids_dev, void* stream);
/* The stable top-k of arbitrary scores (the sort of mlp_predictor.rs:129-131):
 * scores_dev[batch][n] -> ids_dev[batch][min(k, n)].  NaN scores are not supported. */
int kh_topk_select(const float* scores_dev, int64_t batch, int n, int k, int order,
                   int32_t* ids_dev, void* stream);
/* Union of batch top-k sets (the shared active set of a multi-token decode
 * step): ids_dev[batch][k] over [0, n) -> union_dev[<= n] ascending and
 * *count_dev (device int32). */
int kh_union_active(const int32_t* ids_dev, int64_t batch, int k, int n, int32_t* union_dev,
                    int32_t* count_dev, void* stream);
/* kh_predictor_select_top_k (ascending order) and kh_union_active in one call:
 * the top-k kernel marks the selected neurons and the union is read from the
 * marks (mlp_predictor.rs:127-132 per row, then the shared active set).
 * ids_dev[batch][min(k, output)], union_dev[<= output] ascending, *count_dev.
 * The marks live in the handle's per-stream scratch. */
int kh_predictor_select_top_k_union(const kh_predictor* p, const float* x_dev, int64_t batch,
                                    int k, int32_t* ids_dev, int32_t* union_dev,
                                    int32_t* count_dev, void* stream);

/* ======================================================================== */
/* Sparse SwiGLU FFN (crates/klearu-llm/src/sparse/sparse_mlp.rs)           */
/* ======================================================================== */

typedef struct kh_sparse_ffn kh_sparse_ffn;

/* Mlp{gate_proj, up_proj, down_proj} (model/mlp.rs:6-21) from BF16 bits in the
 * reference layout: w_gate/w_up [inter][hidden], w_down [hidden][inter].
 * max_batch bounds the token batch of later forward calls (1..16). */
int kh_sparse_ffn_create(int hidden, int inter, const uint16_t* w_gate_host,
                         const uint16_t* w_up_host, const uint16_t* w_down_host, int max_batch,
                         kh_sparse_ffn** out);
/* Same from device arrays in the reference layout (weights already in HBM);
 * repacks on the device and synchronises. */
int kh_sparse_ffn_create_dev(int hidden, int inter, const uint16_t* w_gate_dev,
                             const uint16_t* w_up_dev, const uint16_t* w_down_dev, int max_batch,
                             kh_sparse_ffn** out);
int kh_sparse_ffn_destroy(kh_sparse_ffn* f);
/* sparse_mlp::forward_sparse (sparse_mlp.rs:4-37) for a batch of tokens sharing
 * one active set: y[b] (=, or += when accumulate != 0) sum over active neurons a
 * of Wd[:, a] * silu(Wg[a].x[b]) * (Wu[a].x[b]).  active_dev: int32 neuron ids
 * (unique, any order); n_active is used as is, or, when n_active_dev is not
 * NULL, *n_active_dev is read on the device and n_active is its upper bound. */
int kh_sparse_ffn_forward(const kh_sparse_ffn* f, const float* x_dev, int64_t batch,
                          const int32_t* active_dev, int n_active, const int32_t* n_active_dev,
                          float* y_dev, int accumulate, void* stream);
/* Ids in an active list must lie in [0, intermediate) (the reference panics,
 * crates/klearu-accel/src/memory/mod.rs:87-92).  The kernels check every id:
 * one outside the range reads row 0 instead (no access leaves the weights)
 * and is recorded on the handle.  kh_sparse_ffn_status synchronises the
 * device and returns KH_ERR_ARG (clearing the record) if any call since the
 * last status call saw such an id, else KH_OK. */
int kh_sparse_ffn_status(const kh_sparse_ffn* f);
/* Per-neuron activations h[b][i] = silu(g)*u of the last forward on `stream`, for tests. */
int kh_sparse_ffn_last_hidden(const kh_sparse_ffn* f, float* h_dev, int64_t batch, int n_active,
                              void* stream);

/* RmsNorm::forward (model/rms_norm.rs:43-64): y[b] = (x[b] * inv_rms) * w with
 * the sum of squares in the reference's sequential order (bit-identical). */
int kh_rmsnorm(const float* x_dev, const float* w_dev, int64_t batch, int n, float eps,
               float* y_dev, void* stream);

/* One decode step (batch 1) of the Deja Vu MLP block as
 * SparseModel::forward_decode_sparse runs it (crates/klearu-llm/src/sparse/mod.rs:115-142):
 *   norm = RmsNorm(hidden) (model/rms_norm.rs:43-64, weight norm_w, eps);
 *   active = predictor.select_top_k(norm, k) (ascending ids into active_dev[k]);
 *   hidden += sparse_mlp::forward_sparse(norm, active).
 * The norm is applied inside the predictor and FFN kernels.  Its sum of squares
 * is the reference's sequential f32 sum, so the normalised row, the scores and
 * the selected set are bit-identical to the reference's for the same hidden
 * row.  norm_ws_dev (>= 1 float, device) receives the row's scale 1/rms.
 * Requires predictor input_dim == hidden, output_dim == intermediate, hidden a
 * multiple of 64 and at most 4096 (larger hidden sizes run the unfused calls:
 * kh_rmsnorm, kh_predictor_select_top_k, kh_sparse_ffn_forward). */
int kh_dejavu_mlp_block(const kh_predictor* p, const kh_sparse_ffn* f, float* hidden_dev,
                        const float* norm_w_dev, float eps, int k, int32_t* active_dev,
                        float* norm_ws_dev, void* stream);
/* kh_dejavu_mlp_block for rows 0..batch-1 of hidden_dev[batch][hidden]
 * (sparse/mod.rs:115-142 per row): each row's RmsNorm (scale to
 * norm_ws_dev[batch]) and top-k ids (active_dev[batch][k], ascending) are the
 * reference's bit for bit, and the FFN runs over the union of the rows'
 * selections, as kh_rmsnorm, kh_predictor_select_top_k_union and
 * kh_sparse_ffn_forward would in sequence (the union is taken inside the
 * FFN's gate/up kernel where the shape allows).  batch 1 is
 * kh_dejavu_mlp_block.  Requires hidden <= 8192. */
int kh_dejavu_mlp_block_batch(const kh_predictor* p, const kh_sparse_ffn* f, float* hidden_dev,
                              int64_t batch, const float* norm_w_dev, float eps, int k,
                              int32_t* active_dev, float* norm_ws_dev, void* stream);

/* ======================================================================== */
/* klearu-dejavu transformer layer: f32 Linear with bias, SparseMlp,        */
/* SparseAttention (crates/klearu-dejavu/src/{transformer/mod.rs,mlp.rs,     */
/* attention.rs}).  Outputs are bit-identical to the reference.  Index lists */
/* are host arrays (the reference's &[usize]); these calls wait until the   */
/* list is uploaded, then leave the kernels queued on `stream`.             */
/* ======================================================================== */

typedef struct kh_dejavu_linear kh_dejavu_linear;

/* Linear{weight [out][in], bias [out]} (transformer/mod.rs:79-111) from host arrays. */
int kh_dejavu_linear_create(int in_features, int out_features, const float* w_host,
                            const float* b_host, kh_dejavu_linear** out);
int kh_dejavu_linear_destroy(kh_dejavu_linear* l);
/* Linear::forward (transformer/mod.rs:114-123): y_dev[batch][out] from x_dev[batch][in]. */
int kh_dejavu_linear_forward(const kh_dejavu_linear* l, const float* x_dev, int64_t batch,
                             float* y_dev, void* stream);
/* Linear::forward_sparse (transformer/mod.rs:126-134): y_dev[b][a] = row idx_host[a]
 * (any order, repeats allowed).  Out-of-range indices are KH_ERR_ARG (the
 * reference panics). */
int kh_dejavu_linear_forward_sparse(const kh_dejavu_linear* l, const float* x_dev, int64_t batch,
                                    const int64_t* idx_host, int64_t n_idx, float* y_dev,
                                    void* stream);

typedef struct kh_dejavu_sparse_mlp kh_dejavu_sparse_mlp;

/* SparseMlp::new(hidden_size, intermediate_size) (mlp.rs:11-16). */
int kh_dejavu_sparse_mlp_create(int hidden, int inter, kh_dejavu_sparse_mlp** out);
int kh_dejavu_sparse_mlp_destroy(kh_dejavu_sparse_mlp* m);
/* SparseMlp::forward (mlp.rs:23-58) for every row of x_dev[batch][hidden] with the
 * same selected neurons: y_dev[batch][hidden]. */
int kh_dejavu_sparse_mlp_forward(const kh_dejavu_sparse_mlp* m, const float* x_dev, int64_t batch,
                                 const kh_dejavu_linear* gate, const kh_dejavu_linear* up,
                                 const kh_dejavu_linear* down, const int64_t* sel_host,
                                 int64_t n_sel, float* y_dev, void* stream);

typedef struct kh_dejavu_sparse_attention kh_dejavu_sparse_attention;

/* SparseAttention::new(config) (attention.rs:9-11): hidden, heads, head_dim. */
int kh_dejavu_sparse_attention_create(int hidden, int num_heads, int head_dim,
                                      kh_dejavu_sparse_attention** out);
int kh_dejavu_sparse_attention_destroy(kh_dejavu_sparse_attention* a);
/* SparseAttention::forward (attention.rs:18-74) for every row of x_dev[batch][hidden]
 * with the same selected heads: y_dev[batch][hidden]. */
int kh_dejavu_sparse_attention_forward(const kh_dejavu_sparse_attention* a, const float* x_dev,
                                       int64_t batch, const kh_dejavu_linear* q,
                                       const kh_dejavu_linear* k, const kh_dejavu_linear* v,
                                       const kh_dejavu_linear* o, const int64_t* heads_host,
                                       int64_t n_heads, float* y_dev, void* stream);

/* ======================================================================== */
/* Head-sparse decode attention (crates/klearu-llm/src/sparse/sparse_attention.rs) */
/* ======================================================================== */

typedef struct kh_sparse_attn kh_sparse_attn;

/* Both kinds hold exactly the rows KvCache (model/kv_cache.rs:5-48) would hold.
 * KH_KV_BF16 (default): rows loaded by kh_sparse_attn_load_cache whose values
 *   are all BF16 values (a BF16 checkpoint's prefill) are stored as BF16, half
 *   the bytes a decode step reads; every other row (appended by a decode step,
 *   loaded from device memory, or loaded with bits BF16 cannot hold) is stored
 *   in f32.  The handle keeps both a BF16 and an f32 array: 6 bytes per cache
 *   element.
 * KH_KV_F32: every row in f32 (4 bytes per cache element). */
#define KH_KV_BF16 0
#define KH_KV_F32 1

/* Attention{q,k,v,o}_proj (model/attention.rs:8-64) + KvCache (model/kv_cache.rs:5-25)
 * + RotaryEmbedding::new(head_dim, max_seq, rope_theta) (model/rope.rs:17-46)
 * for max_batch independent sequences of at most max_seq positions.
 * Weights are BF16 in the reference layout: wq[nh*d][hidden],
 * wk/wv[nkv*d][hidden], wo[hidden][nh*d].  head_dim in {64, 128, 256};
 * hidden a multiple of 8; num_heads a multiple of num_kv_heads (GQA). */
int kh_sparse_attn_create(int hidden, int num_heads, int num_kv_heads, int head_dim,
                          int max_seq, int max_batch, float rope_theta, int kv_dtype,
                          const uint16_t* wq_host, const uint16_t* wk_host,
                          const uint16_t* wv_host, const uint16_t* wo_host, kh_sparse_attn** out);
/* Same with the four weight matrices already in device memory (same layouts). */
int kh_sparse_attn_create_dev(int hidden, int num_heads, int num_kv_heads, int head_dim,
                              int max_seq, int max_batch, float rope_theta, int kv_dtype,
                              const uint16_t* wq_dev, const uint16_t* wk_dev,
                              const uint16_t* wv_dev, const uint16_t* wo_dev,
                              kh_sparse_attn** out);
int kh_sparse_attn_destroy(kh_sparse_attn* a);
/* Fill positions [0, len) of sequence b from f32 host arrays k_host/v_host
 * [nkv][len][d] and set its length (KvCache::append repeated,
 * kv_cache.rs:33-48); the values are kept exactly (BF16 storage only when
 * every value of k and v is a BF16 value).  Synchronous. */
int kh_sparse_attn_load_cache(kh_sparse_attn* a, int64_t b, const float* k_host,
                              const float* v_host, int64_t len);
/* Same from f32 device arrays (e.g. a prefill's K/V), enqueued on `stream`;
 * a KH_KV_BF16 handle checks on the device whether every value is a BF16
 * value and then keeps the rows in BF16, else in f32 (no host round trip). */
int kh_sparse_attn_load_cache_dev(kh_sparse_attn* a, int64_t b, const float* k_dev,
                                  const float* v_dev, int64_t len, void* stream);
/* Copy positions [0, len) of sequence b back as f32 [nkv][len][d]. Synchronous. */
int kh_sparse_attn_read_cache(const kh_sparse_attn* a, int64_t b, float* k_host, float* v_host,
                              int64_t len);
/* KvCache::current_len (kv_cache.rs:27-29) of sequence b (reads the device
 * counter, synchronous). */
int kh_sparse_attn_cache_len(kh_sparse_attn* a, int64_t b, int64_t* len);
/* KvCache::clear (kv_cache.rs:75-78) for every sequence. */
int kh_sparse_attn_clear(kh_sparse_attn* a, void* stream);
/* sparse_attention::forward_sparse (sparse_attention.rs:7-79) for one decode
 * step of sequences 0..batch-1: x_dev[batch][hidden]; RoPE positions
 * pos_dev[batch] (int64; NULL = each sequence's current length, the usual
 * decode position); heads_dev[batch][n_heads] int32 selected heads per token
 * (ids outside [0, num_heads) are skipped as at :48-50; a repeated id adds
 * its head output again, as the reference's += does).  Projects K/V for every
 * kv head and appends them (:39), projects Q and runs softmax attention for
 * the selected heads only, and runs o_proj over the selected heads' columns
 * only.  out_dev[batch][hidden] is written (accumulate = 0) or added to.
 * Returns KH_ERR_CAPACITY when a sequence's cache is full (the reference
 * panics, kv_cache.rs:36).  Mutates the cache. */
int kh_sparse_attn_forward(kh_sparse_attn* a, const float* x_dev, int64_t batch,
                           const int64_t* pos_dev, const int32_t* heads_dev, int n_heads,
                           float* out_dev, int accumulate, void* stream);

/* One decode step (batch 1, sequence 0) of the attention half of a sparse
 * decoder layer as SparseModel::forward_decode_sparse runs it
 * (crates/klearu-llm/src/sparse/mod.rs:56-112):
 *   norm = RmsNorm(hidden) (model/rms_norm.rs:43-64, weight norm_w, eps);
 *   heads = predictor.select_top_k(norm, k) (PredictorStore::predict_heads,
 *           sparse/predictor_store.rs:38-45; ascending ids into heads_dev[k]);
 *   hidden += sparse_attention::forward_sparse(norm, position = cache length, heads).
 * The norm is applied inside the predictor and q/k/v kernels, bit-identical to
 * the reference's (sequential sum of squares); norm_ws_dev (>= 1 float,
 * device) receives the row's scale 1/rms.  Chains with kh_dejavu_mlp_block
 * into a full decoder layer.  Requires predictor input_dim == hidden,
 * output_dim == num_heads, hidden a multiple of 64 and at most 4096.  Returns
 * KH_ERR_CAPACITY when the cache is full. */
int kh_dejavu_attn_block(const kh_predictor* p, kh_sparse_attn* a, float* hidden_dev,
                         const float* norm_w_dev, float eps, int k, int32_t* heads_dev,
                         float* norm_ws_dev, void* stream);
/* kh_dejavu_attn_block for sequences 0..batch-1, one decode step each
 * (sparse/mod.rs:56-112 per token; the reference decodes a batch one token at
 * a time): hidden_dev[batch][hidden] in place, heads_dev[batch][k] (ascending
 * per row), norm_ws_dev[batch] the rows' RmsNorm scales.  Each row's norm and
 * head selection are bit-identical to the reference's; layer 2 of the head
 * predictor and the top k run inside the q/k/v projection.  batch 1 is
 * kh_dejavu_attn_block.  Requires, beyond kh_dejavu_attn_block's limits,
 * hidden a multiple of 1024, at most 64 heads and a head predictor with at
 * most 128 hidden units (else KH_ERR_UNSUPPORTED: use kh_rmsnorm,
 * kh_predictor_select_top_k and kh_sparse_attn_forward). */
int kh_dejavu_attn_block_batch(const kh_predictor* p, kh_sparse_attn* a, float* hidden_dev,
                               int64_t batch, const float* norm_w_dev, float eps, int k,
                               int32_t* heads_dev, float* norm_ws_dev, void* stream);

/* ======================================================================== */
/* On-disk formats: safetensors weights and predictor JSON files            */
/* ======================================================================== */

/* Host-only calls except the *_create_from_* / load / save ones, which build
 * or read device handles. */
typedef struct kh_safetensors kh_safetensors;

#define KH_DT_F32 0
#define KH_DT_F16 1
#define KH_DT_BF16 2

/* SafeTensorsFile::open (crates/klearu-llm/src/weight/safetensors.rs:37-113):
 * memory-maps `path` and parses its header.  `path` may also be a model
 * directory: every *.safetensors file in it is opened in sorted path order
 * (weight/loader.rs:30-49), a later file's tensor shadowing an earlier one of
 * the same name.  A dtype other than F32 / F16 / BF16 fails the open
 * (KH_ERR_UNSUPPORTED, as LlmError::UnsupportedDtype). */
int kh_safetensors_open(const char* path, kh_safetensors** out);
int kh_safetensors_close(kh_safetensors* st);
/* Number of tensors, and the name of tensor i in sorted name order (NUL-
 * terminated into buf[cap]; KH_ERR_CAPACITY if it does not fit). */
int kh_safetensors_count(const kh_safetensors* st, int64_t* n);
int kh_safetensors_name(const kh_safetensors* st, int64_t i, char* buf, int64_t cap);
/* TensorInfo (safetensors.rs:7-14): dtype (KH_DT_*), ndim, and the first
 * min(ndim, max_dims) extents into shape (may be NULL). */
int kh_safetensors_info(const kh_safetensors* st, const char* name, int* dtype, int* ndim,
                        int64_t* shape, int max_dims);
/* tensor_to_f32 (safetensors.rs:135-159): the tensor's n elements converted
 * exactly to f32.  n must equal the element count, and the tensor's bytes must
 * lie in the file and hold exactly that many elements (KH_ERR_ARG otherwise,
 * the reference's "data out of bounds"). */
int kh_safetensors_read_f32(const kh_safetensors* st, const char* name, float* out_host, int64_t n);
/* tensor_data (safetensors.rs:119-133): the tensor's raw little-endian bytes. */
int kh_safetensors_read_raw(const kh_safetensors* st, const char* name, void* out_host,
                            int64_t bytes);
/* The Mlp of decoder layer `layer` (model/mlp.rs:6-21) straight from the
 * file: {prefix}layers.{layer}.mlp.{gate,up,down}_proj.weight with prefix
 * "model.", "model.language_model." or "" (weight/name_map.rs:36-98); hidden
 * and intermediate come from gate_proj's shape.  BF16 tensors are uploaded as
 * they are; F32 / F16 ones only when every value is a BF16 value
 * (KH_ERR_UNSUPPORTED otherwise: the kernels keep BF16 weights).  Equivalent
 * to kh_sparse_ffn_create on the same bits. */
int kh_sparse_ffn_create_from_safetensors(const kh_safetensors* st, int layer, int max_batch,
                                          kh_sparse_ffn** out);
/* The attention of decoder layer `layer` from self_attn.{q,k,v,o}_proj.weight
 * (same naming and dtype rules); hidden comes from q_proj's shape, the head
 * geometry from the model config (config.rs).  Equivalent to
 * kh_sparse_attn_create on the same bits. */
int kh_sparse_attn_create_from_safetensors(const kh_safetensors* st, int layer, int num_heads,
                                           int num_kv_heads, int head_dim, int max_seq,
                                           int max_batch, float rope_theta, int kv_dtype,
                                           kh_sparse_attn** out);

/* SparsityPredictor::load (crates/klearu-dejavu/src/predictor/mlp_predictor.rs:94-98):
 * the serde JSON object {w1: [[f32; input]; hidden], b1, w2: [[f32; hidden];
 * output], b2, input_dim, hidden_dim, output_dim}, fields in any order.  Each
 * number becomes the f32 nearest to the f64 nearest to its decimal, as
 * serde_json reads an f32.  The dims must agree with the arrays (KH_ERR_ARG). */
int kh_predictor_load(const char* path, kh_predictor** out);
/* The same parse into host arrays.  The dims are always written; each array
 * pointer may be NULL (to query the dims first). */
int kh_predictor_read_json(const char* path, int* input_dim, int* hidden_dim, int* output_dim,
                           float* w1_host, float* b1_host, float* w2_host, float* b2_host);
/* SparsityPredictor::save (mlp_predictor.rs:87-92): the same object from host
 * arrays, each f32 as its shortest round-trip decimal in serde_json's spelling
 * ("1.0", "0.25", "1e-7"); non-finite values are rejected (serde_json would
 * write null, which its reader then rejects). */
int kh_predictor_write_json(const char* path, int input_dim, int hidden_dim, int output_dim,
                            const float* w1_host, const float* b1_host, const float* w2_host,
                            const float* b2_host);
/* kh_predictor_write_json of a predictor handle's weights (synchronous). */
int kh_predictor_save(const kh_predictor* p, const char* path);

/* LibSvmDataset (crates/klearu-core/src/data/libsvm.rs:31-183): a LibSVM /
 * extreme-classification text file (`l1,l2,... idx:val ...` per line) parsed
 * on the host as the reference parses it: blank and '#' lines skipped, an
 * inline '#' token ends a line, 1-based indices detected and shifted (no
 * index 0 anywhere and the smallest index 1), indices >= feature_dim clamped
 * to feature_dim - 1, each example's pairs sorted by index with repeated
 * indices summed (SparseVector::from_pairs).  Parse errors return KH_ERR_ARG
 * with "line N: ..." as the reference's messages (:125-175). */
typedef struct kh_libsvm kh_libsvm;
int kh_libsvm_load(const char* path, int64_t feature_dim, int64_t num_labels, kh_libsvm** out);
/* load_from_reader over an in-memory buffer of `len` bytes. */
int kh_libsvm_parse(const char* data, int64_t len, int64_t feature_dim, int64_t num_labels,
                    kh_libsvm** out);
int kh_libsvm_free(kh_libsvm* ds);
/* Examples, stored feature entries, labels in total, feature_dim, num_labels
 * (any pointer may be NULL). */
int kh_libsvm_dims(const kh_libsvm* ds, int64_t* n, int64_t* nnz, int64_t* n_labels,
                   int64_t* feature_dim, int64_t* num_labels);
/* Host copies: features as CSR off[n+1] / idx[nnz] / val[nnz] and labels as
 * CSR label_off[n+1] / labels[n_labels] (any pointer may be NULL). */
int kh_libsvm_copy(const kh_libsvm* ds, int64_t* off, uint32_t* idx, float* val,
                   int64_t* label_off, uint32_t* labels);
/* Examples [row0, row0 + rows) as device CSR (offsets from 0), the layout
 * kh_slide_network_train_step_sparse and the *_sparse entry points read.
 * Synchronous. */
int kh_libsvm_upload(const kh_libsvm* ds, int64_t row0, int64_t rows, int64_t* off_dev,
                     uint32_t* idx_dev, float* val_dev, void* stream);
/* The handle's dims, and its weights copied back to host arrays w1[hidden][input],
 * b1[hidden], w2[output][hidden], b2[output] (synchronous). */
int kh_predictor_dims(const kh_predictor* p, int* input_dim, int* hidden_dim, int* output_dim);
int kh_predictor_weights(const kh_predictor* p, float* w1_host, float* b1_host, float* w2_host,
                         float* b2_host);

/* ======================================================================== */
/* Measurement helper (no counterpart in the reference)                     */
/* ======================================================================== */

/* Reads `bytes` (a positive multiple of 16) of src_dev with 16-byte loads
 * from `blocks` blocks of 256 threads: the achievable HBM read bandwidth that
 * bench.py reports next to each roofline fraction.  sink_dev ([blocks]
 * uint32) is written only to keep the loads alive (in practice never). */
int kh_stream_read(const void* src_dev, int64_t bytes, uint32_t* sink_dev, int blocks, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KLEARU_HIP_H */
