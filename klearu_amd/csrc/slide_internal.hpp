// slide_internal.hpp -- the SLIDE layer handle shared by slide.hip (forward)
// and slide_train.hip (backward, optimizers, network train step).
#pragma once
#include "lsh_internal.hpp"

struct kh_slide_layer {
  int dim = 0, n = 0;
  float* w = nullptr;    // [n][dim]
  float* wtn = nullptr;  // [dim][n]: transposed copy for the non-softmax neuron kernel
  float* bias = nullptr;
  kh_lsh_index* index = nullptr;
  int sampling = 0, top_k = 0, threshold = 0, act = 0;
  mutable kh::StreamWs ws;  // forward scratch per stream
  // optimizer state (Optimizer::create_state per neuron): SGD momentum in
  // st_w1/st_b1; Adam first moments in st_w1/st_b1, second in st_w2/st_b2
  int opt = -1;
  float momentum = 0.0f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
  float* st_w1 = nullptr;
  float* st_w2 = nullptr;
  float* st_b1 = nullptr;
  float* st_b2 = nullptr;
  void free_opt() {
    kh::dev_free(st_w1);
    kh::dev_free(st_w2);
    kh::dev_free(st_b1);
    kh::dev_free(st_b2);
    st_w1 = st_w2 = st_b1 = st_b2 = nullptr;
    opt = -1;
  }
};

namespace kh {

// select_kernel over `batch` rows of query output: active ids per row into
// aids[row*as ..], counts into alen.  count_order: top-k picks listed by count
// descending, then id (the sampler's order) instead of ascending ids.
// clear_dense: per-row dense activations [batch][n] whose previous active
// entries (the aids/alen contents on entry) are zeroed first.
int select_launch(const kh_slide_layer* l, const uint32_t* qids, const uint32_t* qcnt,
                  const int32_t* qlen, int qs, int64_t batch, uint32_t* aids, int as, int32_t* alen,
                  bool count_order, float* clear_dense, hipStream_t st);
// The same with explicit sampling parameters; fallback: an empty pick list
// becomes every neuron 0..num_neurons-1 (layer.rs:82-84).
int select_launch_with(const kh_lsh_index* idx, int sampling, int top_k, int threshold,
                       int num_neurons, const uint32_t* qids, const uint32_t* qcnt,
                       const int32_t* qlen, int qs, int64_t batch, uint32_t* aids, int as,
                       int32_t* alen, bool count_order, float* clear_dense, bool fallback,
                       hipStream_t st);

}  // namespace kh
