// dejavu_layer.hip -- the klearu-dejavu transformer layer's sparse MLP and
// sparse attention (f32 weights with bias) on the GPU (gfx950).
//
// Replaces Linear::forward / forward_sparse
// (crates/klearu-dejavu/src/transformer/mod.rs:114-134), SparseMlp::forward
// (crates/klearu-dejavu/src/mlp.rs:23-58) and SparseAttention::forward
// (crates/klearu-dejavu/src/attention.rs:18-74).
//
// Every output is bit-identical to the reference: each one is a sequential f32
// sum of rounded products in the reference's order, owned by one thread.
//   Linear rows     one thread per (token, output row): -0.0 + w[r][0]*x[0] + ...
//                   then + bias[r].  Weights are stored transposed, WT[in][out],
//                   so the threads of a wave read adjacent floats of one WT row
//                   at every step while the input value is shared.
//   SparseMlp       gate and up chains of a selected neuron in one thread,
//                   h = silu(g) * u; then one thread per (token, output j) adds
//                   WT_down[sel[a]][j] * h[a] for every selected a with h != 0,
//                   in selection order from +0.0, then the bias.
//   SparseAttention q/k/v rows of the selected heads scattered into zeroed
//                   [heads*head_dim] vectors, one thread per (token, selected
//                   head) for the sigmoid score and the scaled v, then o_proj
//                   over the whole (zero-filled) vector like Linear::forward.
// Index lists arrive from the host (the reference's &[usize]), are checked
// there (an out-of-range index is the reference's panic) and are uploaded to
// the handle's scratch; the upload is waited for, so the caller's list may be
// freed on return and the kernels stay queued behind it.
#include <vector>

#include "common.hpp"

struct kh_dejavu_linear {
  int in_f = 0, out_f = 0;
  float* wt = nullptr;    // [in_f][out_f]
  float* bias = nullptr;  // [out_f]
  mutable kh::StreamWs ws;  // forward_sparse row list, per stream
};

struct kh_dejavu_sparse_mlp {
  int hidden = 0, inter = 0;
  mutable kh::StreamWs ws;  // selected neurons and their activations, per stream
};

struct kh_dejavu_sparse_attention {
  int hidden = 0, num_heads = 0, head_dim = 0;
  mutable kh::StreamWs ws;  // row lists and head vectors, per stream
};

namespace kh {

constexpr int kDlThreads = 256;

__global__ __launch_bounds__(kDlThreads) void dl_rows_kernel(
    const float* __restrict__ wt, int in_f, int out_f, const float* __restrict__ bias,
    const float* __restrict__ x, int64_t ldx, int64_t batch, const int64_t* __restrict__ rows,
    int64_t nrows, float* __restrict__ y, int64_t ldy, int scatter) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= batch * nrows) return;
  const int64_t b = gid / nrows, a = gid - b * nrows;
  const int64_t r = rows ? rows[a] : a;
  const float* xb = x + b * ldx;
  float s = -0.0f;
  for (int j = 0; j < in_f; ++j) s = __fadd_rn(s, __fmul_rn(wt[(int64_t)j * out_f + r], xb[j]));
  y[b * ldy + (scatter ? r : a)] = __fadd_rn(s, bias[r]);
}

__global__ __launch_bounds__(kDlThreads) void dl_gateup_kernel(
    const float* __restrict__ wg, const float* __restrict__ bg, const float* __restrict__ wu,
    const float* __restrict__ bu, int hidden, int inter, const float* __restrict__ x,
    int64_t batch, const int64_t* __restrict__ sel, int64_t n, float* __restrict__ h) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= batch * n) return;
  const int64_t b = gid / n, a = gid - b * n;
  const int64_t r = sel[a];
  const float* xb = x + b * hidden;
  float g = -0.0f, u = -0.0f;
  for (int j = 0; j < hidden; ++j) {
    const float xj = xb[j];
    g = __fadd_rn(g, __fmul_rn(wg[(int64_t)j * inter + r], xj));
    u = __fadd_rn(u, __fmul_rn(wu[(int64_t)j * inter + r], xj));
  }
  g = __fadd_rn(g, bg[r]);
  u = __fadd_rn(u, bu[r]);
  h[gid] = __fmul_rn(silu_ref(g), u);
}

__global__ __launch_bounds__(kDlThreads) void dl_down_kernel(
    const float* __restrict__ wdt, const float* __restrict__ bd, int hidden,
    const float* __restrict__ h, int64_t batch, const int64_t* __restrict__ sel, int64_t n,
    float* __restrict__ y) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= batch * hidden) return;
  const int64_t b = gid / hidden;
  const int j = (int)(gid - b * hidden);
  const float* hb = h + b * n;
  float s = 0.0f;
  for (int64_t a = 0; a < n; ++a) {
    const float v = hb[a];
    if (v != 0.0f) s = __fadd_rn(s, __fmul_rn(wdt[sel[a] * hidden + j], v));
  }
  y[gid] = __fadd_rn(s, bd[j]);
}

__global__ void dl_fill_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// q, k, v, att: [batch][qd]; one thread per (token, selected head).
__global__ __launch_bounds__(kDlThreads) void dl_head_score_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ att, int64_t qd, int head_dim, int64_t batch,
    const int64_t* __restrict__ heads, int64_t n_heads, float scale) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= batch * n_heads) return;
  const int64_t b = gid / n_heads, a = gid - b * n_heads;
  const int64_t st = b * qd + heads[a] * head_dim;
  float s = -0.0f;
  for (int d = 0; d < head_dim; ++d) s = __fadd_rn(s, __fmul_rn(q[st + d], k[st + d]));
  s = __fdiv_rn(s, scale);
  const float sc = sigmoid_ref(s);
  for (int d = 0; d < head_dim; ++d) att[st + d] = __fmul_rn(v[st + d], sc);
}

static unsigned grid_for(int64_t threads) {
  return (unsigned)((threads + kDlThreads - 1) / kDlThreads);
}

// Checks idx_host[0..n) against [0, bound) and uploads it to slot 0 of the
// stream's workspace w.
static int upload_indices(WsSet* w, const int64_t* idx_host, int64_t n, int64_t bound,
                          const char* what, hipStream_t st, const int64_t** out) {
  for (int64_t a = 0; a < n; ++a)
    KH_CHECK_ARG(idx_host[a] >= 0 && idx_host[a] < bound,
                 "%s index %lld out of range (%lld)", what, (long long)idx_host[a],
                 (long long)bound);
  int64_t* d = static_cast<int64_t*>(w->get(0, sizeof(int64_t) * (size_t)(n > 0 ? n : 1)));
  if (!d) return KH_ERR_ALLOC;
  if (n > 0) {
    KH_HIP(hipMemcpyAsync(d, idx_host, sizeof(int64_t) * (size_t)n, hipMemcpyHostToDevice, st));
    KH_HIP(hipStreamSynchronize(st));
  }
  *out = d;
  return KH_OK;
}

static int rows_launch(const kh_dejavu_linear* l, const float* x, int64_t ldx, int64_t batch,
                       const int64_t* rows, int64_t nrows, float* y, int64_t ldy, int scatter,
                       hipStream_t st) {
  if (batch * nrows == 0) return KH_OK;
  hipLaunchKernelGGL(dl_rows_kernel, dim3(grid_for(batch * nrows)), dim3(kDlThreads), 0, st,
                     l->wt, l->in_f, l->out_f, l->bias, x, ldx, batch, rows, nrows, y, ldy,
                     scatter);
  KH_LAUNCHED();
  return KH_OK;
}

static int fill_zero(float* p, int64_t n, hipStream_t st) {
  if (n == 0) return KH_OK;
  hipLaunchKernelGGL(dl_fill_kernel, dim3(grid_for(n)), dim3(kDlThreads), 0, st, p, n);
  KH_LAUNCHED();
  return KH_OK;
}

}  // namespace kh

using namespace kh;

extern "C" int kh_dejavu_linear_create(int in_features, int out_features, const float* w_host,
                                       const float* b_host, kh_dejavu_linear** out) {
  KH_CHECK_ARG(out && w_host && b_host, "null argument");
  KH_CHECK_ARG(in_features > 0 && out_features > 0, "bad shape (in %d out %d)", in_features,
               out_features);
  *out = nullptr;
  const size_t n = (size_t)in_features * (size_t)out_features;
  std::vector<float> wt(n);
  for (int r = 0; r < out_features; ++r)
    for (int j = 0; j < in_features; ++j)
      wt[(size_t)j * out_features + r] = w_host[(size_t)r * in_features + j];
  auto* l = new kh_dejavu_linear;
  l->in_f = in_features;
  l->out_f = out_features;
  l->wt = static_cast<float*>(dev_alloc(n * sizeof(float)));
  l->bias = static_cast<float*>(dev_alloc((size_t)out_features * sizeof(float)));
  if (!l->wt || !l->bias) {
    dev_free(l->wt);
    dev_free(l->bias);
    delete l;
    return KH_ERR_ALLOC;
  }
  hipError_t e = hipMemcpy(l->wt, wt.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(l->bias, b_host, (size_t)out_features * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    set_error("hipMemcpy failed: %s", hipGetErrorString(e));
    dev_free(l->wt);
    dev_free(l->bias);
    delete l;
    return KH_ERR_HIP;
  }
  *out = l;
  return KH_OK;
}

extern "C" int kh_dejavu_linear_destroy(kh_dejavu_linear* l) {
  if (!l) return KH_OK;
  dev_free(l->wt);
  dev_free(l->bias);
  delete l;
  return KH_OK;
}

extern "C" int kh_dejavu_linear_forward(const kh_dejavu_linear* l, const float* x_dev,
                                        int64_t batch, float* y_dev, void* stream) {
  KH_CHECK_ARG(l && x_dev && y_dev, "null argument");
  KH_CHECK_ARG(batch >= 0, "bad batch");
  return rows_launch(l, x_dev, l->in_f, batch, nullptr, l->out_f, y_dev, l->out_f, 0,
                     as_stream(stream));
}

extern "C" int kh_dejavu_linear_forward_sparse(const kh_dejavu_linear* l, const float* x_dev,
                                               int64_t batch, const int64_t* idx_host,
                                               int64_t n_idx, float* y_dev, void* stream) {
  KH_CHECK_ARG(l && x_dev && y_dev && (idx_host || n_idx == 0), "null argument");
  KH_CHECK_ARG(batch >= 0 && n_idx >= 0, "bad shape");
  if (batch * n_idx == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  const int64_t* rows = nullptr;
  int rc = upload_indices(l->ws.get(st), idx_host, n_idx, l->out_f, "row", st, &rows);
  if (rc != KH_OK) return rc;
  return rows_launch(l, x_dev, l->in_f, batch, rows, n_idx, y_dev, n_idx, 0, st);
}

extern "C" int kh_dejavu_sparse_mlp_create(int hidden, int inter, kh_dejavu_sparse_mlp** out) {
  KH_CHECK_ARG(out, "null argument");
  KH_CHECK_ARG(hidden > 0 && inter > 0, "bad shape");
  auto* m = new kh_dejavu_sparse_mlp;
  m->hidden = hidden;
  m->inter = inter;
  *out = m;
  return KH_OK;
}

extern "C" int kh_dejavu_sparse_mlp_destroy(kh_dejavu_sparse_mlp* m) {
  delete m;
  return KH_OK;
}

extern "C" int kh_dejavu_sparse_mlp_forward(const kh_dejavu_sparse_mlp* m, const float* x_dev,
                                            int64_t batch, const kh_dejavu_linear* gate,
                                            const kh_dejavu_linear* up,
                                            const kh_dejavu_linear* down, const int64_t* sel_host,
                                            int64_t n_sel, float* y_dev, void* stream) {
  KH_CHECK_ARG(m && gate && up && down && x_dev && y_dev && (sel_host || n_sel == 0),
               "null argument");
  KH_CHECK_ARG(batch >= 0 && n_sel >= 0, "bad shape");
  const int H = m->hidden, I = m->inter;
  KH_CHECK_ARG(gate->in_f == H && gate->out_f == I && up->in_f == H && up->out_f == I &&
                   down->in_f == I && down->out_f == H,
               "projection shapes do not match hidden %d / intermediate %d", H, I);
  if (batch == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  const int64_t* sel = nullptr;
  int rc = upload_indices(m->ws.get(st), sel_host, n_sel, I, "neuron", st, &sel);
  if (rc != KH_OK) return rc;
  float* h = static_cast<float*>(m->ws.get(st)->get(1, sizeof(float) * (size_t)(batch * n_sel + 1)));
  if (!h) return KH_ERR_ALLOC;
  if (batch * n_sel > 0) {
    hipLaunchKernelGGL(dl_gateup_kernel, dim3(grid_for(batch * n_sel)), dim3(kDlThreads), 0, st,
                       gate->wt, gate->bias, up->wt, up->bias, H, I, x_dev, batch, sel, n_sel, h);
    KH_LAUNCHED();
  }
  hipLaunchKernelGGL(dl_down_kernel, dim3(grid_for(batch * H)), dim3(kDlThreads), 0, st, down->wt,
                     down->bias, H, h, batch, sel, n_sel, y_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_dejavu_sparse_attention_create(int hidden, int num_heads, int head_dim,
                                                 kh_dejavu_sparse_attention** out) {
  KH_CHECK_ARG(out, "null argument");
  KH_CHECK_ARG(hidden > 0 && num_heads > 0 && head_dim > 0, "bad shape");
  auto* a = new kh_dejavu_sparse_attention;
  a->hidden = hidden;
  a->num_heads = num_heads;
  a->head_dim = head_dim;
  *out = a;
  return KH_OK;
}

extern "C" int kh_dejavu_sparse_attention_destroy(kh_dejavu_sparse_attention* a) {
  delete a;
  return KH_OK;
}

extern "C" int kh_dejavu_sparse_attention_forward(
    const kh_dejavu_sparse_attention* a, const float* x_dev, int64_t batch, const kh_dejavu_linear* q,
    const kh_dejavu_linear* k, const kh_dejavu_linear* v, const kh_dejavu_linear* o,
    const int64_t* heads_host, int64_t n_heads, float* y_dev, void* stream) {
  KH_CHECK_ARG(a && q && k && v && o && x_dev && y_dev && (heads_host || n_heads == 0),
               "null argument");
  KH_CHECK_ARG(batch >= 0 && n_heads >= 0, "bad shape");
  const int H = a->hidden, hd = a->head_dim;
  const int64_t qd = (int64_t)a->num_heads * hd;
  KH_CHECK_ARG(q->in_f == H && k->in_f == H && v->in_f == H && q->out_f == qd &&
                   k->out_f == qd && v->out_f == qd && o->in_f == qd && o->out_f == H,
               "projection shapes do not match hidden %d / %d heads x %d", H, a->num_heads, hd);
  if (batch == 0) return KH_OK;
  hipStream_t st = as_stream(stream);
  for (int64_t i = 0; i < n_heads; ++i)
    KH_CHECK_ARG(heads_host[i] >= 0 && heads_host[i] < a->num_heads,
                 "head index %lld out of range (%d)", (long long)heads_host[i], a->num_heads);
  // index list: the selected heads, then the q/k/v rows of each selected head
  std::vector<int64_t> lists((size_t)(n_heads + n_heads * hd));
  for (int64_t i = 0; i < n_heads; ++i) {
    lists[(size_t)i] = heads_host[i];
    for (int d = 0; d < hd; ++d) lists[(size_t)(n_heads + i * hd + d)] = heads_host[i] * hd + d;
  }
  const int64_t* dl = nullptr;
  int rc = upload_indices(a->ws.get(st), lists.data(), (int64_t)lists.size(), qd, "row", st, &dl);
  if (rc != KH_OK) return rc;
  float* buf = static_cast<float*>(a->ws.get(st)->get(1, sizeof(float) * (size_t)(4 * batch * qd)));
  if (!buf) return KH_ERR_ALLOC;
  float *qv = buf, *kv = buf + batch * qd, *vv = buf + 2 * batch * qd, *att = buf + 3 * batch * qd;
  if ((rc = fill_zero(buf, 4 * batch * qd, st)) != KH_OK) return rc;
  const int64_t* rows = dl + n_heads;
  const int64_t nrows = n_heads * hd;
  if ((rc = rows_launch(q, x_dev, H, batch, rows, nrows, qv, qd, 1, st)) != KH_OK) return rc;
  if ((rc = rows_launch(k, x_dev, H, batch, rows, nrows, kv, qd, 1, st)) != KH_OK) return rc;
  if ((rc = rows_launch(v, x_dev, H, batch, rows, nrows, vv, qd, 1, st)) != KH_OK) return rc;
  if (batch * n_heads > 0) {
    hipLaunchKernelGGL(dl_head_score_kernel, dim3(grid_for(batch * n_heads)), dim3(kDlThreads), 0,
                       st, qv, kv, vv, att, qd, hd, batch, dl, n_heads, sqrtf((float)hd));
    KH_LAUNCHED();
  }
  return rows_launch(o, att, qd, batch, nullptr, H, y_dev, H, 0, st);
}
