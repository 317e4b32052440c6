// accel.hip -- klearu-accel entry points on the GPU (gfx950).
//
// Replaces dense_dot_dense_simd / sparse_dot_dense_simd / scatter_add_simd
// (crates/klearu-accel/src/simd/mod.rs:19-109) and the Bf16Weights /
// Bf16FullMode methods (crates/klearu-accel/src/bf16/mod.rs:37-134).
//
// The reference's x86_64 kernels fix a summation order (simd/mod.rs:145-236):
// 16 (dense) or 8 (sparse) FMA lanes over chunks, a fixed horizontal-add tree,
// then a scalar tail.  Here each of those accumulator lanes is a GPU lane
// running the same FMA chain, so the results are bit-identical.  The BF16
// dots are sequential sums and run as one chain per row.
#include "common.hpp"

namespace kh {

// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)), the hsum_avx2 tree (simd/mod.rs:128-141).
__device__ __forceinline__ float hsum8_tree(const float v[8]) {
  const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
  return (s0 + s1) + (s2 + s3);
}

// One 16-lane group per row; 4 rows per wave.
__global__ __launch_bounds__(256) void dense_dot_kernel(const float* __restrict__ a, int64_t rows,
                                                        int64_t lda, const float* __restrict__ b,
                                                        int64_t n, float* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 4;
  const int l = threadIdx.x & 15;
  const bool ok = row < rows;
  const float* ar = a + (ok ? row : 0) * lda;
  const int64_t chunks = n / 16;
  float acc = 0.0f;
  if (ok)
    for (int64_t c = 0; c < chunks; ++c) acc = fmaf(ar[c * 16 + l], b[c * 16 + l], acc);
  const int64_t rs = chunks * 16;
  const bool extra = rs + 8 <= n;
  if (ok && extra && l < 8) acc = fmaf(ar[rs + l], b[rs + l], acc);
  // lane l < 8 holds acc0[l], lane l+8 holds acc1[l]
  const float other = __shfl_down(acc, 8, 16);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __shfl(acc + other, i, 16);
  if (!ok || l != 0) return;
  float sum = hsum8_tree(v);
  for (int64_t i = extra ? rs + 8 : rs; i < n; ++i) sum = __fadd_rn(sum, __fmul_rn(ar[i], b[i]));
  out[row] = sum;
}

__global__ __launch_bounds__(64) void sparse_dot_kernel(const uint32_t* __restrict__ idx,
                                                        const float* __restrict__ val, int64_t nnz,
                                                        const float* __restrict__ dense,
                                                        float* __restrict__ out) {
  const int l = threadIdx.x;
  const int64_t chunks = nnz / 8;
  float acc = 0.0f;
  if (l < 8)
    for (int64_t c = 0; c < chunks; ++c) acc = fmaf(val[c * 8 + l], dense[idx[c * 8 + l]], acc);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __shfl(acc, i, 64);
  if (l != 0) return;
  float sum = hsum8_tree(v);
  for (int64_t i = chunks * 8; i < nnz; ++i) sum = __fadd_rn(sum, __fmul_rn(val[i], dense[idx[i]]));
  *out = sum;
}

// Deterministic scatter-add: chunks of 1024 entries in order; within a chunk
// the first occurrence of each index applies all of that index's updates in
// entry order, one rounded add at a time (as scatter_add_avx2's scalar stores).
__global__ __launch_bounds__(1024) void scatter_add_kernel(const uint32_t* __restrict__ idx,
                                                           const float* __restrict__ val,
                                                           int64_t n, float* __restrict__ dense,
                                                           float scale) {
  __shared__ uint32_t sidx[1024];
  __shared__ float sval[1024];
  for (int64_t c0 = 0; c0 < n; c0 += 1024) {
    const int m = (int)min<int64_t>(1024, n - c0);
    const int t = threadIdx.x;
    if (t < m) {
      sidx[t] = idx[c0 + t];
      sval[t] = __fmul_rn(val[c0 + t], scale);
    }
    __syncthreads();
    if (t < m) {
      const uint32_t me = sidx[t];
      bool first = true;
      for (int j = 0; j < t; ++j)
        if (sidx[j] == me) {
          first = false;
          break;
        }
      if (first) {
        float d = dense[me];
        for (int j = t; j < m; ++j)
          if (sidx[j] == me) d = __fadd_rn(d, sval[j]);
        dense[me] = d;
      }
    }
    __syncthreads();
  }
}

__global__ void bf16_from_f32_kernel(const float* __restrict__ x, uint16_t* __restrict__ o, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) o[i] = f32_to_bf16(x[i]);
}
__global__ void bf16_to_f32_kernel(const uint16_t* __restrict__ x, float* __restrict__ o, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) o[i] = bf16_to_f32(x[i]);
}
__global__ void bf16_update_kernel(uint16_t* __restrict__ w, const float* __restrict__ d, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = f32_to_bf16(__fadd_rn(bf16_to_f32(w[i]), d[i]));
}

// Sequential chain per row (Bf16Weights::dot_f32 iterator sum from -0.0).
__global__ void bf16_dot_f32_kernel(const uint16_t* __restrict__ w, int64_t rows, int64_t ldw,
                                    const float* __restrict__ x, int64_t n, float* __restrict__ o) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const uint16_t* wr = w + r * ldw;
  float s = -0.0f;
  for (int64_t i = 0; i < n; ++i) s = __fadd_rn(s, __fmul_rn(bf16_to_f32(wr[i]), x[i]));
  o[r] = s;
}

__global__ void bf16_full_dot_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                     int64_t n, float* __restrict__ o) {
  if (threadIdx.x != 0) return;
  float s = -0.0f;
  for (int64_t i = 0; i < n; ++i)
    s = __fadd_rn(s, __fmul_rn(bf16_to_f32(a[i]), bf16_to_f32(b[i])));
  *o = s;
}

// f32::exp of every element, the same expf_glibc the predictor, SiLU and
// softmax kernels evaluate.
__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = expf_glibc(x[i]);
}

}  // namespace kh

using namespace kh;

extern "C" int kh_dense_dot_dense(const float* a_dev, int64_t rows, int64_t lda, const float* b_dev,
                                  int64_t n, float* out_dev, void* stream) {
  KH_CHECK_ARG(out_dev && ((a_dev && b_dev) || n == 0 || rows == 0), "null argument");
  KH_CHECK_ARG(rows >= 0 && n >= 0 && lda >= n, "bad shape (rows %lld n %lld lda %lld)",
               (long long)rows, (long long)n, (long long)lda);
  if (rows == 0) return KH_OK;
  const int64_t threads = rows * 16;
  hipLaunchKernelGGL(dense_dot_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     as_stream(stream), a_dev, rows, lda, b_dev, n, out_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_sparse_dot_dense(const uint32_t* idx_dev, const float* val_dev, int64_t nnz,
                                   const float* dense_dev, int64_t dense_len, float* out_dev,
                                   void* stream) {
  KH_CHECK_ARG(out_dev && dense_dev && (nnz == 0 || (idx_dev && val_dev)), "null argument");
  KH_CHECK_ARG(nnz >= 0 && dense_len >= 0, "bad shape");
  hipLaunchKernelGGL(sparse_dot_kernel, dim3(1), dim3(64), 0, as_stream(stream), idx_dev, val_dev,
                     nnz, dense_dev, out_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_scatter_add(const uint32_t* idx_dev, const float* val_dev, int64_t n,
                              float* dense_dev, int64_t dense_len, float scale, void* stream) {
  KH_CHECK_ARG(dense_dev && (n == 0 || (idx_dev && val_dev)), "null argument");
  KH_CHECK_ARG(n >= 0 && dense_len >= 0, "bad shape");
  if (n == 0) return KH_OK;
  hipLaunchKernelGGL(scatter_add_kernel, dim3(1), dim3(1024), 0, as_stream(stream), idx_dev,
                     val_dev, n, dense_dev, scale);
  KH_LAUNCHED();
  return KH_OK;
}

#define KH_ELEMENTWISE(kernel, ...)                                                     \
  do {                                                                                  \
    if (n == 0) return KH_OK;                                                           \
    hipLaunchKernelGGL(kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,         \
                       as_stream(stream), __VA_ARGS__);                                 \
    KH_LAUNCHED();                                                                      \
    return KH_OK;                                                                       \
  } while (0)

extern "C" int kh_bf16_from_f32(const float* x_dev, uint16_t* out_dev, int64_t n, void* stream) {
  KH_CHECK_ARG((x_dev && out_dev) || n == 0, "null argument");
  KH_CHECK_ARG(n >= 0, "bad n");
  KH_ELEMENTWISE(bf16_from_f32_kernel, x_dev, out_dev, n);
}

extern "C" int kh_bf16_to_f32(const uint16_t* x_dev, float* out_dev, int64_t n, void* stream) {
  KH_CHECK_ARG((x_dev && out_dev) || n == 0, "null argument");
  KH_CHECK_ARG(n >= 0, "bad n");
  KH_ELEMENTWISE(bf16_to_f32_kernel, x_dev, out_dev, n);
}

extern "C" int kh_bf16_update_from_f32(uint16_t* w_dev, const float* delta_dev, int64_t n,
                                       void* stream) {
  KH_CHECK_ARG((w_dev && delta_dev) || n == 0, "null argument");
  KH_CHECK_ARG(n >= 0, "bad n");
  KH_ELEMENTWISE(bf16_update_kernel, w_dev, delta_dev, n);
}

extern "C" int kh_bf16_dot_f32(const uint16_t* w_dev, int64_t rows, int64_t ldw,
                               const float* x_dev, int64_t n, float* out_dev, void* stream) {
  KH_CHECK_ARG(out_dev && ((w_dev && x_dev) || n == 0 || rows == 0), "null argument");
  KH_CHECK_ARG(rows >= 0 && n >= 0 && ldw >= n, "bad shape");
  if (rows == 0) return KH_OK;
  hipLaunchKernelGGL(bf16_dot_f32_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0,
                     as_stream(stream), w_dev, rows, ldw, x_dev, n, out_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_bf16_full_dot(const uint16_t* a_dev, const uint16_t* b_dev, int64_t n,
                                float* out_dev, void* stream) {
  KH_CHECK_ARG(out_dev && (n == 0 || (a_dev && b_dev)), "null argument");
  KH_CHECK_ARG(n >= 0, "bad n");
  hipLaunchKernelGGL(bf16_full_dot_kernel, dim3(1), dim3(64), 0, as_stream(stream), a_dev, b_dev,
                     n, out_dev);
  KH_LAUNCHED();
  return KH_OK;
}

extern "C" int kh_expf(const float* x_dev, float* y_dev, int64_t n, void* stream) {
  KH_CHECK_ARG((x_dev && y_dev) || n == 0, "null argument");
  KH_CHECK_ARG(n >= 0 && n <= ((int64_t)1 << 38), "bad n");
  KH_ELEMENTWISE(expf_kernel, x_dev, y_dev, n);
}
