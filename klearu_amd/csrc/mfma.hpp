// mfma.hpp -- BF16 matrix-core helpers shared by the batched FFN gate/up and
// the batched attention projections (gfx950, v_mfma_f32_16x16x32_bf16).
//
// Operand layout of v_mfma_f32_16x16x32_bf16 as these kernels use it: lane l
// holds A[l % 16][(l / 16) * 8 + i] and B[(l / 16) * 8 + i][l % 16] for
// i = 0..7, and receives C[(l / 16) * 4 + q][l % 16] for q = 0..3.  Any
// permutation of k applied to both operands leaves the product unchanged.
// Activations x are split into two BF16 terms (x = hi + lo + r,
// |r| <= 2^-17 |x|) so that products with BF16 weights keep f32 accuracy.
#pragma once

#include "common.hpp"

namespace kh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 kh_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float kh_f32x4;

constexpr int kMfSplit = 4;   // waves sharing one 16-row group (k quarters)
constexpr int kMfWaves = 8;   // 2 row groups of 16 per block
constexpr int kMfDepth = 4;   // k-steps of loads in flight per wave

__device__ __forceinline__ kh_bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(kh_bf16x8, v);
}

// x [batch][H] f32 -> hi, lo [16][H] BF16 bits; rows >= batch are zero.
// (A template, so that each translation unit including this header keeps its own copy.)
template <int Unused = 0>
__global__ void xsplit_kernel(const float* __restrict__ x, int batch, int H,
                              uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 16LL * H) return;
  const float v = i / H < batch ? x[i] : 0.0f;
  const uint16_t h = f32_to_bf16(v);
  hi[i] = h;
  lo[i] = f32_to_bf16(v - bf16_to_f32(h));  // exact difference
}

}  // namespace kh
