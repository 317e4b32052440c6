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

__device__ __forceinline__ kh_bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(kh_bf16x8, v);
}

// Eight f32 activations -> their BF16 hi and lo terms (x = hi + lo + r,
// |r| <= 2^-17 |x|), both rounded to nearest even by v_cvt_pk_bf16_f32; the
// difference x - hi is exact.  Done in registers by the MFMA kernels, so the
// activations are read once as f32 (the same bytes as the two BF16 terms).
typedef __bf16 kh_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf16x2(float p, float q) {
  kh_bf16x2 r;
  r.x = static_cast<__bf16>(p);
  r.y = static_cast<__bf16>(q);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ void split_bf16x8(const float4& a, const float4& b, uint4& hi, uint4& lo) {
  hi = make_uint4(cvt_bf16x2(a.x, a.y), cvt_bf16x2(a.z, a.w), cvt_bf16x2(b.x, b.y), cvt_bf16x2(b.z, b.w));
  lo = make_uint4(cvt_bf16x2(a.x - bf16_lo(hi.x), a.y - bf16_hi(hi.x)),
                  cvt_bf16x2(a.z - bf16_lo(hi.y), a.w - bf16_hi(hi.y)),
                  cvt_bf16x2(b.x - bf16_lo(hi.z), b.y - bf16_hi(hi.z)),
                  cvt_bf16x2(b.z - bf16_lo(hi.w), b.w - bf16_hi(hi.w)));
}

}  // namespace kh
