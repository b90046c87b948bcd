// Exact three-part bf16 splits of fp32 values for the bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16), shared by the int8 attention kernels
// (attn_mfma.hpp, attn_i8_rows.hpp) and the fp32 prefill (prefill.hip).
//
// An fp32 value is exactly hi + mid + lo of three bf16 parts: two 8-bit
// truncations, the residual of the first keeps at most 16 significant bits
// and that of the second at most 8. Products of parts are exact in fp32
// (8-bit significands), so a matrix product over parts accumulates exact
// products in fp32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dbi {
namespace {

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float ffrom(uint32_t u) { return __builtin_bit_cast(float, u); }

// the upper halves (bf16) of two fp32 bit patterns, a in the low half
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// x = hi + mid + lo exactly, each part a bf16; parts packed 8 per uint4
__device__ __forceinline__ void split3(const float (&x)[8], uint4 (&part)[3]) {
  uint32_t h[8], m[8], l[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    h[e] = fbits(x[e]) & 0xFFFF0000u;
    const float r1 = x[e] - ffrom(h[e]);
    m[e] = fbits(r1) & 0xFFFF0000u;
    l[e] = fbits(r1 - ffrom(m[e]));
  }
  part[0] = make_uint4(pack_hi(h[0], h[1]), pack_hi(h[2], h[3]), pack_hi(h[4], h[5]),
                       pack_hi(h[6], h[7]));
  part[1] = make_uint4(pack_hi(m[0], m[1]), pack_hi(m[2], m[3]), pack_hi(m[4], m[5]),
                       pack_hi(m[6], m[7]));
  part[2] = make_uint4(pack_hi(l[0], l[1]), pack_hi(l[2], l[3]), pack_hi(l[4], l[5]),
                       pack_hi(l[6], l[7]));
}

// C += A B over 32 k-values, A and B as 8 bf16 per lane
__device__ __forceinline__ f32x4 mfma_bf16(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

}  // namespace
}  // namespace dbi
