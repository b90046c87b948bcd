// Quantize-on-append arithmetic shared by the append kernels and the fused
// decode step (KVCache::quant_head and requantize_kgroup, model.cpp:303-355).
//
// Bit-exactness rests on three facts: max|x| is order-free (NaN inputs are
// skipped the same way std::max skips them), x / 127.0f and 1.0f / s are IEEE
// correctly rounded divisions (HIP's default, never fast-math), and the code
// is round-half-away of one fp32 product, clamped to [-127, 127].
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dbi {

// std::max(a, b) as the reference calls it: keeps a unless a < b
__device__ __forceinline__ float max_f(float a, float b) { return (a < b) ? b : a; }

// clamp(lround(x * inv), -127, 127) as glibc computes it on x86-64: lround of a
// NaN, an infinity or |x| >= 2^63 yields LONG_MIN, which clamps to -127.
// Branch-free (selects only), so unrolled callers keep their loads batched.
__device__ __forceinline__ int8_t quant_code(float x, float inv) {
  const float r = x * inv;
  const float t = fminf(fmaxf(roundf(r), -127.0f), 127.0f);
  return static_cast<int8_t>(fabsf(r) < 9223372036854775808.0f ? static_cast<int>(t) : -127);
}

// quant_head (model.cpp:303-317) of one block with one lane per element: lanes
// of an aligned 32-lane group hold the block's elements (inactive tail lanes
// pass 0), the block max comes from xor shuffles inside the group. Every lane
// returns its code; the block scale is returned through *scale.
__device__ __forceinline__ int8_t quant_lane(float x, float* scale) {
  float m = fabsf(x);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) m = max_f(m, __shfl_xor(m, off, 32));
  const float s = m / 127.0f;
  *scale = s;
  const float inv = s > 0.0f ? 1.0f / s : 0.0f;
  return quant_code(x, inv);
}


// KVCache::slot_for (model.cpp:321-324)
__device__ __forceinline__ int slot_for(int pos, int s, int W) {
  return pos < s ? pos : s + (pos - s) % W;
}

}  // namespace dbi
