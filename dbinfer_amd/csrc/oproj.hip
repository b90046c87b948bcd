// The step after attention in decode_layer (model.cpp:773-774): the output
// projection of the attention row and the residual add,
//   proj = W_o · attn   (tensor::matvec_quant, [dim][in] row-major weights)
//   x[o] += proj[o]
// for unquantized weights: fp32 (tensor::matvec, matmul.cpp:36-43) and f16
// (tensor::matvec_f16, matmul.cpp:45-54; every f16 weight converts exactly to
// fp32 and is fused-multiply-added). The GGUF block formats (Q8_0, Q4_K, ...)
// are not served.
//
// One wave per output row: each lane accumulates its share of the row with
// fused multiply-adds, the wave sums the lanes, and lane 0 adds the result to
// the residual (two roundings, as proj[o] then x[o] + proj[o]). The weights
// are read once, 16 bytes per lane per load with every load of a row issued
// before the first product; the attention row (in floats) is re-read by every
// wave from the caches. HBM-bound: dim * in * sizeof(weight) bytes per call.
// The reduction order differs from the reference's sequential sum, so results
// agree to the rounding of a dot product, not bit for bit.
#include "kv_internal.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

struct OprojArgs {
  const void* w;      // [dim][in], fp32 or f16
  const float* attn;  // [in]
  float* x;           // [dim], residual, updated in place
  int dim, in;
};

__device__ inline float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// elements per 16-byte load: 4 fp32 or 8 f16
template <bool F16>
__global__ __launch_bounds__(kThreads) void oproj_kernel(OprojArgs a) {
  constexpr int E = F16 ? 8 : 4;
  constexpr int kBatch = 64 / E;  // 16-byte weight loads per lane in flight (64 weights)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.dim) return;  // wave-uniform
  const size_t rb = static_cast<size_t>(row) * a.in;
  float acc = 0.0f;
  const int units = a.in / E;  // 16-byte weight units of the row
  auto wload = [&](int u) {
    if constexpr (F16)
      return *reinterpret_cast<const uint4*>(static_cast<const _Float16*>(a.w) + rb +
                                             static_cast<size_t>(u) * E);
    else
      return *reinterpret_cast<const uint4*>(static_cast<const float*>(a.w) + rb +
                                             static_cast<size_t>(u) * E);
  };
  // a lane's units are lane, lane + 64, ...; per round kBatch of them, all
  // loads (weights and the matching attention floats) issued before the
  // first product. Past the row's end a load repeats the last unit and its
  // product is skipped.
  for (int u0 = lane; u0 < units; u0 += 64 * kBatch) {
    uint4 wv[kBatch];
    float4 xv[kBatch][E / 4];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int u = min(u0 + 64 * b, units - 1);
      wv[b] = wload(u);
#pragma unroll
      for (int h = 0; h < E / 4; ++h)
        xv[b][h] = *reinterpret_cast<const float4*>(a.attn + static_cast<size_t>(u) * E + 4 * h);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      // branch-free, so the loads above stay ahead of every product
      float t = acc;
      if constexpr (F16) {
        const h8 hw = __builtin_bit_cast(h8, wv[b]);
        const float xs[8] = {xv[b][0].x, xv[b][0].y, xv[b][0].z, xv[b][0].w,
                             xv[b][1].x, xv[b][1].y, xv[b][1].z, xv[b][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) t = __builtin_fmaf(static_cast<float>(hw[e]), xs[e], t);
      } else {
        const float4 w4 = __builtin_bit_cast(float4, wv[b]);
        t = __builtin_fmaf(w4.x, xv[b][0].x, t);
        t = __builtin_fmaf(w4.y, xv[b][0].y, t);
        t = __builtin_fmaf(w4.z, xv[b][0].z, t);
        t = __builtin_fmaf(w4.w, xv[b][0].w, t);
      }
      acc = u0 + 64 * b < units ? t : acc;
    }
  }
  const float proj = wave_sum64(acc);
  if (lane == 0) a.x[row] = a.x[row] + proj;
}

}  // namespace

hipError_t launch_oproj(const OprojCall& c, hipStream_t st) {
  OprojArgs a{};
  a.w = c.w;
  a.attn = c.attn;
  a.x = c.x;
  a.dim = c.dim;
  a.in = c.in;
  const dim3 grid((c.dim + kRowsPerBlock - 1) / kRowsPerBlock);
  if (c.f16)
    hipLaunchKernelGGL(oproj_kernel<true>, grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(oproj_kernel<false>, grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace dbi
