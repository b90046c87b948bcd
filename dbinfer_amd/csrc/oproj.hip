// The unfused matvecs of decode_layer (model.cpp:738-785) and forward's
// lm_head (:915): tensor::matvec_quant ([out][in] row-major weights) of one
// activation row,
//   y[o] = W[o] · x          (q, k, v, gate, up, lm_head)
//   y[o] += W[o] · x         (o_proj and down, the residual adds)
// for fp32 weights (tensor::matvec, matmul.cpp:36-43), f16 weights
// (tensor::matvec_f16, matmul.cpp:45-54; every f16 weight converts exactly to
// fp32 and is fused-multiply-added) and Q8_0 / Q4_0 rows of an odd block
// count (matvec_q8_0_scalar / matvec_q4_0_scalar, matmul.cpp:56-99; the even
// block counts run the fused kernels of matvec.hip). The layer's rmsnorm
// (ops.cpp:7-17) and silu(gate) * up (model.cpp:781-782, ops.cpp:54-56) for
// these unfused paths are here too.
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
#include "quant.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

struct OprojArgs {
  const void* w;      // [dim][in], fp32 or f16
  const float* attn;  // [in]
  float* x;           // [dim]: x[o] += proj (acc) or x[o] = proj
  int dim, in;
  int acc;
};

// the row's result into the output (two roundings with acc, as proj[o] then
// x[o] + proj[o])
__device__ inline void put_row(const OprojArgs& a, int row, float proj) {
  a.x[row] = a.acc ? a.x[row] + proj : proj;
}

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
  if (lane == 0) put_row(a, row, proj);
}

// global-address-space views (the block pointers are computed as integers)
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f4v gf4;

// Rows whose block count is odd (in % 64 == 32), which the pair-layout
// kernels of matvec.hip do not take, run these per-block kernels (unfused:
// the offload composes them with the rmsnorm and silu kernels below).
//
// Q8_0: a block is an f16 scale then 32 int8 codes (34 bytes). Each
// workgroup first quantizes the activation row into LDS with
// quantize_row_q8_0's arithmetic (amax over the block, d = amax / 127,
// id = 1 / d, the stored scale f16(d), codes clamp(lround(x * id), +-127)),
// one thread per block. Then each wave takes kQRows rows; lane l owns blocks
// l, l + 64, ... of a row. Per block the integer dot product is exact
// (v_dot4_i32_i8) and its term is (f16(dw) * f16(dx)) * sumi in fp32, the
// reference's expression; the terms are then summed in a tree. A block's 34
// bytes are read as the 9 aligned dwords around them (the weights start
// 4-byte aligned, so the first of them never precedes the matrix; the last
// can reach 2 bytes past it, inside the same aligned dword).
constexpr int kQBlocks = 2;  // blocks per lane in flight
constexpr int kQRows = 2;    // rows per wave
constexpr int kQStride = 9;  // LDS dwords per activation block: 8 code dwords, the scale

__device__ inline uint32_t pack4(int8_t a, int8_t b, int8_t c, int8_t d) {
  return static_cast<uint32_t>(static_cast<uint8_t>(a)) |
         (static_cast<uint32_t>(static_cast<uint8_t>(b)) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(c)) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(d)) << 24);
}

// The activation row to Q8_0 blocks in LDS (quantize_row_q8_0's arithmetic,
// one thread per block): 8 code dwords, the f16 scale as a float, and (for
// Q4_0) the block's code sum, kQStride4 dwords per block.
constexpr int kQStride4 = 10;
__device__ inline void quantize_act(const float* x, int nbk, uint32_t* s_xq, int stride) {
  for (int b = threadIdx.x; b < nbk; b += kThreads) {
    gf4* xb = (gf4*)(x + static_cast<size_t>(b) * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f4v t = xb[i];
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = max_f(amax, fabsf(v[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int8_t c0 = quant_code(v[4 * i], id), c1 = quant_code(v[4 * i + 1], id);
      const int8_t c2 = quant_code(v[4 * i + 2], id), c3 = quant_code(v[4 * i + 3], id);
      s_xq[b * stride + i] = pack4(c0, c1, c2, c3);
      sum += c0 + c1 + c2 + c3;
    }
    s_xq[b * stride + 8] = __float_as_uint(static_cast<float>(static_cast<_Float16>(d)));
    if (stride > 9) s_xq[b * stride + 9] = static_cast<uint32_t>(sum);
  }
}

__global__ __launch_bounds__(kThreads) void oproj_q8_kernel(OprojArgs a) {
  extern __shared__ uint32_t s_xq[];  // [nbk][kQStride]
  const int nbk = a.in / 32;
  quantize_act(a.attn, nbk, s_xq, kQStride);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * kQRows;
  for (int rr = 0; rr < kQRows; ++rr) {
    const int row = row0 + rr;
    if (row >= a.dim) break;  // wave-uniform
    const uintptr_t wrow =
        reinterpret_cast<uintptr_t>(a.w) + static_cast<size_t>(row) * nbk * 34;
    float acc = 0.0f;
    for (int b0 = lane; b0 < nbk; b0 += 64 * kQBlocks) {
      uint32_t wd[kQBlocks][9];
      uint32_t off[kQBlocks];
#pragma unroll
      for (int q = 0; q < kQBlocks; ++q) {
        const int b = min(b0 + 64 * q, nbk - 1);
        const uintptr_t p = wrow + static_cast<size_t>(b) * 34;
        off[q] = static_cast<uint32_t>(p & 2);
        gu32* base = (gu32*)(p & ~static_cast<uintptr_t>(3));
#pragma unroll
        for (int i = 0; i < 9; ++i) wd[q][i] = base[i];
      }
#pragma unroll
      for (int q = 0; q < kQBlocks; ++q) {
        const int b = min(b0 + 64 * q, nbk - 1);
        const uint32_t* xq = s_xq + b * kQStride;
        const bool hi = off[q] != 0;  // block starts 2 bytes into its first dword
        const uint16_t dbits = static_cast<uint16_t>(hi ? wd[q][0] >> 16 : wd[q][0] & 0xffffu);
        const float dw = static_cast<float>(__builtin_bit_cast(_Float16, dbits));
        int sumi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t wc = hi ? wd[q][i + 1] : ((wd[q][i] >> 16) | (wd[q][i + 1] << 16));
          sumi = __builtin_amdgcn_sdot4(static_cast<int>(wc), static_cast<int>(xq[i]), sumi,
                                        false);
        }
        const float term = (dw * __uint_as_float(xq[8])) * static_cast<float>(sumi);
        acc = b0 + 64 * q < nbk ? acc + term : acc;
      }
    }
    const float proj = wave_sum64(acc);
    if (lane == 0) put_row(a, row, proj);
  }
}

// Q4_0: a block is an f16 scale then 16 bytes of nibbles (18 bytes); element
// j of the block is the low nibble of byte j, element j + 16 its high
// nibble, each minus 8. Per block the integer sum is exact: the nibbles
// (0..15, positive as signed bytes) dot the activation codes with
// v_dot4_i32_i8, minus 8 times the block's code sum; the term is
// (f16(dw) * f16(dx)) * sumi as matvec_q4_0_scalar writes it. A block's 18
// bytes are read as the 5 aligned dwords around them (blocks start 2-byte
// aligned; the last dword can reach 2 bytes past the matrix, inside the
// same aligned dword).
__global__ __launch_bounds__(kThreads) void oproj_q4_kernel(OprojArgs a) {
  extern __shared__ uint32_t s_xq4[];  // [nbk][kQStride4]
  const int nbk = a.in / 32;
  quantize_act(a.attn, nbk, s_xq4, kQStride4);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * kQRows;
  for (int rr = 0; rr < kQRows; ++rr) {
    const int row = row0 + rr;
    if (row >= a.dim) break;  // wave-uniform
    const uintptr_t wrow =
        reinterpret_cast<uintptr_t>(a.w) + static_cast<size_t>(row) * nbk * 18;
    float acc = 0.0f;
    for (int b0 = lane; b0 < nbk; b0 += 64 * kQBlocks) {
      uint32_t wd[kQBlocks][5];
      uint32_t off[kQBlocks];
#pragma unroll
      for (int q = 0; q < kQBlocks; ++q) {
        const int b = min(b0 + 64 * q, nbk - 1);
        const uintptr_t p = wrow + static_cast<size_t>(b) * 18;
        off[q] = static_cast<uint32_t>(p & 2);
        gu32* base = (gu32*)(p & ~static_cast<uintptr_t>(3));
#pragma unroll
        for (int i = 0; i < 5; ++i) wd[q][i] = base[i];
      }
#pragma unroll
      for (int q = 0; q < kQBlocks; ++q) {
        const int b = min(b0 + 64 * q, nbk - 1);
        const uint32_t* xq = s_xq4 + b * kQStride4;
        const bool hi = off[q] != 0;  // block starts 2 bytes into its first dword
        const uint16_t dbits = static_cast<uint16_t>(hi ? wd[q][0] >> 16 : wd[q][0] & 0xffffu);
        const float dw = static_cast<float>(__builtin_bit_cast(_Float16, dbits));
        int sumi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t c = hi ? wd[q][i + 1] : ((wd[q][i] >> 16) | (wd[q][i + 1] << 16));
          const uint32_t lo = c & 0x0F0F0F0Fu, hn = (c >> 4) & 0x0F0F0F0Fu;
          sumi = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(xq[i]), sumi, false);
          sumi = __builtin_amdgcn_sdot4(static_cast<int>(hn), static_cast<int>(xq[4 + i]), sumi,
                                        false);
        }
        sumi -= 8 * static_cast<int>(xq[9]);
        const float term = (dw * __uint_as_float(xq[8])) * static_cast<float>(sumi);
        acc = b0 + 64 * q < nbk ? acc + term : acc;
      }
    }
    const float proj = wave_sum64(acc);
    if (lane == 0) put_row(a, row, proj);
  }
}

// rmsnorm of one row (ops.cpp:7-17): the sum of squares over the workgroup
// (a tree, so it agrees with the reference's sequential sum to a rounding),
// scale = 1 / sqrt(sumsq / dim + eps), out[i] = x[i] * scale * w[i].
constexpr int kNormThreads = 1024;
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* x, const float* w,
                                                               float eps, float* out, int dim) {
  __shared__ float s_part[kNormThreads / 64];
  float ss = 0.0f;
  for (int i = threadIdx.x; i < dim; i += kNormThreads) ss += x[i] * x[i];
  ss = wave_sum64(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
  const float scale = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
  for (int i = threadIdx.x; i < dim; i += kNormThreads) out[i] = x[i] * scale * w[i];
}

// silu(gate) then gate *= up (model.cpp:781-782, ops.cpp:54-56)
__global__ __launch_bounds__(256) void silu_mul_kernel(float* g, const float* u, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float x = g[i];
    g[i] = (x / (1.0f + expf(-x))) * u[i];
  }
}

}  // namespace

hipError_t launch_oproj(const OprojCall& c, hipStream_t st) {
  OprojArgs a{};
  a.w = c.w;
  a.attn = c.attn;
  a.x = c.x;
  a.dim = c.dim;
  a.in = c.in;
  a.acc = c.overwrite ? 0 : 1;
  const dim3 grid((c.dim + kRowsPerBlock - 1) / kRowsPerBlock);
  if (c.q4) {
    const int rows_per_block = kRowsPerBlock * kQRows;
    const size_t lds = static_cast<size_t>(c.in / 32) * kQStride4 * sizeof(uint32_t);
    hipLaunchKernelGGL(oproj_q4_kernel, dim3((c.dim + rows_per_block - 1) / rows_per_block),
                       dim3(kThreads), lds, st, a);
  } else if (c.q8) {
    const int rows_per_block = kRowsPerBlock * kQRows;
    const size_t lds = static_cast<size_t>(c.in / 32) * kQStride * sizeof(uint32_t);
    hipLaunchKernelGGL(oproj_q8_kernel, dim3((c.dim + rows_per_block - 1) / rows_per_block),
                       dim3(kThreads), lds, st, a);
  } else if (c.f16)
    hipLaunchKernelGGL(oproj_kernel<true>, grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(oproj_kernel<false>, grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int dim,
                          hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, st, x, w, eps, out, dim);
  return hipGetLastError();
}

hipError_t launch_silu_mul(float* g, const float* u, int n, hipStream_t st) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, st, g, u, n);
  return hipGetLastError();
}

}  // namespace dbi
