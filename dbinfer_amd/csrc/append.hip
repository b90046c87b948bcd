// Append kernels: one launch writes n consecutive positions of one layer and
// leaves the storage exactly as n sequential KVCache::append calls would
// (model.cpp:357-404).
//
// The int8 arithmetic (quant.hpp) is bit-exact with the reference; codes are
// stored as signed bytes in the granule layout of kv_internal.hpp.
#include "kv_internal.hpp"
#include "quant.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;

// In a batch, a ring row is overwritten by row p + W when that row is in the
// same batch; only the last writer of each slot stores (sequential result).
__device__ __forceinline__ bool ring_row_final(int p, int end, int s, int W) {
  return p < s || p + W >= end;
}

// fp32 copy into dense slot pos or ring slot slot_for(pos) (model.cpp:386-402).
__global__ __launch_bounds__(kThreads) void append_f32_kernel(KvGeom g, float* kst, float* vst,
                                                              int layer, int pos0, int n,
                                                              const float* __restrict__ k,
                                                              const float* __restrict__ v) {
  const int P = g.nkv * g.hd;
  const size_t total = static_cast<size_t>(n) * P;
  for (size_t idx = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; idx < total;
       idx += static_cast<size_t>(gridDim.x) * kThreads) {
    const int r = static_cast<int>(idx / P);
    const int c = static_cast<int>(idx % P);
    const int p = pos0 + r;
    int slot = p;
    if (g.ring) {
      if (!ring_row_final(p, pos0 + n, g.n_sink, g.window)) continue;
      slot = slot_for(p, g.n_sink, g.window);
    }
    const int kh = c / g.hd, i = c % g.hd;
    const size_t hb = (static_cast<size_t>(layer) * g.nkv + kh) * head_elems(g);
    kst[hb + k_off(g, slot, i)] = k[idx];
    vst[hb + v_off(g, slot, i)] = v[idx];
  }
}

// Ring int8: quant_head of K and V per kv head into slot_for(pos)
// (model.cpp:386-396). One lane per element, 32 lanes per block.
__global__ __launch_bounds__(kThreads) void append_i8_ring_kernel(KvGeom g, KvStore s, int layer,
                                                                  int pos0, int n,
                                                                  const float* __restrict__ k,
                                                                  const float* __restrict__ v) {
  const int P = g.nkv * g.hd;
  const size_t blocks = static_cast<size_t>(n) * g.nkv * g.nb;
  const size_t bidx = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) / kBlock;
  const int t = threadIdx.x % kBlock;
  if (bidx >= blocks) return;  // whole 32-lane groups leave together
  const int b = static_cast<int>(bidx % g.nb);
  const int kh = static_cast<int>((bidx / g.nb) % g.nkv);
  const int r = static_cast<int>(bidx / (static_cast<size_t>(g.nb) * g.nkv));
  const int p = pos0 + r;
  const int i = b * kBlock + t;
  const bool in = i < g.hd;
  const size_t src = static_cast<size_t>(r) * P + kh * g.hd + i;
  const float kx = in ? k[src] : 0.0f;
  const float vx = in ? v[src] : 0.0f;
  float ks, vs;
  const int8_t kc = quant_lane(kx, &ks);
  const int8_t vc = quant_lane(vx, &vs);
  if (!ring_row_final(p, pos0 + n, g.n_sink, g.window)) return;
  const int slot = slot_for(p, g.n_sink, g.window);
  const size_t head = static_cast<size_t>(layer) * g.nkv + kh;
  const size_t row = head * g.capg + slot;
  if (in) {
    s.k8[head * head_elems(g) + k_off(g, slot, i)] = kc;
    s.v8[head * head_elems(g) + v_off(g, slot, i)] = vc;
  }
  if (t == 0) {
    s.k_scale[row * g.nb + b] = ks;
    s.v_scale[row * g.nb + b] = vs;
  }
}

// Dense int8 key side (model.cpp:358-384, requantize_kgroup :329-355) of a
// batch [pos0, pos0 + n): one thread per (32-token group, channel). The
// result is that of n sequential appends: a group ends requantized over its
// raw rows [0, within] that are not sinks, with within the batch's last row
// in the group. Those rows come from the batch, or, before pos0 in the first
// group, from the staging rows k_raw left by earlier appends (which keeps the
// reference's staging-row aliasing after a rollback). Groups are
// independent; the staging rows are rewritten afterwards
// (append_i8_kraw_kernel), so every reader here sees them as they were.
__global__ __launch_bounds__(kThreads) void append_i8_kgroup_kernel(KvGeom g, KvStore s, int layer,
                                                                    int pos0, int n,
                                                                    const float* __restrict__ k) {
  const int P = g.nkv * g.hd;
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= P) return;
  const int kh = c / g.hd, i = c % g.hd;
  const int grp = pos0 / kKGroup + static_cast<int>(blockIdx.y);
  const int first = grp * kKGroup, end = pos0 + n;
  const int within = min(end - 1, first + kKGroup - 1) - first;
  const float* raw = s.k_raw + static_cast<size_t>(layer) * kKGroup * P + c;
  const size_t head = static_cast<size_t>(layer) * g.nkv + kh;
  float x[kKGroup];
  float mx = 0.0f;
#pragma unroll
  for (int w = 0; w < kKGroup; ++w) {
    const int p = first + w;  // uniform over the block
    x[w] = w > within ? 0.0f
                      : (p >= pos0 ? k[static_cast<size_t>(p - pos0) * P + c]
                                   : raw[static_cast<size_t>(w) * P]);
    if (w <= within && p >= g.n_sink) mx = max_f(mx, fabsf(x[w]));
  }
  const float sc = mx / 127.0f;
  s.k_scale[(head * g.ngroups + grp) * g.hd + i] = sc;
  const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
#pragma unroll
  for (int w = 0; w < kKGroup; ++w)
    if (w <= within && first + w >= g.n_sink)
      s.k8[head * head_elems(g) + k_off(g, first + w, i)] = quant_code(x[w], inv);
}

// The staging rows after the batch: k_raw[w] holds the batch's last row p
// with p % 32 == w (n sequential appends each copy k into k_raw[p % 32]).
__global__ __launch_bounds__(kThreads) void append_i8_kraw_kernel(KvGeom g, KvStore s, int layer,
                                                                  int pos0, int n,
                                                                  const float* __restrict__ k) {
  const int P = g.nkv * g.hd;
  const size_t idx = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (idx >= static_cast<size_t>(kKGroup) * P) return;
  const int w = static_cast<int>(idx / P), c = static_cast<int>(idx % P);
  const int last = pos0 + n - 1;
  const int p = last - (((last - w) % kKGroup) + kKGroup) % kKGroup;
  if (p >= pos0)
    s.k_raw[static_cast<size_t>(layer) * kKGroup * P + idx] = k[static_cast<size_t>(p - pos0) * P + c];
}

// Dense int8 value side (model.cpp:366-384), one lane per element, 32 lanes
// per (row, kv head, block): fp32 sink copy of K and V for pos < n_sink, else
// quant_head of V.
__global__ __launch_bounds__(kThreads) void append_i8_dense_v_kernel(KvGeom g, KvStore s, int layer,
                                                                     int pos0, int n,
                                                                     const float* __restrict__ k,
                                                                     const float* __restrict__ v) {
  const int P = g.nkv * g.hd;
  const size_t blocks = static_cast<size_t>(n) * g.nkv * g.nb;
  const size_t bidx = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) / kBlock;
  const int t = threadIdx.x % kBlock;
  if (bidx >= blocks) return;  // whole 32-lane groups leave together
  const int b = static_cast<int>(bidx % g.nb);
  const int kh = static_cast<int>((bidx / g.nb) % g.nkv);
  const int r = static_cast<int>(bidx / (static_cast<size_t>(g.nb) * g.nkv));
  const int p = pos0 + r;
  const int i = b * kBlock + t;
  const bool in = i < g.hd;
  const size_t src = static_cast<size_t>(r) * P + kh * g.hd + i;
  const size_t head = static_cast<size_t>(layer) * g.nkv + kh;
  const float vx = in ? v[src] : 0.0f;
  if (p < g.n_sink) {  // uniform over the 32-lane group
    if (in) {
      const size_t dst = (head * g.n_sink + p) * g.hd + i;
      s.k_sink[dst] = k[src];
      s.v_sink[dst] = vx;
    }
    return;
  }
  float vs;
  const int8_t vc = quant_lane(vx, &vs);
  if (in) s.v8[head * head_elems(g) + v_off(g, p, i)] = vc;
  if (t == 0) s.v_scale[(head * g.capg + p) * g.nb + b] = vs;
}

int grid_for(size_t work) {
  const size_t blocks = (work + kThreads - 1) / kThreads;
  return static_cast<int>(blocks < 65536 ? (blocks == 0 ? 1 : blocks) : 65536);
}

// [L][len][nkv][hd] <-> the head-major K (is_k) or V store
template <typename T>
__global__ __launch_bounds__(kThreads) void prefix_pack_kernel(KvGeom g, const T* store, T* dst,
                                                               int len, int unpack, int is_k) {
  const size_t P = static_cast<size_t>(g.nkv) * g.hd;
  const size_t total = static_cast<size_t>(g.n_layers) * len * P;
  for (size_t idx = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; idx < total;
       idx += static_cast<size_t>(gridDim.x) * kThreads) {
    const size_t l = idx / (len * P);
    const size_t rem = idx % (len * P);
    const size_t p = rem / P;
    const size_t kh = (rem % P) / g.hd;
    const size_t i = rem % g.hd;
    const size_t st = (l * g.nkv + kh) * head_elems(g) +
                      (is_k ? k_off(g, static_cast<int>(p), static_cast<int>(i))
                            : v_off(g, static_cast<int>(p), static_cast<int>(i)));
    if (unpack)
      const_cast<T*>(store)[st] = dst[idx];
    else
      dst[idx] = store[st];
  }
}

// Row-major per-head arrays: store [L][nkv][dev_rows][inner] <-> file
// [L][rows][nkv][inner], the first `rows` rows of every head.
__global__ __launch_bounds__(kThreads) void rows_pack_kernel(const float* store, float* file,
                                                             int n_layers, int nkv, int dev_rows,
                                                             int rows, int inner, int unpack) {
  const size_t per_layer = static_cast<size_t>(rows) * nkv * inner;
  const size_t total = static_cast<size_t>(n_layers) * per_layer;
  for (size_t idx = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; idx < total;
       idx += static_cast<size_t>(gridDim.x) * kThreads) {
    const size_t l = idx / per_layer;
    const size_t rem = idx % per_layer;
    const size_t r = rem / (static_cast<size_t>(nkv) * inner);
    const size_t kh = (rem / inner) % nkv;
    const size_t i = rem % inner;
    const size_t st = ((l * nkv + kh) * dev_rows + r) * inner + i;
    if (unpack)
      const_cast<float*>(store)[st] = file[idx];
    else
      file[idx] = store[st];
  }
}

}  // namespace

hipError_t launch_append(const KvGeom& g, const KvStore& s, int layer, int pos0, int n,
                         const float* k, const float* v, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const size_t P = static_cast<size_t>(g.nkv) * g.hd;
  if (!g.int8) {
    hipLaunchKernelGGL(append_f32_kernel, dim3(grid_for(n * P)), dim3(kThreads), 0, st, g, s.k,
                       s.v, layer, pos0, n, k, v);
  } else if (g.ring) {
    const size_t lanes = static_cast<size_t>(n) * g.nkv * g.nb * kBlock;
    hipLaunchKernelGGL(append_i8_ring_kernel, dim3((lanes + kThreads - 1) / kThreads),
                       dim3(kThreads), 0, st, g, s, layer, pos0, n, k, v);
  } else {
    const int n_groups = (pos0 + n - 1) / kKGroup - pos0 / kKGroup + 1;
    if (n_groups > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(append_i8_kgroup_kernel,
                       dim3(static_cast<unsigned>((P + kThreads - 1) / kThreads), n_groups),
                       dim3(kThreads), 0, st, g, s, layer, pos0, n, k);
    hipLaunchKernelGGL(append_i8_kraw_kernel, dim3(grid_for(kKGroup * P)), dim3(kThreads), 0, st, g,
                       s, layer, pos0, n, k);
    const size_t vwork = static_cast<size_t>(n) * g.nkv * g.nb * kBlock;
    hipLaunchKernelGGL(append_i8_dense_v_kernel, dim3((vwork + kThreads - 1) / kThreads),
                       dim3(kThreads), 0, st, g, s, layer, pos0, n, k, v);
  }
  return hipGetLastError();
}

hipError_t launch_prefix_pack(const KvGeom& g, const float* src_store, float* dst, int len,
                              bool is_k, hipStream_t st) {
  const size_t total = static_cast<size_t>(g.n_layers) * len * g.nkv * g.hd;
  hipLaunchKernelGGL(prefix_pack_kernel<float>, dim3(grid_for(total)), dim3(kThreads), 0, st, g,
                     src_store, dst, len, 0, is_k ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_prefix_unpack(const KvGeom& g, const float* src, float* dst_store, int len,
                                bool is_k, hipStream_t st) {
  const size_t total = static_cast<size_t>(g.n_layers) * len * g.nkv * g.hd;
  hipLaunchKernelGGL(prefix_pack_kernel<float>, dim3(grid_for(total)), dim3(kThreads), 0, st, g,
                     dst_store, const_cast<float*>(src), len, 1, is_k ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_prefix_codes(const KvGeom& g, int8_t* store, int8_t* file, int len, bool is_k,
                               bool unpack, hipStream_t st) {
  const size_t total = static_cast<size_t>(g.n_layers) * len * g.nkv * g.hd;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(prefix_pack_kernel<uint8_t>, dim3(grid_for(total)), dim3(kThreads), 0, st,
                     g, reinterpret_cast<const uint8_t*>(store),
                     reinterpret_cast<uint8_t*>(file), len, unpack ? 1 : 0, is_k ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_rows_pack(float* store, float* file, int n_layers, int nkv, int dev_rows,
                            int rows, int inner, bool unpack, hipStream_t st) {
  const size_t total = static_cast<size_t>(n_layers) * rows * nkv * inner;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(rows_pack_kernel, dim3(grid_for(total)), dim3(kThreads), 0, st, store, file,
                     n_layers, nkv, dev_rows, rows, inner, unpack ? 1 : 0);
  return hipGetLastError();
}

}  // namespace dbi
