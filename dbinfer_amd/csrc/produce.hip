// On-device producer of one layer step's attention inputs: the q/k/v bias
// adds and the NeoX rope that the reference applies on the host between the
// projections and the cache (decode: model.cpp:747-763; chunk rows:
// model.cpp:935-954). The roped rows then feed the append and attention
// kernels unchanged, so the keys that int8 append quantizes are exactly the
// keys the reference quantizes.
//
// Arithmetic (bit-exact with the reference):
//  - bias: one fp32 add per element, x + b (model.cpp:747-755);
//  - rope (tensor::rope, ops.cpp:19-38): pair (j, j + hd/2) at position p
//    becomes (float)(a*c - b*s), (float)(b*c + a*s) in fp64, with
//    c = cos(p * inv_j), s = sin(p * inv_j), inv_j = pow(theta, -2j/hd).
//    The cos/sin pairs come from a table the handle builds once on the host
//    with the same libm calls (rope_table below), so the device never
//    evaluates a transcendental; the products and the sum are rounded one by
//    one (no fused multiply-add), as the reference's scalar code does.
// A ring appends un-roped keys and ropes inside attention
// (model.cpp:662-700), so for rings the producer adds the biases only.
#include <cmath>

#include "kv_internal.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;

struct ProduceArgs {
  const float* q;  // [rows][nh*hd]
  const float* k;  // [rows][nkv*hd]
  const float* v;  // [rows][nkv*hd]
  const float* qb;  // [nh*hd] or null
  const float* kb;  // [nkv*hd] or null
  const float* vb;  // [nkv*hd] or null
  float* qo;
  float* ko;
  float* vo;
  const double2* cs;  // [cap][hd/2] (cos, sin); null: no rope
  int rows, nh, nkv, hd, pos0;
};

// fp64 rotation of one NeoX pair, each product and sum rounded on its own
__device__ __forceinline__ float2 rotate(float a, float b, double c, double s) {
#pragma clang fp contract(off)
  const double x = static_cast<double>(a) * c - static_cast<double>(b) * s;
  const double y = static_cast<double>(b) * c + static_cast<double>(a) * s;
  return make_float2(static_cast<float>(x), static_cast<float>(y));
}

// One thread per pair (j, j + hd/2) of one head of one row: the nh query
// heads, then the nkv key heads, then the nkv value heads (bias only).
// Consecutive threads take consecutive j, so each half-row is one coalesced
// access.
__global__ __launch_bounds__(kThreads) void produce_kernel(ProduceArgs a) {
  const int half = a.hd / 2;
  const int heads = a.nh + 2 * a.nkv;
  const size_t per_row = static_cast<size_t>(heads) * half;
  const size_t idx = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (idx >= per_row * a.rows) return;
  const int r = static_cast<int>(idx / per_row);
  const int w = static_cast<int>(idx % per_row);
  const int h = w / half, j = w % half;
  const float* src;
  const float* bias;
  float* dst;
  int hh, row_len;
  if (h < a.nh) {
    hh = h;
    row_len = a.nh * a.hd;
    src = a.q;
    bias = a.qb;
    dst = a.qo;
  } else if (h < a.nh + a.nkv) {
    hh = h - a.nh;
    row_len = a.nkv * a.hd;
    src = a.k;
    bias = a.kb;
    dst = a.ko;
  } else {
    hh = h - a.nh - a.nkv;
    row_len = a.nkv * a.hd;
    src = a.v;
    bias = a.vb;
    dst = a.vo;
  }
  const size_t at = static_cast<size_t>(r) * row_len + static_cast<size_t>(hh) * a.hd + j;
  const int e = hh * a.hd + j;
  float x0 = src[at], x1 = src[at + half];
  if (bias != nullptr) {
    x0 += bias[e];
    x1 += bias[e + half];
  }
  if (a.cs != nullptr && h < a.nh + a.nkv) {
    const double2 t = a.cs[static_cast<size_t>(a.pos0 + r) * half + j];
    const float2 y = rotate(x0, x1, t.x, t.y);
    x0 = y.x;
    x1 = y.y;
  }
  dst[at] = x0;
  dst[at + half] = x1;
}

}  // namespace

bool rope_table_host(const KvGeom& g, float theta, double2* tab) {
  if (g.hd < 2 || g.hd % 2 != 0) return false;
  const int half = g.hd / 2;
  for (int j = 0; j < half; ++j) {
    // ops.cpp:27-30, evaluated per (position, pair) exactly as the reference
    const double inv = std::pow(static_cast<double>(theta),
                                -2.0 * static_cast<double>(j) / static_cast<double>(g.hd));
    for (int p = 0; p < g.cap; ++p) {
      const double ang = static_cast<double>(p) * inv;
      tab[static_cast<size_t>(p) * half + j] = make_double2(std::cos(ang), std::sin(ang));
    }
  }
  return true;
}

hipError_t launch_produce(const KvGeom& g, const double2* rope_dd, const ProduceCall& c,
                          hipStream_t st) {
  ProduceArgs a{};
  a.q = c.q;
  a.k = c.k;
  a.v = c.v;
  a.qb = c.q_bias;
  a.kb = c.k_bias;
  a.vb = c.v_bias;
  a.qo = c.q_out;
  a.ko = c.k_out;
  a.vo = c.v_out;
  a.cs = g.ring ? nullptr : rope_dd;
  a.rows = c.rows;
  a.nh = c.n_heads;
  a.nkv = g.nkv;
  a.hd = g.hd;
  a.pos0 = c.pos0;
  const size_t total = static_cast<size_t>(c.rows) * (c.n_heads + 2 * g.nkv) * (g.hd / 2);
  if (total == 0) return hipSuccess;
  const unsigned blocks = static_cast<unsigned>((total + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(produce_kernel, dim3(blocks), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace dbi
