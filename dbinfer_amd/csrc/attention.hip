// GQA attention over the three cache layouts (model.cpp:567-728) and the
// causal chunk rows of decode_layer_chunk (model.cpp:956-981).
//
// Design (CDNA4, wave64):
//  - Grid (split, kv_head, query_row). One workgroup of 4 waves streams one
//    contiguous range of key positions of ONE kv head and serves all G = gqa
//    query heads of that head from the same bytes, so K/V cross HBM once per
//    kv head (the reference re-reads them per query head, model.cpp:575-596).
//  - A wave owns 32-position tiles (tile t -> wave t % 4). Inside a tile each
//    "lane row" of LPR = HD/EPL lanes holds EPL elements of one position;
//    a wave covers 64/LPR positions per load, each load instruction reading
//    contiguous 64-128 B runs of a row (coalesced).
//  - q is pre-scaled by scale*log2(e) so softmax is exp2; each lane row keeps
//    its own online-softmax state (m, l, o[EPL]); the QK partial dot is
//    reduced over the LPR lanes with DPP row ops, the per-row states are
//    merged with cross-lane shuffles, the 4 waves through LDS.
//  - Split-K: every split writes (m, l, o[HD]) per query head; the last
//    workgroup of a (row, kv head) to arrive (agent-scope atomic ticket, self-
//    resetting) merges the splits and writes out = o / l.
//  - int8 dense: the tile is exactly one 32-token K group, so the per-channel
//    K scale folds into q once per tile (qs = q * ks, the reference's
//    (q_i * ks_i) * k8_i); V's per-block scale folds into the softmax weight
//    ((w * vs_b) * v8_i). Sinks (pos < n_sink) are read from the fp32 arrays.
//  - ring: keys are stored un-roped; each resident key is dequantized (int8:
//    per-block scale) and roped at its cache-relative position from an fp32
//    cos/sin table once per kv head, and q is roped at n_res - 1. Lane element
//    mapping pairs dim d with d + HD/2 inside the lane, so the rotation needs
//    no cross-lane traffic.
#include <cmath>

#include "kv_internal.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = 32;
constexpr int kMaxSplits = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMinit = -1.0e30f;  // finite: exp2(kMinit - kMinit) == 1, no NaN

enum Kind { kF32Dense = 0, kI8Dense = 1, kF32Ring = 2, kI8Ring = 3 };

struct AttnParams {
  const float* kf;
  const float* vf;
  const int8_t* k8;
  const int8_t* v8;
  const float* ks;
  const float* vs;
  const float* ksink;
  const float* vsink;
  const float2* rope;
  const float* q;
  float* out;
  float* part;
  unsigned* counters;
  int cap, ng, n_sink, nkv, n_heads;
  int rows, pos0;
  int ring_nres, ring_s, ring_W, ring_base;
  int nsplit, tiles_per_split;
  float qscale;
};


template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over the LPR consecutive lanes of a lane row.
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  if constexpr (LPR >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if constexpr (LPR >= 16) x += dpp<0x140>(x); // row_mirror
  if constexpr (LPR >= 32) x += __shfl_xor(x, 16);
  if constexpr (LPR >= 64) x += __shfl_xor(x, 32);
  return x;
}

template <int N>
struct VecLoad;
template <>
struct VecLoad<4> {
  using T = unsigned;
};
template <>
struct VecLoad<8> {
  using T = uint2;
};
template <>
struct VecLoad<16> {
  using T = uint4;
};

__device__ __forceinline__ float i8f(unsigned w, int byte) {
  return static_cast<float>(static_cast<int>(w << (24 - 8 * byte)) >> 24);
}

// Unpacks CH int8 codes to float.
template <int CH>
__device__ __forceinline__ void unpack_i8(const typename VecLoad<CH>::T& raw, float* f) {
  if constexpr (CH == 4) {
#pragma unroll
    for (int b = 0; b < 4; ++b) f[b] = i8f(raw, b);
  } else if constexpr (CH == 8) {
#pragma unroll
    for (int b = 0; b < 4; ++b) f[b] = i8f(raw.x, b);
#pragma unroll
    for (int b = 0; b < 4; ++b) f[4 + b] = i8f(raw.y, b);
  } else {
    const unsigned w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) f[4 * j + b] = i8f(w[j], b);
  }
}

template <int HD, int G, int EPL, int KIND>
struct Cfg {
  static constexpr bool kInt8 = (KIND == kI8Dense || KIND == kI8Ring);
  static constexpr bool kRing = (KIND == kF32Ring || KIND == kI8Ring);
  static constexpr int LPR = HD / EPL;         // lanes per position row
  static constexpr int RPW = 64 / LPR;         // positions per wave load
  static constexpr int STEPS = kTile / RPW;    // row steps per tile
  static constexpr int UMAX = kInt8 ? 4 : 2;   // positions per lane per inner step
  static constexpr int U = STEPS < UMAX ? STEPS : UMAX;
  // dims per contiguous chunk: fp32 16 B loads; int8 one load per lane
  // (dense) or two half-head loads (ring, so d and d + HD/2 share a lane)
  static constexpr int CH = !kInt8 ? 4 : (kRing ? EPL / 2 : EPL);
  static constexpr int NCH = EPL / CH;
  static constexpr int NB = HD / kBlock;
  static_assert(LPR * EPL == HD, "lane mapping");
  static_assert(kTile % RPW == 0 && STEPS % U == 0, "tile mapping");
  static_assert(!kRing || NCH % 2 == 0, "ring pairs d with d + HD/2 in one lane");
  __device__ static constexpr int dim(int j, int t, int lr) { return (j * LPR + lr) * CH + t; }
};

template <int HD, int G, int EPL, int KIND>
__global__ __launch_bounds__(kThreads) void attn_kernel(const AttnParams P) {
  using C = Cfg<HD, G, EPL, KIND>;
  constexpr int LPR = C::LPR, RPW = C::RPW, U = C::U, CH = C::CH, NCH = C::NCH;
  constexpr int NB = C::NB;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane % LPR;
  const int rw = lane / LPR;
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int qrow = blockIdx.z;

  const int nkeys = C::kRing ? P.ring_nres : P.pos0 + qrow + 1;

  // ---- query group of this kv head: roped (ring), scaled to log2 domain
  float qv[G][EPL];
  {
    const float* qb = P.q + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int t = 0; t < CH; ++t) qv[g][j * CH + t] = qb[g * HD + C::dim(j, t, lr)];
    if constexpr (C::kRing) {
      const int qpos = P.ring_nres - 1;
#pragma unroll
      for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          const float2 cs = P.rope[static_cast<size_t>(qpos) * (HD / 2) + C::dim(j, t, lr)];
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float a = qv[g][j * CH + t];
            const float b = qv[g][(j + NCH / 2) * CH + t];
            qv[g][j * CH + t] = a * cs.x - b * cs.y;
            qv[g][(j + NCH / 2) * CH + t] = b * cs.x + a * cs.y;
          }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e) qv[g][e] *= P.qscale;
  }

  float m[G], l[G], o[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kMinit;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.0f;
  }

  // online-softmax update of this lane row with U scores per head
  auto update = [&](float (&s)[G][U], auto&& vval) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[g][u]);
      const float alpha = exp2f(m[g] - mx);
      m[g] = mx;
      float p[U];
      float psum = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u] = exp2f(s[g][u] - mx);
        psum += p[u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float acc = o[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) acc += vval(p, u, e);
        o[g][e] = acc;
      }
    }
  };

  const size_t head_rows = static_cast<size_t>(kh) * P.cap;  // first row of this kv head

  // ---- fp32 sinks of the dense int8 cache (model.cpp:623-626, 640-644)
  if constexpr (KIND == kI8Dense) {
    if (split == 0 && wave == 0) {
      const int ns = min(P.n_sink, nkeys);
      for (int p0 = 0; p0 < ns; p0 += RPW) {
        const int p = p0 + rw;
        const bool valid = p < ns;
        const int pl = valid ? p : 0;
        const float* kr = P.ksink + (static_cast<size_t>(kh) * P.n_sink + pl) * HD;
        const float* vr = P.vsink + (static_cast<size_t>(kh) * P.n_sink + pl) * HD;
        float kx[EPL], vx[EPL];
#pragma unroll
        for (int j = 0; j < NCH; ++j)
#pragma unroll
          for (int t = 0; t < CH; ++t) {
            kx[j * CH + t] = kr[C::dim(j, t, lr)];
            vx[j * CH + t] = vr[C::dim(j, t, lr)];
          }
        float s[G][U];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc = 0.0f;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc += qv[g][e] * kx[e];
          acc = row_sum<LPR>(acc);
          s[g][0] = valid ? acc : -INFINITY;
#pragma unroll
          for (int u = 1; u < U; ++u) s[g][u] = -INFINITY;
        }
        update(s, [&](const float* pw, int u, int e) { return u == 0 ? pw[0] * vx[e] : 0.0f; });
      }
    }
  }

  // ---- main stream over this split's tiles
  const int ntiles = (nkeys + kTile - 1) / kTile;
  const int t_begin = split * P.tiles_per_split;
  const int t_end = min(t_begin + P.tiles_per_split, ntiles);

  for (int tile = t_begin + wave; tile < t_end; tile += kWaves) {
    const int tb = tile * kTile;
    float qs[KIND == kI8Dense ? G : 1][KIND == kI8Dense ? EPL : 1];
    if constexpr (KIND == kI8Dense) {
      // per-channel K scales of group `tile` (model.cpp:627-629)
      const float* ksr = P.ks + (static_cast<size_t>(kh) * P.ng + tile) * HD;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int t = 0; t < CH; ++t) {
          const float ksv = ksr[C::dim(j, t, lr)];
#pragma unroll
          for (int g = 0; g < G; ++g) qs[g][j * CH + t] = qv[g][j * CH + t] * ksv;
        }
    }
#pragma unroll 1
    for (int st = 0; st < C::STEPS; st += U) {
      int pu[U];
      bool valid[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        pu[u] = tb + (st + u) * RPW + rw;
        valid[u] = pu[u] < nkeys && (KIND != kI8Dense || pu[u] >= P.n_sink);
        pu[u] = min(pu[u], nkeys - 1);
      }
      float s[G][U];
      if constexpr (!C::kInt8) {
        float kx[U][EPL], vx[U][EPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float* kr = P.kf + (head_rows + pu[u]) * HD;
          const float* vr = P.vf + (head_rows + pu[u]) * HD;
#pragma unroll
          for (int j = 0; j < NCH; ++j) {
            const float4 a = *reinterpret_cast<const float4*>(kr + C::dim(j, 0, lr));
            const float4 b = *reinterpret_cast<const float4*>(vr + C::dim(j, 0, lr));
            kx[u][j * 4 + 0] = a.x;
            kx[u][j * 4 + 1] = a.y;
            kx[u][j * 4 + 2] = a.z;
            kx[u][j * 4 + 3] = a.w;
            vx[u][j * 4 + 0] = b.x;
            vx[u][j * 4 + 1] = b.y;
            vx[u][j * 4 + 2] = b.z;
            vx[u][j * 4 + 3] = b.w;
          }
        }
        if constexpr (C::kRing) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int slot = pu[u];
            const int rp = slot < P.ring_s ? slot
                                           : P.ring_s + ((slot - P.ring_s - P.ring_base + P.ring_W) %
                                                         P.ring_W);
            const float2* cst = P.rope + static_cast<size_t>(rp) * (HD / 2);
#pragma unroll
            for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
              for (int t = 0; t < CH; ++t) {
                const float2 cs = cst[C::dim(j, t, lr)];
                const float a = kx[u][j * CH + t];
                const float b = kx[u][(j + NCH / 2) * CH + t];
                kx[u][j * CH + t] = a * cs.x - b * cs.y;
                kx[u][(j + NCH / 2) * CH + t] = b * cs.x + a * cs.y;
              }
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc += qv[g][e] * kx[u][e];
            acc = row_sum<LPR>(acc);
            s[g][u] = valid[u] ? acc : -INFINITY;
          }
        update(s, [&](const float* pw, int u, int e) { return pw[u] * vx[u][e]; });
      } else {
        using VT = typename VecLoad<CH>::T;
        VT kraw[U][NCH], vraw[U][NCH];
        float vsc[U][NCH];
        float ksc[U][KIND == kI8Ring ? NCH : 1];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int8_t* kr = P.k8 + (head_rows + pu[u]) * HD;
          const int8_t* vr = P.v8 + (head_rows + pu[u]) * HD;
          const float* vsr = P.vs + (head_rows + pu[u]) * NB;
#pragma unroll
          for (int j = 0; j < NCH; ++j) {
            kraw[u][j] = *reinterpret_cast<const VT*>(kr + C::dim(j, 0, lr));
            vraw[u][j] = *reinterpret_cast<const VT*>(vr + C::dim(j, 0, lr));
            vsc[u][j] = vsr[C::dim(j, 0, lr) / kBlock];
            if constexpr (KIND == kI8Ring)
              ksc[u][j] = P.ks[(head_rows + pu[u]) * NB + C::dim(j, 0, lr) / kBlock];
          }
        }
        if constexpr (KIND == kI8Dense) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float kx[EPL];
#pragma unroll
            for (int j = 0; j < NCH; ++j) unpack_i8<CH>(kraw[u][j], kx + j * CH);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              float acc = 0.0f;
#pragma unroll
              for (int e = 0; e < EPL; ++e) acc += qs[g][e] * kx[e];
              acc = row_sum<LPR>(acc);
              s[g][u] = valid[u] ? acc : -INFINITY;
            }
          }
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float kx[EPL];
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
              unpack_i8<CH>(kraw[u][j], kx + j * CH);
#pragma unroll
              for (int t = 0; t < CH; ++t) kx[j * CH + t] = ksc[u][j] * kx[j * CH + t];
            }
            const int slot = pu[u];
            const int rp = slot < P.ring_s ? slot
                                           : P.ring_s + ((slot - P.ring_s - P.ring_base + P.ring_W) %
                                                         P.ring_W);
            const float2* cst = P.rope + static_cast<size_t>(rp) * (HD / 2);
#pragma unroll
            for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
              for (int t = 0; t < CH; ++t) {
                const float2 cs = cst[C::dim(j, t, lr)];
                const float a = kx[j * CH + t];
                const float b = kx[(j + NCH / 2) * CH + t];
                kx[j * CH + t] = a * cs.x - b * cs.y;
                kx[(j + NCH / 2) * CH + t] = b * cs.x + a * cs.y;
              }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              float acc = 0.0f;
#pragma unroll
              for (int e = 0; e < EPL; ++e) acc += qv[g][e] * kx[e];
              acc = row_sum<LPR>(acc);
              s[g][u] = valid[u] ? acc : -INFINITY;
            }
          }
        }
        float vx[U][EPL];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < NCH; ++j) unpack_i8<CH>(vraw[u][j], vx[u] + j * CH);
        update(s, [&](const float* pw, int u, int e) {
          return (pw[u] * vsc[u][e / CH]) * vx[u][e];
        });
      }
    }
  }

  // ---- merge the lane rows of this wave (all rows end with the wave max)
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off);
      const float lo = __shfl_xor(l[g], off);
      const float mn = fmaxf(m[g], mo);
      const float a = exp2f(m[g] - mn);
      const float b = exp2f(mo - mn);
      l[g] = l[g] * a + lo * b;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float oo = __shfl_xor(o[g][e], off);
        o[g][e] = o[g][e] * a + oo * b;
      }
      m[g] = mn;
    }
  }

  // ---- merge the 4 waves through LDS
  __shared__ float s_o[kWaves][G][HD];
  __shared__ float s_ml[kWaves][G][2];
  __shared__ float s_w[G][kMaxSplits];
  __shared__ unsigned s_ticket;
  if (rw == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int t = 0; t < CH; ++t) s_o[wave][g][C::dim(j, t, lr)] = o[g][j * CH + t];
    if (lr == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_ml[wave][g][0] = m[g];
        s_ml[wave][g][1] = l[g];
      }
    }
  }
  __syncthreads();

  const size_t rec_floats = static_cast<size_t>(G) * (HD + 2);
  const size_t head_base = (static_cast<size_t>(qrow) * P.nkv + kh);
  float* out_base = P.out + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;

  if (P.nsplit == 1) {
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
      const int g = idx / HD, d = idx % HD;
      float M = kMinit;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = exp2f(s_ml[w][g][0] - M);
        L += s_ml[w][g][1] * f;
        O += s_o[w][g][d] * f;
      }
      out_base[static_cast<size_t>(g) * HD + d] = O / L;
    }
    return;
  }

  float* rec = P.part + (head_base * P.nsplit + split) * rec_floats;
  for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
    const int g = idx / HD, d = idx % HD;
    float M = kMinit;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) O += s_o[w][g][d] * exp2f(s_ml[w][g][0] - M);
    rec[idx] = O;
  }
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float M = kMinit;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += s_ml[w][g][1] * exp2f(s_ml[w][g][0] - M);
    rec[G * HD + 2 * g] = M;
    rec[G * HD + 2 * g + 1] = L;
  }

  // publish this split, take a ticket; the last arrival merges all splits
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) s_ticket = atomicAdd(P.counters + head_base, 1u);
  __syncthreads();
  if (s_ticket != static_cast<unsigned>(P.nsplit - 1)) return;
  __threadfence();

  const float* recs = P.part + head_base * P.nsplit * rec_floats;
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float M = kMinit;
    for (int sp = 0; sp < P.nsplit; ++sp) M = fmaxf(M, recs[sp * rec_floats + G * HD + 2 * g]);
    float L = 0.0f;
    for (int sp = 0; sp < P.nsplit; ++sp) {
      const float w = exp2f(recs[sp * rec_floats + G * HD + 2 * g] - M);
      s_w[g][sp] = w;
      L += recs[sp * rec_floats + G * HD + 2 * g + 1] * w;
    }
    const float inv_l = 1.0f / L;
    for (int sp = 0; sp < P.nsplit; ++sp) s_w[g][sp] *= inv_l;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
    const int g = idx / HD;
    float O = 0.0f;
    for (int sp = 0; sp < P.nsplit; ++sp) O += recs[sp * rec_floats + idx] * s_w[g][sp];
    out_base[idx] = O;
  }
  if (threadIdx.x == 0) P.counters[head_base] = 0u;
}

// ---------------------------------------------------------------------------
// dispatch

template <int HD, int G, int KIND>
void* kernel_for() {
  constexpr int EPL = G <= 4 ? 16 : 8;
  return reinterpret_cast<void*>(&attn_kernel<HD, G, EPL, KIND>);
}

template <int HD, int KIND>
void* pick_g(int G) {
  switch (G) {
    case 1: return kernel_for<HD, 1, KIND>();
    case 2: return kernel_for<HD, 2, KIND>();
    case 3: return kernel_for<HD, 3, KIND>();
    case 4: return kernel_for<HD, 4, KIND>();
    case 5: return kernel_for<HD, 5, KIND>();
    case 6: return kernel_for<HD, 6, KIND>();
    case 7: return kernel_for<HD, 7, KIND>();
    case 8: return kernel_for<HD, 8, KIND>();
    default: return nullptr;
  }
}

template <int HD>
void* pick_kind(int kind, int G) {
  switch (kind) {
    case kF32Dense: return pick_g<HD, kF32Dense>(G);
    case kI8Dense: return pick_g<HD, kI8Dense>(G);
    case kF32Ring: return pick_g<HD, kF32Ring>(G);
    case kI8Ring: return pick_g<HD, kI8Ring>(G);
    default: return nullptr;
  }
}

void* pick_kernel(int hd, int kind, int G) {
  if (hd == 64) return pick_kind<64>(kind, G);
  if (hd == 128) return pick_kind<128>(kind, G);
  return nullptr;
}

int kind_of(const KvGeom& g) {
  return (g.ring ? 2 : 0) + (g.int8 ? 1 : 0);
}

int target_blocks() { return 512; }

void plan(const KvGeom& g, const AttnCall& c, int* nsplit, int* tiles_per_split) {
  const int nkeys_max = g.ring ? c.ring.n_res : c.pos0 + c.rows;
  const int ntiles = (nkeys_max + kTile - 1) / kTile;
  const int units = g.nkv * c.rows;
  int want = (target_blocks() + units - 1) / units;
  const int max_by_tiles = (ntiles + kWaves - 1) / kWaves;  // >= one tile per wave
  if (want > max_by_tiles) want = max_by_tiles;
  if (want > kMaxSplits) want = kMaxSplits;
  if (want < 1) want = 1;
  const int tps = (ntiles + want - 1) / want;
  *tiles_per_split = tps;
  *nsplit = (ntiles + tps - 1) / tps;
}

}  // namespace

bool attention_supported(const KvGeom& g, int n_heads) {
  if (n_heads <= 0 || n_heads % g.nkv != 0) return false;
  return pick_kernel(g.hd, kind_of(g), n_heads / g.nkv) != nullptr;
}

void attention_workspace_need(const KvGeom& g, const AttnCall& c, size_t* part_floats,
                              size_t* counters) {
  int nsplit = 1, tps = 1;
  plan(g, c, &nsplit, &tps);
  const int G = c.n_heads / g.nkv;
  *part_floats = nsplit > 1 ? static_cast<size_t>(c.rows) * g.nkv * nsplit * G * (g.hd + 2) : 0;
  *counters = static_cast<size_t>(c.rows) * g.nkv;
}

hipError_t launch_attention(const KvGeom& g, const KvStore& s, Workspace& ws, const AttnCall& c,
                            hipStream_t st) {
  const int G = c.n_heads / g.nkv;
  void* fn = pick_kernel(g.hd, kind_of(g), G);
  if (fn == nullptr) return hipErrorNotSupported;
  AttnParams p{};
  const size_t layer_rows = static_cast<size_t>(c.layer) * g.nkv * g.cap;
  if (!g.int8) {
    p.kf = s.k + layer_rows * g.hd;
    p.vf = s.v + layer_rows * g.hd;
  } else {
    p.k8 = s.k8 + layer_rows * g.hd;
    p.v8 = s.v8 + layer_rows * g.hd;
    p.vs = s.v_scale + layer_rows * g.nb;
    if (g.ring) {
      p.ks = s.k_scale + layer_rows * g.nb;
    } else {
      p.ks = s.k_scale + static_cast<size_t>(c.layer) * g.nkv * g.ngroups * g.hd;
      if (g.n_sink > 0) {
        p.ksink = s.k_sink + static_cast<size_t>(c.layer) * g.nkv * g.n_sink * g.hd;
        p.vsink = s.v_sink + static_cast<size_t>(c.layer) * g.nkv * g.n_sink * g.hd;
      }
    }
  }
  p.rope = s.rope_cs;
  p.q = c.q;
  p.out = c.out;
  p.part = ws.part;
  p.counters = ws.counters;
  p.cap = g.cap;
  p.ng = g.ngroups;
  p.n_sink = g.int8 && !g.ring ? g.n_sink : 0;
  p.nkv = g.nkv;
  p.n_heads = c.n_heads;
  p.rows = c.rows;
  p.pos0 = c.pos0;
  p.ring_nres = c.ring.n_res;
  p.ring_s = c.ring.s;
  p.ring_W = c.ring.W > 0 ? c.ring.W : 1;
  p.ring_base = c.ring.base;
  plan(g, c, &p.nsplit, &p.tiles_per_split);
  p.qscale = c.scale * kLog2e;
  void* args[] = {&p};
  return hipLaunchKernel(fn, dim3(p.nsplit, g.nkv, c.rows), dim3(kThreads), args, 0, st);
}

}  // namespace dbi
