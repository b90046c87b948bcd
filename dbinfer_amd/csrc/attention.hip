// GQA attention over the three cache layouts (model.cpp:567-728) and the
// causal chunk rows of decode_layer_chunk (model.cpp:956-981).
//
// Design (CDNA4, wave64):
//  - Grid (split, kv_head, query_row), 8 waves per workgroup. A workgroup
//    streams one contiguous range of key positions of ONE kv head and serves
//    all G = gqa query heads of that head from the same bytes, so K/V cross
//    HBM once per kv head (the reference re-reads them per query head,
//    model.cpp:575-596).
//  - The query group (G x HD floats) is staged once in LDS: roped (ring) and
//    pre-scaled by scale*log2(e) so softmax runs on exp2.
//  - A wave owns 32-position tiles (tile t -> wave t % 8). Inside a tile each
//    "lane row" of LPR = HD/EPL lanes holds EPL elements of one position, a
//    wave covers 64/LPR positions per load and each load instruction reads
//    contiguous 64-128 B runs of a row. All loads of a step (K, V and their
//    scales) are issued before anything waits on them.
//  - Each lane row keeps its own online-softmax state (m, l, o[EPL]); the QK
//    partial dot is reduced over the LPR lanes with DPP row ops; lane rows are
//    merged with DPP row_ror and the gfx950 permlane16/32 swaps (no LDS
//    crossbar); the 8 waves merge through LDS.
//  - Split-K: each split writes (o[G][HD], m[G], l[G]) of its range; a small
//    merge kernel, the next launch on the stream, combines the splits of every
//    (row, query head) with all loads in one round and writes out = o / l.
//    The kernel boundary is the release/acquire: inside one kernel, making
//    one workgroup's stores visible to another across the per-XCD L2 caches
//    takes an agent-scope fence (a whole-L2 writeback) per workgroup.
//  - int8 dense: a tile is exactly one 32-token K group, so the per-channel K
//    scale folds into q once per tile (qs = q * ks, the reference's
//    (q_i * ks_i) * k8_i); V's per-block scale folds into the softmax weight
//    ((w * vs_b) * v8_i). Sinks (pos < n_sink) come from the fp32 arrays.
//  - ring: keys are stored un-roped; each resident key is dequantized (int8:
//    per-block scale) and roped at its cache-relative position from an fp32
//    cos/sin table once per kv head, q at n_res - 1. The lane element mapping
//    keeps dim d and d + HD/2 in one lane, so the rotation is lane-local.
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "kv_internal.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = 32;
constexpr int kMaxSplits = 32;
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
  int cap, ng, n_sink, nkv, n_heads;
  int rows, pos0;
  int ring_nres, ring_s, ring_W, ring_base;
  int nsplit, tiles_per_split;
  float qscale;
};

// ---------------------------------------------------------------------------
// cross-lane helpers

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over the LPR consecutive lanes of a lane row (all lanes get the sum).
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  if constexpr (LPR >= 2) x += dpp<0xB1>(x);    // quad_perm [1,0,3,2]
  if constexpr (LPR >= 4) x += dpp<0x4E>(x);    // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) x += dpp<0x141>(x);   // row_half_mirror
  if constexpr (LPR >= 16) x += dpp<0x140>(x);  // row_mirror
  if constexpr (LPR >= 32) x += __shfl_xor(x, 16);
  if constexpr (LPR >= 64) x += __shfl_xor(x, 32);
  return x;
}

// The gfx950 permlane swaps exchange rows between their two register
// operands. They are emitted through asm: the compiler's builtins for them
// fold the two results into one when both are combined (r0 + r1 compiles to
// r0 + r0). Both operands start as the same value; afterwards {a, b} hold
// {own, partner} in a lane-dependent order, which is all a commutative
// combine needs. The s_nop covers the VALU-write -> permlane-read hazard.
template <int OFF>
__device__ __forceinline__ void swap_pair(float x, float& a, float& b) {
  a = x;
  b = x;
  if constexpr (OFF == 16) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  } else {
    static_assert(OFF == 32, "swap offset");
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  }
}

// Raw v_exp_f32 (2^x). Softmax weights below 2^-126 are far under the
// output tolerance, so the denormal-range handling of exp2f is not needed.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum with the partner lane OFF rows away: OFF 4 is a rotation by 4
// inside each 16-lane DPP row (after the OFF 8 step every lane has met the
// other three lanes of its residue class), 8 is lane ^ 8 (row_ror:8), 16 and
// 32 are lane ^ 16 / lane ^ 32 through the permlane swaps.
template <int OFF>
__device__ __forceinline__ float xmax(float x) {
  if constexpr (OFF == 4) {
    return fmaxf(x, dpp<0x124>(x));
  } else if constexpr (OFF == 8) {
    return fmaxf(x, dpp<0x128>(x));
  } else {
    float a, b;
    swap_pair<OFF>(x, a, b);
    return fmaxf(a, b);
  }
}
template <int OFF>
__device__ __forceinline__ float xsum(float x) {
  if constexpr (OFF == 4) {
    return x + dpp<0x124>(x);
  } else if constexpr (OFF == 8) {
    return x + dpp<0x128>(x);
  } else {
    float a, b;
    swap_pair<OFF>(x, a, b);
    return a + b;
  }
}
// Reductions over the lane rows of a wave (lanes sharing lane % LPR).
template <int LPR>
__device__ __forceinline__ float rows_max(float x) {
  if constexpr (LPR <= 4) x = xmax<4>(x);
  if constexpr (LPR <= 8) x = xmax<8>(x);
  if constexpr (LPR <= 16) x = xmax<16>(x);
  return xmax<32>(x);
}
template <int LPR>
__device__ __forceinline__ float rows_sum(float x) {
  if constexpr (LPR <= 4) x = xsum<4>(x);
  if constexpr (LPR <= 8) x = xsum<8>(x);
  if constexpr (LPR <= 16) x = xsum<16>(x);
  return xsum<32>(x);
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

// int8 code of byte b of w, biased by +128 (w ^ 0x80808080 per dword), as
// float: one v_cvt_f32_ubyteN per element.
__device__ __forceinline__ float u8f(unsigned w, int byte) {
  return static_cast<float>((w >> (8 * byte)) & 0xFFu);
}

// Unpacks CH int8 codes to float, biased by +128 (callers subtract 128 times
// the sum of their multipliers).
template <int CH>
__device__ __forceinline__ void unpack_biased(const typename VecLoad<CH>::T& raw, float* f) {
  constexpr unsigned kFlip = 0x80808080u;
  if constexpr (CH == 4) {
    const unsigned w = raw ^ kFlip;
#pragma unroll
    for (int b = 0; b < 4; ++b) f[b] = u8f(w, b);
  } else if constexpr (CH == 8) {
    const unsigned w0 = raw.x ^ kFlip, w1 = raw.y ^ kFlip;
#pragma unroll
    for (int b = 0; b < 4; ++b) f[b] = u8f(w0, b);
#pragma unroll
    for (int b = 0; b < 4; ++b) f[4 + b] = u8f(w1, b);
  } else {
    const unsigned w[4] = {raw.x ^ kFlip, raw.y ^ kFlip, raw.z ^ kFlip, raw.w ^ kFlip};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) f[4 * j + b] = u8f(w[j], b);
  }
}

template <int HD, int G, int EPL, int KIND>
struct Cfg {
  static constexpr bool kInt8 = (KIND == kI8Dense || KIND == kI8Ring);
  static constexpr bool kRing = (KIND == kF32Ring || KIND == kI8Ring);
  static constexpr int LPR = HD / EPL;         // lanes per position row
  static constexpr int RPW = 64 / LPR;         // positions per wave load
  static constexpr int STEPS = kTile / RPW;    // row steps per tile
  // dims per contiguous chunk: fp32 16 B loads; int8 one load per lane
  // (dense) or two half-head loads (ring, so d and d + HD/2 share a lane)
  static constexpr int CH = !kInt8 ? 4 : (kRing ? EPL / 2 : EPL);
  static constexpr int NCH = EPL / CH;
  // positions per lane per step, from a VGPR budget: q (or q*ks) and o take
  // 2*G*EPL, each in-flight position its raw K/V, scales and rope table
  // (two step buffers are live: the current one and the prefetched next one)
  static constexpr int kBudget = (kInt8 && G >= 7) ? 150 : 170;
  static constexpr int PER_POS = !kInt8 ? 2 * EPL + (kRing ? EPL : 0)
                                        : EPL / 2 + NCH + (kRing ? NCH + EPL : 0);
  static constexpr int FIXED = 2 * G * EPL + (kInt8 ? EPL : 0) + (KIND == kI8Dense ? 2 * EPL : 0);
  static constexpr int UFIT = (kBudget - FIXED) / (2 * PER_POS);
  static constexpr int UMAX = kInt8 ? 4 : 2;
  static constexpr int UCAP = UFIT < 1 ? 1 : (UFIT > UMAX ? UMAX : UFIT);
  static constexpr int UPOW = UCAP >= 4 ? 4 : (UCAP >= 2 ? 2 : 1);
  static constexpr int U = STEPS < UPOW ? STEPS : UPOW;
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
  using VT = typename VecLoad<CH>::T;

  __shared__ float s_q[G][HD];
  __shared__ float s_o[kWaves][G][HD];
  __shared__ float s_ml[kWaves][G][2];
  __shared__ float s_f[G][kWaves];
  __shared__ float s_M[G];
  __shared__ float s_L[G];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane % LPR;
  const int rw = lane / LPR;
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int qrow = blockIdx.z;

  const int nkeys = C::kRing ? P.ring_nres : P.pos0 + qrow + 1;
  const int ntiles = (nkeys + kTile - 1) / kTile;
  const int t_begin = split * P.tiles_per_split;
  const int t_end = min(t_begin + P.tiles_per_split, ntiles);
  const size_t head_rows = static_cast<size_t>(kh) * P.cap;  // first row of this kv head

  // ---- raw loads of one step (U positions per lane row); two buffers so the
  // next step's loads are in flight while the current one is computed
  struct StepBuf {
    VT kraw[U][NCH], vraw[U][NCH];      // int8 codes
    float4 kf4[U][NCH], vf4[U][NCH];    // fp32 rows
    float vsc[U][NCH];                  // int8 V block scales
    float ksc[U][NCH];                  // ring int8 K block scales
    float2 cs[U][(NCH / 2) * CH + 1];   // ring rope cos/sin of each key
    float ksv[EPL];                     // dense int8 per-channel K scales of the tile
    int pu[U];
    bool valid[U];
  };
  StepBuf cur, nxt;

  auto rope_pos = [&](int slot) {
    if (slot < P.ring_s) return slot;
    int r = slot - P.ring_s - P.ring_base;
    r += r < 0 ? P.ring_W : 0;
    return P.ring_s + r;
  };

  auto issue = [&](int tile, int st, StepBuf& b) {
    const int tb = tile * kTile;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = tb + (st + u) * RPW + rw;
      b.valid[u] = p < nkeys && (KIND != kI8Dense || p >= P.n_sink);
      b.pu[u] = min(p, nkeys - 1);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t row = head_rows + b.pu[u];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        if constexpr (!C::kInt8) {
          b.kf4[u][j] = *reinterpret_cast<const float4*>(P.kf + row * HD + C::dim(j, 0, lr));
          b.vf4[u][j] = *reinterpret_cast<const float4*>(P.vf + row * HD + C::dim(j, 0, lr));
        } else {
          b.kraw[u][j] = *reinterpret_cast<const VT*>(P.k8 + row * HD + C::dim(j, 0, lr));
          b.vraw[u][j] = *reinterpret_cast<const VT*>(P.v8 + row * HD + C::dim(j, 0, lr));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t row = head_rows + b.pu[u];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        if constexpr (C::kInt8) b.vsc[u][j] = P.vs[row * NB + C::dim(j, 0, lr) / kBlock];
        if constexpr (KIND == kI8Ring) b.ksc[u][j] = P.ks[row * NB + C::dim(j, 0, lr) / kBlock];
      }
      if constexpr (C::kRing) {
        const float2* cst = P.rope + static_cast<size_t>(rope_pos(b.pu[u])) * (HD / 2);
#pragma unroll
        for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
          for (int t = 0; t < CH; ++t) b.cs[u][j * CH + t] = cst[C::dim(j, t, lr)];
      }
    }
    if constexpr (KIND == kI8Dense) {
      if (st == 0) {
        // per-channel K scales of group `tile` (model.cpp:627-629)
        const float* ksr = P.ks + (static_cast<size_t>(kh) * P.ng + tile) * HD;
#pragma unroll
        for (int j = 0; j < NCH; ++j)
#pragma unroll
          for (int t = 0; t < CH; ++t) b.ksv[j * CH + t] = ksr[C::dim(j, t, lr)];
      }
    }
  };

  // first step's loads go out before the query is staged
  const int first_tile = t_begin + wave;
  if (first_tile < t_end) issue(first_tile, 0, cur);

  // ---- stage the query group in LDS: rope (ring), scale to the log2 domain
  {
    const float* qb = P.q + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;
    if constexpr (C::kRing) {
      const int qpos = P.ring_nres - 1;
      for (int i = threadIdx.x; i < G * (HD / 2); i += kThreads) {
        const int g = i / (HD / 2), d = i % (HD / 2);
        const float2 c = P.rope[static_cast<size_t>(qpos) * (HD / 2) + d];
        const float a = qb[g * HD + d], b = qb[g * HD + d + HD / 2];
        s_q[g][d] = (a * c.x - b * c.y) * P.qscale;
        s_q[g][d + HD / 2] = (b * c.x + a * c.y) * P.qscale;
      }
    } else {
      for (int i = threadIdx.x; i < G * HD; i += kThreads) s_q[i / HD][i % HD] = qb[i] * P.qscale;
    }
  }
  __syncthreads();

  // q of this lane's elements (dense int8 reads it per tile from LDS instead)
  float qv[KIND == kI8Dense ? 1 : G][EPL];
  if constexpr (KIND != kI8Dense) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int t = 0; t < CH; ++t) qv[g][j * CH + t] = s_q[g][C::dim(j, t, lr)];
  }

  // online-softmax state: m is shared by the whole wave (every lane holds the
  // wave maximum), l and o are per lane row and summed over rows at the end.
  // int8 V is unpacked with a +128 bias; corr accumulates the weight each
  // chunk received, and 128 * corr is taken off o once at the end.
  constexpr bool kBias = C::kInt8;
  float m[G], l[G], o[G][EPL];
  float corr[kBias ? G : 1][kBias ? NCH : 1];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kMinit;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.0f;
    if constexpr (kBias)
#pragma unroll
      for (int j = 0; j < NCH; ++j) corr[g][j] = 0.0f;
  }

  // one step: scores s[g][u] of U positions per lane row; vrow(u, vx, mul)
  // yields position u's V elements and per-chunk weight multiplier
  auto update = [&](float (&s)[G][U], auto&& vrow, auto biased_tag) {
    constexpr bool kB = decltype(biased_tag)::value;
    float p[G][U];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[g][u]);
      mx = rows_max<LPR>(mx);
      const float mn = fmaxf(m[g], mx);
      const float alpha = fast_exp2(m[g] - mn);
      m[g] = mn;
      float psum = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[g][u] = fast_exp2(s[g][u] - mn);
        psum += p[g][u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[g][e] *= alpha;
      if constexpr (kBias)
#pragma unroll
        for (int j = 0; j < NCH; ++j) corr[g][j] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vx[EPL];
      float mul[NCH];
      vrow(u, vx, mul);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          const float pw = p[g][u] * mul[j];
          if constexpr (kB) corr[g][j] += pw;
#pragma unroll
          for (int t = 0; t < CH; ++t) o[g][j * CH + t] += pw * vx[j * CH + t];
        }
    }
  };
  using Unbiased = std::integral_constant<bool, false>;
  using Biased = std::integral_constant<bool, kBias>;

  // ---- fp32 sinks of the dense int8 cache (model.cpp:623-626, 640-644)
  if constexpr (KIND == kI8Dense) {
    if (split == 0 && wave == kWaves - 1) {
      const int ns = min(P.n_sink, nkeys);
      for (int p0 = 0; p0 < ns; p0 += RPW) {
        const int p = p0 + rw;
        const bool ok = p < ns;
        const int pl = ok ? p : 0;
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
          for (int j = 0; j < NCH; ++j)
#pragma unroll
            for (int t = 0; t < CH; ++t) acc += s_q[g][C::dim(j, t, lr)] * kx[j * CH + t];
          acc = row_sum<LPR>(acc);
          s[g][0] = ok ? acc : -INFINITY;
#pragma unroll
          for (int u = 1; u < U; ++u) s[g][u] = -INFINITY;
        }
        update(
            s,
            [&](int u, float* x, float* mul) {
#pragma unroll
              for (int e = 0; e < EPL; ++e) x[e] = u == 0 ? vx[e] : 0.0f;
#pragma unroll
              for (int j = 0; j < NCH; ++j) mul[j] = 1.0f;
            },
            Unbiased{});
      }
    }
  }

  // ---- main stream over this wave's tiles of the split
  float qs[KIND == kI8Dense ? G : 1][KIND == kI8Dense ? EPL : 1];
  float qsum[KIND == kI8Dense ? G : 1];
  int tile = first_tile, st = 0;
  while (tile < t_end) {
    // prefetch the next step of this wave
    int ntile = tile, nst = st + U;
    if (nst == C::STEPS) {
      nst = 0;
      ntile += kWaves;
    }
    if (ntile < t_end) issue(ntile, nst, nxt);
    if constexpr (KIND == kI8Dense) {
      if (st == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          qsum[g] = 0.0f;
#pragma unroll
          for (int j = 0; j < NCH; ++j)
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              qs[g][j * CH + t] = s_q[g][C::dim(j, t, lr)] * cur.ksv[j * CH + t];
              qsum[g] += qs[g][j * CH + t];
            }
          qsum[g] *= 128.0f;
        }
      }
    }
    float s[G][U];
    if constexpr (!C::kInt8) {
      float kx[U][EPL];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          kx[u][j * 4 + 0] = cur.kf4[u][j].x;
          kx[u][j * 4 + 1] = cur.kf4[u][j].y;
          kx[u][j * 4 + 2] = cur.kf4[u][j].z;
          kx[u][j * 4 + 3] = cur.kf4[u][j].w;
        }
      if constexpr (C::kRing) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              const float2 c = cur.cs[u][j * CH + t];
              const float a = kx[u][j * CH + t];
              const float b = kx[u][(j + NCH / 2) * CH + t];
              kx[u][j * CH + t] = a * c.x - b * c.y;
              kx[u][(j + NCH / 2) * CH + t] = b * c.x + a * c.y;
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
          s[g][u] = cur.valid[u] ? acc : -INFINITY;
        }
      update(
          s,
          [&](int u, float* x, float* mul) {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
              x[j * 4 + 0] = cur.vf4[u][j].x;
              x[j * 4 + 1] = cur.vf4[u][j].y;
              x[j * 4 + 2] = cur.vf4[u][j].z;
              x[j * 4 + 3] = cur.vf4[u][j].w;
              mul[j] = 1.0f;
            }
          },
          Unbiased{});
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float kx[EPL];
#pragma unroll
        for (int j = 0; j < NCH; ++j) unpack_biased<CH>(cur.kraw[u][j], kx + j * CH);
        if constexpr (KIND == kI8Ring) {
          // dequantize (ks * code, model.cpp:689-690), then rope
#pragma unroll
          for (int j = 0; j < NCH; ++j)
#pragma unroll
            for (int t = 0; t < CH; ++t) kx[j * CH + t] = cur.ksc[u][j] * (kx[j * CH + t] - 128.0f);
#pragma unroll
          for (int j = 0; j < NCH / 2; ++j)
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              const float2 c = cur.cs[u][j * CH + t];
              const float a = kx[j * CH + t];
              const float b = kx[(j + NCH / 2) * CH + t];
              kx[j * CH + t] = a * c.x - b * c.y;
              kx[(j + NCH / 2) * CH + t] = b * c.x + a * c.y;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc;
          if constexpr (KIND == kI8Dense) {
            acc = -qsum[g];
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc += qs[g][e] * kx[e];
          } else {
            acc = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc += qv[g][e] * kx[e];
          }
          acc = row_sum<LPR>(acc);
          s[g][u] = cur.valid[u] ? acc : -INFINITY;
        }
      }
      update(
          s,
          [&](int u, float* x, float* mul) {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
              unpack_biased<CH>(cur.vraw[u][j], x + j * CH);
              mul[j] = cur.vsc[u][j];
            }
          },
          Biased{});
    }
    cur = nxt;
    tile = ntile;
    st = nst;
  }

  // ---- sum the lane rows of this wave (m is already the wave maximum)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = rows_sum<LPR>(l[g]);
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        float x = o[g][j * CH + t];
        if constexpr (kBias) x -= 128.0f * corr[g][j];
        o[g][j * CH + t] = rows_sum<LPR>(x);
      }
  }

  // ---- merge the waves through LDS
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
  if (static_cast<int>(threadIdx.x) < G) {
    const int g = threadIdx.x;
    float M = kMinit;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(s_ml[w][g][0] - M);
      s_f[g][w] = f;
      L += s_ml[w][g][1] * f;
    }
    s_M[g] = M;
    s_L[g] = L;
  }
  __syncthreads();

  const int rec_floats = G * (HD + 2);
  const size_t head_base = static_cast<size_t>(qrow) * P.nkv + kh;
  float* out_base = P.out + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;

  if (P.nsplit == 1) {
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
      const int g = idx / HD, d = idx % HD;
      float O = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) O += s_o[w][g][d] * s_f[g][w];
      out_base[idx] = O / s_L[g];
    }
    return;
  }

  // ---- publish this split's (o[G][HD], m[G], l[G]); merge_kernel, the next
  // launch on the stream, combines the splits (a kernel boundary is the
  // cheapest release/acquire across this part's per-XCD L2 caches)
  float* rec = P.part + (head_base * P.nsplit + split) * rec_floats;
  for (int idx = threadIdx.x; idx < G * HD + 2 * G; idx += kThreads) {
    float v;
    if (idx < G * HD) {
      const int g = idx / HD, d = idx % HD;
      v = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += s_o[w][g][d] * s_f[g][w];
    } else {
      const int r = idx - G * HD;
      v = r < G ? s_M[r] : s_L[r - G];
    }
    rec[idx] = v;
  }
}

// Combines the split partials of one (row, query head): one thread per
// output dim; every split's (m, l, o[d]) is loaded in a single round.
template <int HD>
__global__ __launch_bounds__(HD) void merge_kernel(const float* __restrict__ part,
                                                   float* __restrict__ out, int nkv, int G,
                                                   int nsplit, int n_heads) {
  const int h = blockIdx.x;
  const int row = blockIdx.y;
  const int kh = h / G, g = h % G;
  const int d = threadIdx.x;
  const int rec_floats = G * (HD + 2);
  const float* recs = part + ((static_cast<size_t>(row) * nkv + kh) * nsplit) * rec_floats;
  float mv[kMaxSplits], lv[kMaxSplits], ov[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    if (sp < nsplit) {
      const float* r = recs + static_cast<size_t>(sp) * rec_floats;
      mv[sp] = r[G * HD + g];
      lv[sp] = r[G * HD + G + g];
      ov[sp] = r[g * HD + d];
    } else {
      mv[sp] = kMinit;
      lv[sp] = 0.0f;
      ov[sp] = 0.0f;
    }
  }
  float M = kMinit;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) M = fmaxf(M, mv[sp]);
  float L = 0.0f, O = 0.0f;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    const float w = fast_exp2(mv[sp] - M);
    L += lv[sp] * w;
    O += ov[sp] * w;
  }
  out[(static_cast<size_t>(row) * n_heads + h) * HD + d] = O / L;
}

// ---------------------------------------------------------------------------
// dispatch

// Elements per lane: 16 keeps the lane-row count (and the end-of-wave row
// merge) small; 8 halves the q / o registers where G is large or int8 wants
// more positions in flight.
template <int HD, int G, int KIND>
constexpr int epl_for() {
#ifdef DBI_EPL_RULE
  return DBI_EPL_RULE;
#else
  return (KIND == kI8Dense || KIND == kI8Ring) ? 8 : (G <= 2 ? 16 : 8);
#endif
}

template <int HD, int G, int KIND>
void* kernel_for() {
  return reinterpret_cast<void*>(&attn_kernel<HD, G, epl_for<HD, G, KIND>(), KIND>);
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

int kind_of(const KvGeom& g) { return (g.ring ? 2 : 0) + (g.int8 ? 1 : 0); }

// Workgroups one launch aims for (split-K fan-out: one 8-wave workgroup per
// CU); DBI_ATTN_TARGET_BLOCKS overrides it for tuning sweeps.
int target_blocks() {
  static const int v = [] {
    const char* e = std::getenv("DBI_ATTN_TARGET_BLOCKS");
    const int x = e ? std::atoi(e) : 0;
    return x > 0 ? x : 256;
  }();
  return v;
}

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

size_t attention_workspace_need(const KvGeom& g, const AttnCall& c) {
  int nsplit = 1, tps = 1;
  plan(g, c, &nsplit, &tps);
  const int G = c.n_heads / g.nkv;
  return nsplit > 1 ? static_cast<size_t>(c.rows) * g.nkv * nsplit * G * (g.hd + 2) : 0;
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
  hipError_t e = hipLaunchKernel(fn, dim3(p.nsplit, g.nkv, c.rows), dim3(kThreads), args, 0, st);
  if (e != hipSuccess || p.nsplit == 1) return e;
  if (g.hd == 64)
    hipLaunchKernelGGL(merge_kernel<64>, dim3(c.n_heads, c.rows), dim3(64), 0, st, ws.part, c.out,
                       g.nkv, G, p.nsplit, c.n_heads);
  else
    hipLaunchKernelGGL(merge_kernel<128>, dim3(c.n_heads, c.rows), dim3(128), 0, st, ws.part,
                       c.out, g.nkv, G, p.nsplit, c.n_heads);
  return hipGetLastError();
}

}  // namespace dbi
