// Causal chunk attention of the dense fp32 cache on the matrix cores: the
// attention loop of decode_layer_chunk (model.cpp:956-981), rows c of a
// chunk at pos0 attending keys [0, pos0 + c], for chunks long enough to
// make QK^T and PV real matrix products (the prefill chunks of config 2).
//
// Design (CDNA4 v_mfma_f32_16x16x4_f32, fp32 in and out, so the result stays
// within the fp32 tolerance of the CPU path):
//  - A workgroup of 4 waves owns 64 query vectors of one kv head: each wave
//    16 vectors (16/G rows x the G query heads sharing the kv head). The
//    workgroup walks its keys in stages of SK keys: the stage's K and V are
//    copied into LDS once, by LDS-direct loads (no registers), and every
//    wave reads its MFMA operands from there. Stages are double-buffered:
//    the next stage's copy is in flight while the current one computes.
//  - Keys can be split over KS workgroups (grid z) to fill the GPU on short
//    chunks; a split writes its unnormalized (o, m, l) and prefill_merge
//    combines them.
//  - S^T = K Q^T: A = K (16 keys x 4 dims), B = Q^T (4 dims x 16 vectors),
//    one instruction per 4 dims, in four independent accumulator chains.
//    Dims are permuted per lane group so that every lane's operands are 16
//    contiguous floats: in instruction (h, s), k-index kk stands for dim
//    16 kk + 64 h + s. The result holds S[vector l % 16][key 4 (l / 16) + v]
//    in lane l.
//  - O^T += V^T P^T: A = V^T (16 dims x 4 keys), B = P^T straight from the S
//    registers (instruction j uses key 4 kk + j, the score lane l already
//    holds). Output tile tt row i stands for dim (hd/16) i + tt, so a lane's
//    V operands are hd/16 contiguous floats per key and its output is hd/4
//    contiguous floats of its vector.
//  - Online softmax per vector (= per lane % 16); the four lane groups
//    holding one vector combine through two xor shuffles.
//  - LDS holds the stage in the cache's own granule layout (kv_internal.hpp),
//    so the copy is a straight contiguous one and the operand offsets are
//    the layout's offsets relative to the stage.
#include <cmath>
#include <type_traits>

#include "kv_internal.hpp"

namespace dbi {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPWaves = 4;
constexpr int kPThreads = 64 * kPWaves;
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kMinitP = -1.0e30f;  // finite: exp2(kMinit - kMinit) == 1

struct PrefillParams {
  const float* kf;  // this layer's K, V: [nkv][capg * hd], granule layout
  const float* vf;
  const float* q;   // [rows][n_heads][hd]
  float* out;       // [rows][n_heads][hd]
  float* part;      // KS > 1: [KS][rows][n_heads][hd + 2] (o unnormalized, m, l)
  int capg, n_heads, rows, pos0, ks;
  float qscale;     // scale * log2(e)
};

// One 16-byte LDS-direct copy per lane: lane l reads src + 16 voff bytes
// (src wave-uniform) and lands at LDS byte address dst + 16 l (dst
// wave-uniform, through m0). Issued as asm, so the compiler does not track
// the copy: it would otherwise wait for every copy in flight (vmcnt 0)
// before each LDS read, the next stage's included, since it cannot tell the
// copy's destination from the buffer being read. Stage arrival is waited for
// explicitly (s_waitcnt vmcnt, then the barrier).
// m0 is saved and restored around the copy (the register is reserved to
// the compiler).
__device__ __forceinline__ void lds_copy16(const float* src, uint32_t voff, uint32_t dst) {
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %1\n\ts_mov_b32 m0, %0"
      : "=&s"(keep)
      : "s"(src), "v"(voff), "s"(dst)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const float* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const float*)p));
}

// Workgroup barrier that waits for this wave's LDS accesses only. The
// compiler's __syncthreads also waits for every vector memory load (vmcnt 0)
// when LDS-direct copies are in flight, which would drain the prefetched
// stages at every stage; stage arrival is waited for explicitly instead.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float4 lds4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// Lane-group exchanges of the softmax through the gfx950 permlane swaps
// (VALU, no LDS round trip like a bpermute). After v_permlane16_swap of
// (x, x), a lane holds its own x and the x of lane ^ 16 (one in each
// register); v_permlane32_swap does the same for lane ^ 32. Emitted through
// asm: the compiler's builtins fold the two results into one when both are
// used.
__device__ __forceinline__ float xmax16(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float xmax32(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float xsum16(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float xsum32(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}

// Stage buffers hold the cache's granule layout with its 16-byte units
// permuted inside every aligned run of 16 units: unit u sits at swz_u(u) =
// u ^ m(u), m's bits 0-2 the parities of u >> 3 under the masks 62, 53, 15
// and its bit 3 the parity of u >> 4 under 54. The masks were picked by
// exhaustive check of every K and V operand read of both head dims: each
// read (64 lanes x 16 bytes) then hits distinct banks in every group of 8
// lanes (32 banks) and of 16 lanes (64 banks). The map is linear over GF(2),
// so an offset that is a lane part XOR a constant permutes as the XOR of the
// two permuted parts (the constant one folds at compile time).
__host__ __device__ constexpr int parity(int x) { return __builtin_popcount(x) & 1; }
__host__ __device__ constexpr int swz_u(int u) {
  return u ^ (parity(62 & (u >> 3)) | (parity(53 & (u >> 3)) << 1) |
              (parity(15 & (u >> 3)) << 2) | (parity(54 & (u >> 4)) << 3));
}
// the unit that swz_u places at s
__host__ __device__ constexpr int swz_u_inv(int s) {
  const int b3 = ((s >> 3) & 1) ^ parity(54 & (s >> 4));
  const int u3 = (s & ~15) | (b3 << 3) | (s & 7);  // bits 3.. of the unit
  return u3 ^ (parity(62 & (u3 >> 3)) | (parity(53 & (u3 >> 3)) << 1) |
               (parity(15 & (u3 >> 3)) << 2));
}
static_assert(swz_u_inv(swz_u(777)) == 777 && swz_u(swz_u_inv(1000)) == 1000, "bijection");
static_assert((swz_u(300 ^ 517) ^ swz_u(300)) == swz_u(517), "linear");

template <int HD>
struct Stage {
  static constexpr int SK = HD == 64 ? 64 : 32;                // keys per stage
  static constexpr int FL = SK * HD;                           // floats of K (or V)
  static constexpr int NDMA = FL * 4 / (kPThreads * 16);       // 16-byte copies per thread
};

// NBUF stage buffers: NBUF - 1 stage copies are in flight ahead of the one
// being computed (2: two workgroups per CU share the CU's LDS).
template <int HD, int G, int NBUF>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(const PrefillParams P) {
  using S = Stage<HD>;
  constexpr int SK = S::SK, FL = S::FL, NDMA = S::NDMA;
  constexpr int RPV = 16 / G;    // rows per wave
  constexpr int NQ = HD / 4;     // QK instructions per 16-key tile
  constexpr int NH = HD / 64;    // 16-dim runs per lane group
  constexpr int VD = HD / 16;    // V dims per lane per key = output tiles
  constexpr int NT = HD / 16;
  // one array per stage buffer ([K, V][stage]), picked at compile time
  __shared__ __align__(16) float s_b0[2 * FL];
  __shared__ __align__(16) float s_b1[2 * FL];
  __shared__ __align__(16) float s_b2[NBUF > 2 ? 2 * FL : 4];
  __shared__ __align__(16) float s_b3[NBUF > 3 ? 2 * FL : 4];
  auto bufp = [&](int b) -> float* { return b == 0 ? s_b0 : b == 1 ? s_b1 : b == 2 ? s_b2 : s_b3; };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = blockIdx.y;
  const int gq = lane >> 4;      // lane group
  const int vec = lane & 15;     // query vector of this lane
  const int rowb = blockIdx.x * (kPWaves * RPV);     // first row of the workgroup
  const int row0 = rowb + wave * RPV;                 // first row of the wave
  const bool wave_live = row0 < P.rows;               // wave-uniform
  const int row = min(row0 + vec / G, P.rows - 1);
  const int head = kh * G + vec % G;
  const int limit = P.pos0 + row;  // last key of this vector
  // the workgroup's keys [0, last_key], in stages; split z takes its share
  const int last_key = P.pos0 + min(rowb + kPWaves * RPV - 1, P.rows - 1);
  const int n_stages = last_key / SK + 1;
  const int st_begin = n_stages * static_cast<int>(blockIdx.z) / P.ks;
  const int st_end = n_stages * (static_cast<int>(blockIdx.z) + 1) / P.ks;
  const int wave_last = P.pos0 + min(row0 + RPV - 1, P.rows - 1);  // wave-uniform

  const size_t head_el = static_cast<size_t>(kh) * P.capg * HD;
  const float* kbase = P.kf + head_el;
  const float* vbase = P.vf + head_el;

  // stage copy: K then V, 16 bytes per lane per instruction; copy m of this
  // wave fills units [m * kPThreads + 64 * wave, + 64) of the buffer, and
  // lane l's slot holds unit swz_u_inv(slot) of the stage, from the same
  // 1 KiB (the permutation stays within 16-unit runs)
  uint32_t src_off[NDMA];
#pragma unroll
  for (int m = 0; m < NDMA; ++m) {
    const int u0 = m * kPThreads + 64 * wave;
    src_off[m] = 16u * static_cast<uint32_t>(swz_u_inv(u0 + lane) - u0);
  }
  auto copy_stage = [&](int st, float* dst) {
    const size_t off = static_cast<size_t>(st) * FL;
    const uint32_t d = lds_addr(dst);
#pragma unroll
    for (int m = 0; m < NDMA; ++m) {
      const int e = (m * kPThreads + wave * 64) * 4;  // this wave's KiB of the copy
      lds_copy16(kbase + off + e, src_off[m], d + 4 * e);
      lds_copy16(vbase + off + e, src_off[m], d + 4 * (FL + e));
    }
  };
  // permuted operand units: a tile's K read (tile t, dims run h, step s4) is
  // unit kb[h] ^ (t * 4 HD) ^ s4 and a V read (tile t, key j of the lane
  // group, half u) is vb ^ (t * 4 HD) ^ unit(j, 0) ^ 64 u, the lane parts
  // kb, vb those of tile 0 (no carries between the parts)
  int skb[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h)
    skb[h] = swz_u(static_cast<int>(k_off_tiled(HD, false, vec, 16 * gq + 64 * h)) >> 2);
  const int svb = swz_u(static_cast<int>(v_off_tiled(HD, false, 4 * gq, VD * vec)) >> 2);
  auto k_at = [&](int t, int h, int s4) { return 4 * (skb[h] ^ swz_u(t * 4 * HD ^ s4)); };
  auto v_at = [&](int t, int j, int u) {
    return 4 * (svb ^ swz_u(t * 4 * HD ^ (static_cast<int>(v_off_tiled(HD, false, j, 0)) >> 2) ^
                            (64 * u)));
  };

  // Q^T operands: dims 16 gq + 64 h + s, pre-scaled into the log2 domain
  float qv[NQ];
  {
    const float* qp = P.q + (static_cast<size_t>(row) * P.n_heads + head) * HD + 16 * gq;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float4 t = *reinterpret_cast<const float4*>(qp + 64 * h + 4 * s4);
        qv[16 * h + 4 * s4 + 0] = t.x * P.qscale;
        qv[16 * h + 4 * s4 + 1] = t.y * P.qscale;
        qv[16 * h + 4 * s4 + 2] = t.z * P.qscale;
        qv[16 * h + 4 * s4 + 3] = t.w * P.qscale;
      }
  }

  f4 acc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kMinitP, l_run = 0.0f;

  // S^T of tile t (keys st*SK + 16t ..) in four independent chains
  auto qk = [&](int t, const float* sk, f4 (&sc)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) sc[c] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float4 x = lds4(sk + k_at(t, h, s4));
        const int i = 16 * h + 4 * s4;
        sc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, qv[i + 0], sc[0], 0, 0, 0);
        sc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, qv[i + 1], sc[1], 0, 0, 0);
        sc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, qv[i + 2], sc[2], 0, 0, 0);
        sc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, qv[i + 3], sc[3], 0, 0, 0);
      }
    }
  };

  // online softmax of tile t's scores, then O^T += V^T P^T. MASK: the tile
  // reaches past some row's last key or past the workgroup's last key
  // (causal diagonal, chunk tail); other tiles skip the masks.
  auto soft_pv = [&](int st, int t, const float* sv, const f4 (&sc)[4], auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    const int kb = st * SK + 16 * t;  // first key of the tile (wave-uniform)
    const f4 s = (sc[0] + sc[1]) + (sc[2] + sc[3]);
    float sv4[4];
    float mx = kMinitP;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int key = kb + 4 * gq + v;
      sv4[v] = !MASK || key <= limit ? s[v] : -INFINITY;
      mx = fmaxf(mx, sv4[v]);
    }
    mx = xmax32(xmax16(mx));
    const float mn = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
    float pv[4], ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      pv[v] = __builtin_amdgcn_exp2f(sv4[v] - mn);
      ls += pv[v];
    }
    ls = xsum32(xsum16(ls));
    l_run = l_run * alpha + ls;
    m_run = mn;
    // once the running maxima settle, alpha is exactly 1 in every lane and
    // the rescale (a multiply by 1) is skipped
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
    }

    // O^T += V^T P^T: output tile tt row i is dim VD i + tt. Keys past the
    // workgroup's last row are never weighted and read as 0.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = kb + 4 * gq + j;
      float vd[VD];
#pragma unroll
      for (int u = 0; u < VD / 4; ++u) {
        const float4 x = lds4(sv + v_at(t, j, u));
        vd[4 * u + 0] = !MASK || key <= last_key ? x.x : 0.0f;
        vd[4 * u + 1] = !MASK || key <= last_key ? x.y : 0.0f;
        vd[4 * u + 2] = !MASK || key <= last_key ? x.z : 0.0f;
        vd[4 * u + 3] = !MASK || key <= last_key ? x.w : 0.0f;
      }
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[tt], pv[j], acc[tt], 0, 0, 0);
    }
  };

  // A stage's tiles, software-pipelined: tile t + 1's QK^T products are
  // issued before tile t's softmax, so the matrix core works through them
  // while the wave's VALU runs the softmax. Tiles past every row of the wave
  // (the causal tail) are skipped.
  constexpr int NTS = SK / 16;  // tiles per stage
  // keys every row of the wave attends, and that the workgroup holds
  const int wave_full = min(P.pos0 + row0, last_key);
  // A stage whose tiles are all full and unmasked runs as one straight-line
  // block: the LDS operands of tile t + 1 (V) and t + 2 (K) are read while
  // tile t's products run, and tile t + 1's QK^T products are issued before
  // tile t's softmax, so the scheduler can place the softmax's VALU and the
  // reads between matrix instructions. Same operations in the same order as
  // the general path (the rescale is unconditional: a multiply by exactly 1
  // when the maxima hold), so the results are identical.
  auto stage_full = [&](const float* sk, const float* sv) {
    constexpr int NK = NQ / 4;  // 16-byte K reads per tile
    auto ld_k = [&](int t, float4 (&x)[NK]) {
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) x[4 * h + s4] = lds4(sk + k_at(t, h, s4));
    };
    auto ld_v = [&](int t, float4 (&x)[4][VD / 4]) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < VD / 4; ++u) x[j][u] = lds4(sv + v_at(t, j, u));
    };
    auto mm_qk = [&](const float4 (&x)[NK], f4 (&sc)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) sc[c] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i4 = 0; i4 < NK; ++i4) {
        const int i = 4 * i4;
        sc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[i4].x, qv[i + 0], sc[0], 0, 0, 0);
        sc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[i4].y, qv[i + 1], sc[1], 0, 0, 0);
        sc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[i4].z, qv[i + 2], sc[2], 0, 0, 0);
        sc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[i4].w, qv[i + 3], sc[3], 0, 0, 0);
      }
    };
    auto softmax = [&](const f4 (&sc)[4], float (&pv)[4]) {
      const f4 s = (sc[0] + sc[1]) + (sc[2] + sc[3]);
      float mx = kMinitP;
#pragma unroll
      for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s[v]);
      mx = xmax32(xmax16(mx));
      const float mn = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
      float ls = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        pv[v] = __builtin_amdgcn_exp2f(s[v] - mn);
        ls += pv[v];
      }
      ls = xsum32(xsum16(ls));
      l_run = l_run * alpha + ls;
      m_run = mn;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
    };
    auto mm_pv = [&](const float4 (&x)[4][VD / 4], const float (&pv)[4]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float vd[VD];
#pragma unroll
        for (int u = 0; u < VD / 4; ++u) {
          vd[4 * u + 0] = x[j][u].x;
          vd[4 * u + 1] = x[j][u].y;
          vd[4 * u + 2] = x[j][u].z;
          vd[4 * u + 3] = x[j][u].w;
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[tt], pv[j], acc[tt], 0, 0, 0);
      }
    };
    float4 kx[2][NK], vx[2][4][VD / 4];
    f4 sc[2][4];
    ld_k(0, kx[0]);
    ld_v(0, vx[0]);
    if (NTS > 1) ld_k(1, kx[1]);
    mm_qk(kx[0], sc[0]);
#pragma unroll
    for (int t = 0; t < NTS; ++t) {
      if (t + 1 < NTS) mm_qk(kx[(t + 1) & 1], sc[(t + 1) & 1]);
      if (t + 2 < NTS) ld_k(t + 2, kx[t & 1]);
      if (t + 1 < NTS) ld_v(t + 1, vx[(t + 1) & 1]);
      float pv[4];
      softmax(sc[t & 1], pv);
      mm_pv(vx[t & 1], pv);
    }
  };

  auto compute_stage = [&](int st, const float* sk, const float* sv) {
    const int nt = !wave_live ? 0 : min(NTS, max(0, (wave_last - st * SK) / 16 + 1));  // uniform
    if (wave_live && st * SK + SK - 1 <= wave_full) {  // uniform: every tile full
      stage_full(sk, sv);
      return;
    }
    f4 sc[2][4];
    if (nt > 0) qk(0, sk, sc[0]);
#pragma unroll
    for (int t = 0; t < NTS; ++t) {
      if (t < nt) {
        if (t + 1 < nt) qk(t + 1, sk, sc[(t + 1) & 1]);
        if (st * SK + 16 * t + 15 <= wave_full)  // uniform
          soft_pv(st, t, sv, sc[t & 1], std::false_type{});
        else
          soft_pv(st, t, sv, sc[t & 1], std::true_type{});
      }
    }
  };

#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i)
    if (st_begin + i < st_end) copy_stage(st_begin + i, bufp(i));
  // unrolled by the buffer count, so every buffer index is a constant
  for (int st0 = st_begin; st0 < st_end; st0 += NBUF) {
#pragma unroll
    for (int b = 0; b < NBUF; ++b) {
      const int st = st0 + b;
      if (st >= st_end) break;  // uniform
      if (st + NBUF - 1 < st_end) copy_stage(st + NBUF - 1, bufp((b + NBUF - 1) % NBUF));
      // stage st has landed once at most the copies of the stages after it
      // are outstanding (loads complete in order)
      const int after = min(st_end - 1 - st, NBUF - 1);  // uniform
      if (after >= 3)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * 2 * NDMA) : "memory");
      else if (after == 2)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * 2 * NDMA) : "memory");
      else if (after == 1)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NDMA) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();  // every wave's part of stage st has landed
      compute_stage(st, bufp(b), bufp(b) + FL);
      lds_barrier();  // every wave is done with this buffer before it is refilled
    }
  }

  // lane holds O^T[dim VD (4 gq + v) + tt][vec]: dims 4 VD gq .. 4 VD gq + 4 VD - 1
  if (!wave_live || row0 + vec / G >= P.rows) return;
  const size_t rh = static_cast<size_t>(row) * P.n_heads + head;
  if (P.ks == 1) {
    const float inv = 1.0f / l_run;
    float* op = P.out + rh * HD + 4 * VD * gq;
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int tt = 0; tt < NT; tt += 4)
        *reinterpret_cast<float4*>(op + VD * v + tt) =
            make_float4(acc[tt][v] * inv, acc[tt + 1][v] * inv, acc[tt + 2][v] * inv,
                        acc[tt + 3][v] * inv);
    return;
  }
  float* rec = P.part + (static_cast<size_t>(blockIdx.z) * P.rows * P.n_heads + rh) * (HD + 2);
  float* op = rec + 4 * VD * gq;
#pragma unroll
  for (int v = 0; v < 4; ++v)
#pragma unroll
    for (int tt = 0; tt < NT; tt += 4)
      *reinterpret_cast<float4*>(op + VD * v + tt) =
          make_float4(acc[tt][v], acc[tt + 1][v], acc[tt + 2][v], acc[tt + 3][v]);
  if (gq == 0) {
    rec[HD] = m_run;
    rec[HD + 1] = l_run;
  }
}

// Combines the KS key splits of every (row, query head): one thread per dim,
// 256 / HD (row, head) pairs per workgroup. Every record load of a thread is
// issued before any of them is used (one round trip, not one per split).
constexpr int kMergeThreads = 256;
template <int HD, int KS>
__global__ __launch_bounds__(kMergeThreads) void prefill_merge(const float* __restrict__ part,
                                                               float* __restrict__ out,
                                                               int n_vec) {
  const int rh = blockIdx.x * (kMergeThreads / HD) + static_cast<int>(threadIdx.x) / HD;
  const int d = threadIdx.x % HD;
  if (rh >= n_vec) return;
  float o[KS], m[KS], l[KS];
#pragma unroll
  for (int z = 0; z < KS; ++z) {
    const float* r = part + (static_cast<size_t>(z) * n_vec + rh) * (HD + 2);
    o[z] = r[d];
    m[z] = r[HD];
    l[z] = r[HD + 1];
  }
  float M = kMinitP;
#pragma unroll
  for (int z = 0; z < KS; ++z) M = fmaxf(M, m[z]);
  float L = 0.0f, O = 0.0f;
#pragma unroll
  for (int z = 0; z < KS; ++z) {
    const float w = __builtin_amdgcn_exp2f(m[z] - M);
    L += l[z] * w;
    O += o[z] * w;
  }
  out[static_cast<size_t>(rh) * HD + d] = O / L;
}

template <int HD>
void launch_merge(const float* part, float* out, int n_vec, int ks, hipStream_t st) {
  const dim3 grid((n_vec + kMergeThreads / HD - 1) / (kMergeThreads / HD));
  static_assert(kPrefillMaxSplits == 8, "merge instances for 2, 4 and 8 splits");
  if (ks == 2)
    hipLaunchKernelGGL((prefill_merge<HD, 2>), grid, dim3(kMergeThreads), 0, st, part, out, n_vec);
  else if (ks == 4)
    hipLaunchKernelGGL((prefill_merge<HD, 4>), grid, dim3(kMergeThreads), 0, st, part, out, n_vec);
  else
    hipLaunchKernelGGL((prefill_merge<HD, 8>), grid, dim3(kMergeThreads), 0, st, part, out, n_vec);
}

template <int HD, int NBUF>
void* prefill_for(int G) {
  switch (G) {
    case 1: return reinterpret_cast<void*>(&prefill_kernel<HD, 1, NBUF>);
    case 2: return reinterpret_cast<void*>(&prefill_kernel<HD, 2, NBUF>);
    case 4: return reinterpret_cast<void*>(&prefill_kernel<HD, 4, NBUF>);
    case 8: return reinterpret_cast<void*>(&prefill_kernel<HD, 8, NBUF>);
    default: return nullptr;
  }
}

void* pick_prefill(int hd, int G, int /*rows*/) {
  return hd == 64 ? prefill_for<64, 2>(G) : prefill_for<128, 2>(G);
}

// key splits: two workgroups per CU (one wave per SIMD cannot hide the LDS
// and matrix-core latencies by itself), at least two stages each
int prefill_splits(const KvGeom& g, const AttnCall& c) {
  const int G = c.n_heads / g.nkv;
  const int rows_per_block = kPWaves * (16 / G);
  const int blocks = (c.rows + rows_per_block - 1) / rows_per_block * g.nkv;
  const int sk = g.hd == 64 ? Stage<64>::SK : Stage<128>::SK;
  const int stages = (c.pos0 + c.rows - 1) / sk + 1;
  int ks = 1;
  while (ks < kPrefillMaxSplits && blocks * ks < 512 && stages / (2 * ks) >= 2) ks *= 2;
  return ks;
}

}  // namespace

int prefill_split_count(const KvGeom& g, const AttnCall& c) { return prefill_splits(g, c); }

bool prefill_supported(const KvGeom& g, int n_heads, int rows) {
  if (g.int8 || g.ring || !g.tiled || rows < kPrefillMinRows || n_heads % g.nkv != 0)
    return false;
  return pick_prefill(g.hd, n_heads / g.nkv, rows) != nullptr;
}

size_t prefill_workspace_need(const KvGeom& g, const AttnCall& c) {
  const int ks = prefill_splits(g, c);
  return ks > 1 ? static_cast<size_t>(ks) * c.rows * c.n_heads * (g.hd + 2) : 0;
}

hipError_t launch_prefill(const KvGeom& g, const KvStore& s, Workspace& ws, const AttnCall& c,
                          hipStream_t st) {
  const int G = c.n_heads / g.nkv;
  void* fn = pick_prefill(g.hd, G, c.rows);
  if (fn == nullptr) return hipErrorNotSupported;
  const int ks = prefill_splits(g, c);
  if (ks > 1 && ws.part_floats < prefill_workspace_need(g, c)) return hipErrorInvalidValue;
  PrefillParams p{};
  const size_t layer_el = static_cast<size_t>(c.layer) * g.nkv * head_elems(g);
  p.kf = s.k + layer_el;
  p.vf = s.v + layer_el;
  p.q = c.q;
  p.out = c.out;
  p.part = ws.part;
  p.capg = g.capg;
  p.n_heads = c.n_heads;
  p.rows = c.rows;
  p.pos0 = c.pos0;
  p.ks = ks;
  p.qscale = c.scale * kLog2eP;
  const int rows_per_block = kPWaves * (16 / G);
  void* args[] = {&p};
  hipError_t e = hipLaunchKernel(fn, dim3((c.rows + rows_per_block - 1) / rows_per_block, g.nkv, ks),
                                 dim3(kPThreads), args, 0, st);
  if (e != hipSuccess || ks == 1) return e;
  if (g.hd == 64)
    launch_merge<64>(ws.part, c.out, c.rows * c.n_heads, ks, st);
  else
    launch_merge<128>(ws.part, c.out, c.rows * c.n_heads, ks, st);
  return hipGetLastError();
}

}  // namespace dbi
