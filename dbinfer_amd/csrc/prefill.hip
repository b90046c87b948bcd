// Causal chunk attention of the dense fp32 cache on the matrix cores: the
// attention loop of decode_layer_chunk (model.cpp:956-981), rows c of a
// chunk at pos0 attending keys [0, pos0 + c], for chunks long enough to
// make QK^T and PV real matrix products (the prefill chunks of config 2).
//
// Design (CDNA4 v_mfma_f32_16x16x32_bf16 over exact three-part splits of the
// fp32 operands, bf16x3.hpp, so the result stays within the fp32 tolerance
// of the CPU path):
//  - A workgroup of 8 waves (one per CU) owns 128 query vectors of one kv
//    head: each wave 16 columns, 16/G rows x the G query heads sharing the
//    kv head (G = 3, 5, 6, 7 leave 16 mod G padding columns, which compute
//    and write nothing of use). The grid is (kv head, row block, key
//    split): with kv heads along x, every row block and split of one head
//    runs on one XCD, whose L2 serves the head's K/V to all of them.
//  - The workgroup walks its keys in stages of 32 (one pair of 16-key
//    tiles). Staging: a stage's fp32 K and V are loaded into registers while
//    earlier stages compute, split once per workgroup into hi, mid and lo
//    bf16 parts and written to LDS in the matrix cores' operand layout
//    (waves 0-3 K, 4-7 V): every operand read of the waves is one 16-byte
//    LDS load of 8 bf16, and no wave converts K or V itself. Three stage
//    buffers: a step issues the next stage's QK^T before its own softmax.
//  - Keys can be split over KS workgroups (grid z) to fill the GPU on short
//    chunks; a split writes its unnormalized (o, m, l) and prefill_merge
//    combines them.
//  - S^T = K Q^T: A = K (16 keys x 32 dims), B = Q^T (32 dims x 16 vectors),
//    six bf16 products per 32-dim step. In k-step ks = 2 h + hf, lane group
//    gq's k-index 8 gq + e stands for dim 16 gq + 64 h + 8 hf + e. The
//    result holds S[vector l % 16][key 4 (l / 16) + v] in lane l.
//  - O^T += V^T P^T over the pair's 32 keys: B = P^T straight from the
//    score registers (k-index 8 gq + e: key 4 gq + e of the first tile for
//    e < 4, key 4 gq + e - 4 of the second otherwise), A = V^T in the same
//    key order. Output tile tt row i stands for dim (hd/16) i + tt, so a
//    lane's output is hd/4 contiguous floats of its vector.
//  - Online softmax per vector (= per lane % 16) with a lazy reference
//    maximum; the four lane groups holding one vector combine through two
//    lane swaps.
#include <cmath>
#include <type_traits>

#include "bf16x3.hpp"
#include "kv_internal.hpp"

namespace dbi {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kPWaves = 8;
constexpr int kPThreads = 64 * kPWaves;
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kMinitP = -1.0e30f;  // finite: exp2(kMinit - kMinit) == 1
constexpr float kLazyLog2 = 8.0f;    // weights relative to the running maximum: at most 2^8

struct PrefillParams {
  const float* kf;  // this layer's K, V: [nkv][capg * hd], granule layout
  const float* vf;
  const float* q;   // [rows][n_heads][hd]
  float* out;       // [rows][n_heads][hd]
  float* part;      // KS > 1: o [KS][rows][n_heads][hd] (unnormalized), then (m, l) [KS][rows][n_heads][2]
  int capg, n_heads, rows, pos0, ks;
  float qscale;     // scale * log2(e)
};

// Workgroup barrier after this wave's LDS accesses have completed.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Lane-group exchanges of the softmax through the gfx950 permlane swaps
// (VALU, no LDS round trip like a bpermute). After v_permlane16_swap of
// (x, x), a lane holds its own x and the x of lane ^ 16 (one in each
// register); v_permlane32_swap does the same for lane ^ 32. Emitted through
// asm: the compiler's builtins fold the two results into one when both are
// used. The maxima take the max inside the asm too: fmaxf on asm results
// costs two NaN-quieting v_max of its operands first.
__device__ __forceinline__ float xmax16(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 0\n\tv_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}
__device__ __forceinline__ float xmax32(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 0\n\tv_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
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

// One stage in LDS: parts p = 0, 1, 2 (hi, mid, lo) of K, then of V, each a
// plane of SK x HD bf16.
//  - K plane: key k's dims 8 u .. 8 u + 7 are the 16-byte unit
//    k * HD/8 + (u ^ kswz(k)). The swizzle puts the 8 (16) keys of one
//    operand read's 8-lane (16-lane) group on distinct banks of 128 (256)
//    bytes.
//  - V plane: unit (j, s) = j * HD + s holds keys kv(j, e), e < 8, of dim
//    vdim(s): kv(j, e) = 4 j + e for e < 4 and 16 + 4 j + e - 4 otherwise
//    (the PV k-order of lane group j), vdim(s) = (HD/16) (s % 16) + s / 16
//    (lane i of output tile tt reads s = 16 tt + i: 16 contiguous units).
template <int HD>
struct Stage {
  static constexpr int SK = 32;                   // keys per stage
  static constexpr int NBUF = 3;                  // stage buffers (one workgroup per CU)
  static constexpr int UPR = HD / 8;              // 16-byte units per key of a K part
  static constexpr int PLANE = SK * HD * 2;       // bytes of one part of K or V
  static constexpr int BYTES = 6 * PLANE;
  static constexpr int STG = kPThreads / 2;       // staging lanes of K (and of V)
  static constexpr int NU = SK * HD / 8 / STG;    // staging lane: K units, or V dims
};

template <int HD>
__host__ __device__ constexpr int kswz(int key) {
  return HD == 64 ? ((key & 7) ^ ((key >> 3) & 1)) : (key & 15);
}

template <int HD, int G>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(const PrefillParams P) {
  using S = Stage<HD>;
  constexpr int SK = S::SK, NBUF = S::NBUF, UPR = S::UPR, PLANE = S::PLANE, NU = S::NU;
  constexpr int RPV = 16 / G;    // rows per wave (columns past RPV G pad the tile)
  constexpr int NH = HD / 64;    // 64-dim runs of a K row
  constexpr int VD = HD / 16;    // output tiles
  constexpr int NT = VD;
  __shared__ __align__(16) char s_stage[NBUF * S::BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = blockIdx.x;  // (grid x: the kv heads, see launch_prefill)
  const int gq = lane >> 4;      // lane group
  const int vec = lane & 15;     // query vector of this lane
  const int rowb = blockIdx.y * (kPWaves * RPV);     // first row of the workgroup
  const int row0 = rowb + wave * RPV;                 // first row of the wave
  const bool wave_live = row0 < P.rows;               // wave-uniform
  // (a padding column repeats the wave's last row; it writes nothing)
  const int row = min(row0 + min(vec / G, RPV - 1), P.rows - 1);
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

  // ---- staging. K lanes (the first half of the waves, t < STG): units
  // n = t + STG m, key n / UPR, dims 8 (n % UPR) .. + 7 (two float4 of the
  // granule layout). V lanes (t = STG + (HD / NU) j + c): keys kv(j, e) x
  // NU consecutive dims. The source offsets of stage 0 (stage st adds
  // st * SK * HD: a stage is two whole granules).
  constexpr int STG = S::STG;
  static_assert(NU == 1 || NU == 2, "staging shapes");
  const bool k_stager = wave < kPWaves / 2;  // uniform
  uint32_t src[8];
  uint32_t dst[NU];  // K: the unit's byte offset in a part plane; V: [0] of dim NU c
  int vkey[8];
  if (k_stager) {
#pragma unroll
    for (int m = 0; m < NU; ++m) {
      const int n = static_cast<int>(threadIdx.x) + STG * m;
      const int key = n / UPR, u = n % UPR;
      src[2 * m] = static_cast<uint32_t>(k_off_tiled(HD, false, key, 8 * u));
      src[2 * m + 1] = static_cast<uint32_t>(k_off_tiled(HD, false, key, 8 * u + 4));
      dst[m] = static_cast<uint32_t>((key * UPR + (u ^ kswz<HD>(key))) * 16);
    }
#pragma unroll
    for (int e = 2 * NU; e < 8; ++e) src[e] = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) vkey[e] = 0;
  } else {
    const int t = static_cast<int>(threadIdx.x) - STG;
    const int j = t / (HD / NU), c = t % (HD / NU);
    // lane c writes units s, s + 16, .. with s = c % 16 + 16 NU (c / 16):
    // 16 consecutive lanes write 16 consecutive units (no bank conflicts);
    // their dims vdim(s + 16 m) = d + m are consecutive
    const int s0 = c % 16 + 16 * NU * (c / 16);
    const int d = VD * (c % 16) + NU * (c / 16);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      vkey[e] = e < 4 ? 4 * j + e : 16 + 4 * j + e - 4;
      src[e] = static_cast<uint32_t>(v_off_tiled(HD, false, vkey[e], d));
    }
    dst[0] = static_cast<uint32_t>((j * HD + s0) * 16);
#pragma unroll
    for (int m = 1; m < NU; ++m) dst[m] = dst[0] + 256u * m;
  }
  // the loaded stage: K lanes hold unit m in r[2 m], r[2 m + 1]; V lanes key
  // e's dim in component e % 4 of r[e / 4] (NU = 1) or its two dims in half
  // e % 2 of r[e / 2] (NU = 2).
  // Buffer loads from a resource over the stage (src offsets in bytes).
#pragma unroll
  for (int e = 0; e < 8; ++e) src[e] *= 4u;
  float4 r[2 * NU];
  auto load_stage = [&](int st) {
    const size_t so = static_cast<size_t>(st) * SK * HD;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>((k_stager ? kbase : vbase) + so), static_cast<short>(0), SK * HD * 4,
        0x00020000);
    if (k_stager) {
#pragma unroll
      for (int i = 0; i < 2 * NU; ++i)
        r[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, src[i], 0, 0));
    } else if constexpr (NU == 1) {
#pragma unroll
      for (int e = 0; e < 8; e += 4) {
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          x[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, src[e + i], 0, 0));
        r[e / 4] = make_float4(x[0], x[1], x[2], x[3]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float2 a =
            __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, src[e], 0, 0));
        const float2 b =
            __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, src[e + 1], 0, 0));
        r[e / 2] = make_float4(a.x, a.y, b.x, b.y);
      }
    }
  };
  auto vdim = [&](int e, int m) -> float {
    if constexpr (NU == 1) {
      const float4 x = r[e / 4];
      return e % 4 == 0 ? x.x : e % 4 == 1 ? x.y : e % 4 == 2 ? x.z : x.w;
    } else {
      const float4 x = r[e / 2];
      return (e & 1) == 0 ? (m == 0 ? x.x : x.y) : (m == 0 ? x.z : x.w);
    }
  };
  // split and store; V of keys past the workgroup's last key is stored as 0
  // (its weight is 0, and the cache past the chunk may hold anything)
  auto store_stage = [&](int st, char* sb) {
    if (k_stager) {
#pragma unroll
      for (int m = 0; m < NU; ++m) {
        const float4 a = r[2 * m], b = r[2 * m + 1];
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint4 part[3];
        split3(x, part);
#pragma unroll
        for (int p = 0; p < 3; ++p) *reinterpret_cast<uint4*>(sb + p * PLANE + dst[m]) = part[p];
      }
    } else {
      const bool tail = st * SK + SK - 1 > last_key;  // uniform
#pragma unroll
      for (int m = 0; m < NU; ++m) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = vdim(e, m);
          x[e] = !tail || st * SK + vkey[e] <= last_key ? v : 0.0f;
        }
        uint4 part[3];
        split3(x, part);
#pragma unroll
        for (int p = 0; p < 3; ++p)
          *reinterpret_cast<uint4*>(sb + (3 + p) * PLANE + dst[m]) = part[p];
      }
    }
  };

  // ---- operands. Q^T: dims 16 gq + 64 h + 8 hf + e of k-step 2 h + hf,
  // pre-scaled into the log2 domain, in three bf16 parts
  constexpr int KS = HD / 32;
  uint4 qp[KS][3];
  {
    const float* qp_src = P.q + (static_cast<size_t>(row) * P.n_heads + head) * HD + 16 * gq;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const float4 a = *reinterpret_cast<const float4*>(qp_src + 64 * (ks / 2) + 8 * (ks % 2));
      const float4 b = *reinterpret_cast<const float4*>(qp_src + 64 * (ks / 2) + 8 * (ks % 2) + 4);
      const float x[8] = {a.x * P.qscale, a.y * P.qscale, a.z * P.qscale, a.w * P.qscale,
                          b.x * P.qscale, b.y * P.qscale, b.z * P.qscale, b.w * P.qscale};
      split3(x, qp[ks]);
    }
  }
  // lane byte offsets of the K reads (tile 0, k-step 2 h + hf) and V reads
  // (output tile 0) within a part plane
  int klo[NH][2];
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
      klo[h][hf] = (vec * UPR + ((2 * gq + 8 * h + hf) ^ kswz<HD>(vec))) * 16;
  const int vlo = (gq * HD + vec) * 16;

  f4 acc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kMinitP, l_run = 0.0f;

  // a b = sum of a_i b_j over the parts; the six terms with i + j <= 2 are
  // kept (the dropped ones are below 2^-23 |a b|, the size of the fp32
  // rounding the reference's own sums carry). One accumulator chain: the
  // matrix cores forward a dependent accumulation at full rate.
  auto terms1 = [&](const uint4 (&a)[3], const uint4 (&b)[3], f4& c) {
    c = mfma_bf16(a[2], b[0], c);
    c = mfma_bf16(a[1], b[1], c);
    c = mfma_bf16(a[0], b[2], c);
    c = mfma_bf16(a[1], b[0], c);
    c = mfma_bf16(a[0], b[1], c);
    c = mfma_bf16(a[0], b[0], c);
  };

  // keys every row of the wave attends, and that the workgroup holds
  const int wave_full = min(P.pos0 + row0, last_key);

  // S^T of a stage's two tiles: sc[u] holds tile u (lane l: S[vector l % 16]
  // [key 4 (l / 16) + v])
  auto qk = [&](const char* sb, f4 (&sc)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      sc[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          uint4 kp[3];
#pragma unroll
          for (int p = 0; p < 3; ++p)
            kp[p] = *reinterpret_cast<const uint4*>(sb + p * PLANE + u * 16 * UPR * 16 + klo[h][hf]);
          terms1(kp, qp[2 * h + hf], sc[u]);
        }
    }
  };
  // Online softmax of a stage's 32 keys, then O^T += V^T P^T. MASK: the
  // stage reaches past some row's last key (causal diagonal, chunk tail).
  auto soft_pv = [&](int st, const char* sb, const f4 (&sc)[2], auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    const int kb = st * SK;  // first key of the stage (wave-uniform)
    float s8[8];
    float mx = kMinitP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f4 s = sc[u];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = kb + 16 * u + 4 * gq + v;
        s8[4 * u + v] = !MASK || key <= limit ? s[v] : -INFINITY;
        mx = fmaxf(mx, s8[4 * u + v]);
      }
    }
    mx = xmax32(xmax16(mx));
    // The reference maximum m_run moves only when a score passes it by more
    // than 2^kLazyLog2 (so every weight is at most 2^kLazyLog2: the splits
    // stay exact and the sums far from fp32's range), and then to the
    // stage's maximum. Otherwise alpha is exactly 1 in every lane and the
    // rescale is skipped: after the first stages it almost never runs.
    const float mn = mx > m_run + kLazyLog2 ? mx : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
    float pv8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv8[e] = __builtin_amdgcn_exp2f(s8[e] - mn);
    float ls = pv8[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) ls += pv8[e];
    ls = xsum32(xsum16(ls));
    l_run = l_run * alpha + ls;
    m_run = mn;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
    }
    uint4 pb[3];
    split3(pv8, pb);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      uint4 va[3];
#pragma unroll
      for (int p = 0; p < 3; ++p)
        va[p] = *reinterpret_cast<const uint4*>(sb + (3 + p) * PLANE + tt * 256 + vlo);
      terms1(va, pb, acc[tt]);
    }
  };
  // stages past every row of the wave (the causal tail) are skipped
  auto live = [&](int st) { return wave_live && st * SK <= wave_last; };  // uniform
  auto soft_pv_stage = [&](int st, const char* sb, const f4 (&sc)[2]) {
    if (st * SK + SK - 1 <= wave_full)
      soft_pv(st, sb, sc, std::false_type{});
    else
      soft_pv(st, sb, sc, std::true_type{});
  };

  // The next stages' loads are in flight while a stage computes; the
  // compiler waits for them where the split reads them.
  if (st_begin < st_end) {
    load_stage(st_begin);
    store_stage(st_begin, s_stage);
  }
  static_assert(NBUF == 3, "three stage buffers");
  {
    // Three buffers hold stages s, s + 1 (both stored) and s + 2 (being
    // stored); the S^T products of stage s + 1 are issued before the
    // softmax of stage s, so the matrix cores work through them while the
    // wave's VALU runs the softmax, the splits and the staging. One barrier
    // per stage: stage s + 2 is stored into the buffer stage s - 1 was read
    // from, and read after the next barrier.
    if (st_begin + 1 < st_end) {
      load_stage(st_begin + 1);
      store_stage(st_begin + 1, s_stage + S::BYTES);
    }
    lds_barrier();
    f4 sa[2], sb2[2];
    if (st_begin < st_end && live(st_begin)) qk(s_stage, sa);
    // stage st in buffer B; cur / nxt its and the next stage's scores
    auto step = [&](int st, auto b_c, f4 (&cur)[2], f4 (&nxt)[2]) {
      constexpr int B = decltype(b_c)::value;
      if (st + 2 < st_end) load_stage(st + 2);
      if (st + 1 < st_end && live(st + 1)) qk(s_stage + ((B + 1) % 3) * S::BYTES, nxt);
      if (live(st)) soft_pv_stage(st, s_stage + B * S::BYTES, cur);
      if (st + 2 < st_end) store_stage(st + 2, s_stage + ((B + 2) % 3) * S::BYTES);
      lds_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    for (int st = st_begin; st < st_end; st += 6) {
      step(st, I0{}, sa, sb2);
      if (st + 1 >= st_end) break;  // uniform
      step(st + 1, I1{}, sb2, sa);
      if (st + 2 >= st_end) break;
      step(st + 2, I2{}, sa, sb2);
      if (st + 3 >= st_end) break;
      step(st + 3, I0{}, sb2, sa);
      if (st + 4 >= st_end) break;
      step(st + 4, I1{}, sa, sb2);
      if (st + 5 >= st_end) break;
      step(st + 5, I2{}, sb2, sa);
    }
  }

  // lane holds O^T[dim VD (4 gq + v) + tt][vec]: dims 4 VD gq .. 4 VD gq + 4 VD - 1
  if (!wave_live || vec >= RPV * G || row0 + vec / G >= P.rows) return;
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
  // split records: o at [z][vector][HD], (m, l) at [z][vector][2] after
  // every o
  const size_t n_vec = static_cast<size_t>(P.rows) * P.n_heads;
  float* op = P.part + (blockIdx.z * n_vec + rh) * HD + 4 * VD * gq;
#pragma unroll
  for (int v = 0; v < 4; ++v)
#pragma unroll
    for (int tt = 0; tt < NT; tt += 4)
      *reinterpret_cast<float4*>(op + VD * v + tt) =
          make_float4(acc[tt][v], acc[tt + 1][v], acc[tt + 2][v], acc[tt + 3][v]);
  if (gq == 0)
    *reinterpret_cast<float2*>(P.part + P.ks * n_vec * HD + (blockIdx.z * n_vec + rh) * 2) =
        make_float2(m_run, l_run);
}

// Combines the KS key splits of every (row, query head): HD / 4 threads per
// vector, 4 dims each; a workgroup serves rows of one kv head (grid x, as
// in the chunk kernel, so it runs on the XCD that wrote the records). Every
// record load of a thread is issued before any of them is used.
constexpr int kMergeThreads = 256;
template <int HD, int KS>
__global__ __launch_bounds__(kMergeThreads) void prefill_merge(const float* __restrict__ part,
                                                               float* __restrict__ out, int rows,
                                                               int n_heads, int G) {
  constexpr int TPV = HD / 4;                // threads per vector
  constexpr int VPW = kMergeThreads / TPV;   // vectors per workgroup (>= 8 >= G)
  const int rpw = VPW / G;                   // rows per workgroup
  const int kh = blockIdx.x;
  const int j = static_cast<int>(threadIdx.x) / TPV, d4 = static_cast<int>(threadIdx.x) % TPV;
  const int row = static_cast<int>(blockIdx.y) * rpw + j / G;
  if (j >= rpw * G || row >= rows) return;
  const size_t n_vec = static_cast<size_t>(rows) * n_heads;
  const size_t rh = static_cast<size_t>(row) * n_heads + kh * G + j % G;
  float4 o[KS];
  float2 ml[KS];
#pragma unroll
  for (int z = 0; z < KS; ++z) {
    o[z] = *reinterpret_cast<const float4*>(part + (z * n_vec + rh) * HD + 4 * d4);
    ml[z] = *reinterpret_cast<const float2*>(part + KS * n_vec * HD + (z * n_vec + rh) * 2);
  }
  float M = kMinitP;
#pragma unroll
  for (int z = 0; z < KS; ++z) M = fmaxf(M, ml[z].x);
  float L = 0.0f;
  float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int z = 0; z < KS; ++z) {
    const float w = __builtin_amdgcn_exp2f(ml[z].x - M);
    L += ml[z].y * w;
    O.x += o[z].x * w;
    O.y += o[z].y * w;
    O.z += o[z].z * w;
    O.w += o[z].w * w;
  }
  *reinterpret_cast<float4*>(out + rh * HD + 4 * d4) = make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
}

template <int HD>
void launch_merge(const float* part, float* out, int rows, int n_heads, int nkv, int ks,
                  hipStream_t st) {
  const int G = n_heads / nkv;
  const int rpw = kMergeThreads / (HD / 4) / G;
  const dim3 grid(nkv, (rows + rpw - 1) / rpw);
  static_assert(kPrefillMaxSplits == 8, "merge instances for 2, 4 and 8 splits");
  if (ks == 2)
    hipLaunchKernelGGL((prefill_merge<HD, 2>), grid, dim3(kMergeThreads), 0, st, part, out, rows,
                       n_heads, G);
  else if (ks == 4)
    hipLaunchKernelGGL((prefill_merge<HD, 4>), grid, dim3(kMergeThreads), 0, st, part, out, rows,
                       n_heads, G);
  else
    hipLaunchKernelGGL((prefill_merge<HD, 8>), grid, dim3(kMergeThreads), 0, st, part, out, rows,
                       n_heads, G);
}

template <int HD>
void* prefill_for(int G) {
  switch (G) {
    case 1: return reinterpret_cast<void*>(&prefill_kernel<HD, 1>);
    case 2: return reinterpret_cast<void*>(&prefill_kernel<HD, 2>);
    case 3: return reinterpret_cast<void*>(&prefill_kernel<HD, 3>);
    case 4: return reinterpret_cast<void*>(&prefill_kernel<HD, 4>);
    case 5: return reinterpret_cast<void*>(&prefill_kernel<HD, 5>);
    case 6: return reinterpret_cast<void*>(&prefill_kernel<HD, 6>);
    case 7: return reinterpret_cast<void*>(&prefill_kernel<HD, 7>);
    case 8: return reinterpret_cast<void*>(&prefill_kernel<HD, 8>);
    default: return nullptr;
  }
}

void* pick_prefill(int hd, int G, int /*rows*/) {
  return hd == 64 ? prefill_for<64>(G) : prefill_for<128>(G);
}

// key splits: one workgroup per CU (two waves per SIMD), at least two
// stages each
constexpr int kPrefillTargetBlocks = 256;
int prefill_splits(const KvGeom& g, const AttnCall& c) {
  const int G = c.n_heads / g.nkv;
  const int rows_per_block = kPWaves * (16 / G);
  const int blocks = (c.rows + rows_per_block - 1) / rows_per_block * g.nkv;
  const int sk = g.hd == 64 ? Stage<64>::SK : Stage<128>::SK;
  const int stages = (c.pos0 + c.rows - 1) / sk + 1;
  int ks = 1;
  while (ks < kPrefillMaxSplits && blocks * ks < kPrefillTargetBlocks && stages / (2 * ks) >= 2)
    ks *= 2;
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
  // kv heads along grid x: workgroups go to the 8 XCDs round-robin by
  // linear id, so with 8 kv heads every row block and split of one head
  // runs on one XCD, and that XCD's L2 serves the head's K/V to all of them
  hipError_t e = hipLaunchKernel(fn, dim3(g.nkv, (c.rows + rows_per_block - 1) / rows_per_block, ks),
                                 dim3(kPThreads), args, 0, st);
  if (e != hipSuccess || ks == 1) return e;
  if (g.hd == 64)
    launch_merge<64>(ws.part, c.out, c.rows, c.n_heads, g.nkv, ks, st);
  else
    launch_merge<128>(ws.part, c.out, c.rows, c.n_heads, g.nkv, ks, st);
  return hipGetLastError();
}

}  // namespace dbi
