// Dense int8 GQA attention on the matrix cores (attend_dense_int8,
// model.cpp:600-661; the causal chunk rows of decode_layer_chunk,
// model.cpp:956-981), instantiated by attn_inst_i8_dense_*.hip.
//
// Design (CDNA4, wave64, v_mfma_f32_16x16x32_bf16):
//  - Grid and split plan as attn_kernel: (split, kv head, query row), 8 waves
//    per workgroup, 32-position chunks (one K group each), chunk t -> wave
//    t % 8; every query head of the kv head is served from the same bytes.
//  - Exact bf16 products: int8 codes are exact in bf16, and an fp32 value is
//    exactly hi + mid + lo of three bf16 parts (split3), so each score is the
//    fp32 accumulation of exact products q~_i * k8_i, q~ = (q * scale * log2 e)
//    * ks (the reference's (q_i * ks_i) * k8_i, per K group), and each output
//    the fp32 accumulation of exact (p * vs) * v8 products. (Two parts are not
//    enough: a 2^-18 weight error times an outlier channel's |v| exceeds the
//    reference's own fp32 error where the output cancels.)
//  - QK^T: A = the chunk's K codes (rows: positions, read straight from the
//    layout of kv_internal.hpp), B = q~ in three parts (columns: (query,
//    V block) pairs, each query repeated once per 32-channel V block), built
//    per chunk by the whole wave (8 values per lane) and read back from LDS.
//  - Softmax on the scores as they leave the matrix core: lane n + 16g holds
//    column n at positions 16h + 4g + i, so a column's max and sum are lane-
//    local plus two permlane swaps, and the weight of (query, block) at those
//    positions is exactly the PV A operand of that lane (row = column): the
//    V layout stores each lane's 8 positions in that order. No LDS transpose.
//  - PV: A = weight * V block scale in three bf16 parts, B = the V codes of a
//    16-channel tile; row (query, block) is kept for the tiles of its block.
//  - Records, merge and fused append as attn_kernel; the fp32 sinks by wave 0
//    of split 0, their loads issued at entry with q.
#pragma once

#include "attn_kernel.hpp"
#include "bf16x3.hpp"

namespace dbi {
namespace {

// 8 signed int8 codes (bytes of lo, then hi) -> 8 bf16, exactly (|code| <=
// 127 leaves the low 16 bits of its fp32 value zero)
__device__ __forceinline__ bf16x8 codes_bf16(uint32_t lo, uint32_t hi) {
  float f[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) f[b] = static_cast<float>(static_cast<int8_t>(lo >> (8 * b)));
#pragma unroll
  for (int b = 0; b < 4; ++b) f[4 + b] = static_cast<float>(static_cast<int8_t>(hi >> (8 * b)));
  uint4 w;
  w.x = pack_hi(fbits(f[0]), fbits(f[1]));
  w.y = pack_hi(fbits(f[2]), fbits(f[3]));
  w.z = pack_hi(fbits(f[4]), fbits(f[5]));
  w.w = pack_hi(fbits(f[6]), fbits(f[7]));
  return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ f32x4 mfma(const uint4& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

using i32x4 = int __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 mfma_i8(const i32x4& a, const uint4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// planes[i] = byte i of d0, d1, d2, d3 (in that byte order): a 4 x 4 byte
// transpose in eight v_perm_b32
__device__ __forceinline__ void byte_planes(const uint32_t (&d)[4], uint32_t (&planes)[4]) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(d[1], d[0], 0x05010400u);  // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(d[1], d[0], 0x07030602u);  // a2 b2 a3 b3
  const uint32_t cd_lo = __builtin_amdgcn_perm(d[3], d[2], 0x05010400u);
  const uint32_t cd_hi = __builtin_amdgcn_perm(d[3], d[2], 0x07030602u);
  planes[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);
  planes[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
  planes[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  planes[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// max / sum of a lane's value over the 16 lanes of its row (DPP butterfly)
__device__ __forceinline__ float row16_max(float a) {
  a = fmaxf(a, dpp<kX1>(a));
  a = fmaxf(a, dpp<kX2>(a));
  a = fmaxf(a, dpp<kX7>(a));
  return fmaxf(a, dpp<kX8>(a));
}
__device__ __forceinline__ float row16_sum(float a) {
  a += dpp<kX1>(a);
  a += dpp<kX2>(a);
  a += dpp<kX7>(a);
  return a + dpp<kX8>(a);
}

// max / sum of a lane's value over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four
// 16-lane rows of one matrix column)
__device__ __forceinline__ float col_max(float a) {
  float b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  a = fmaxf(a, b);
  b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}
__device__ __forceinline__ float col_sum(float a) {
  a = swap16_sum(a, a);
  return swap32_sum(a, a);
}

// NQ: query vectors of a workgroup (rows x heads)
template <int HD, int NQ>
struct MCfg {
  static constexpr int NBK = HD / kBlock;      // V blocks per head
  static constexpr int QVT = 16 / NBK;         // query vectors per 16-column tile
  static constexpr int NT = (NQ + QVT - 1) / QVT;  // column tiles
  static constexpr int LPQ = HD / 8;           // lanes per query in the q~ layout
  static constexpr int NJ = HD / 32;           // QK k-steps (32 channels)
  static constexpr int KL = HD / 64;           // K loads per granule (two k-steps each)
  static constexpr int NTV = HD / 16;          // PV channel tiles
  static constexpr int VL = HD / 32;           // V loads per chunk (two tiles each)
  static constexpr int QROW = HD / 8 + 4;      // uint4 per q~ row in LDS (64-byte pad: no
                                               // bank conflicts between the 4 x 4 lane groups)
  static constexpr int NT2 = (NQ + 3) / 4;     // int8 QK^T row tiles: 4 queries x 4 digits
  static constexpr int KS = HD / 64;           // int8 QK^T k-steps (64 channels)
  // queries a weight / rescale row of LDS holds (the PV tiles may cover more
  // than the QK^T tiles: hd 64 puts 8 queries in a PV tile)
  static constexpr int NQS = (NT2 * 4 > NT * QVT) ? NT2 * 4 : NT * QVT;
  static_assert(HD == 64 || HD == 128, "head dim");
  static_assert(QVT * LPQ == 64, "one q~ tile per wave pass");
};

// One chunk's loads.
template <int HD, int NQ>
struct MBuf {
  using C = MCfg<HD, NQ>;
  uint4 k[2][C::KL];  // K: granule h, load jp
  float4 ks[2];       // the K group's channel scales of this lane's 8 q~ channels
  uint4 v[C::VL];     // V: load tp
  float vs[8];        // V block scale of slot s (position 16(s/4) + 4g + s%4, block col % NBK)
};

// finish() for the nr <= NR query rows [row0, row0 + nr) of a workgroup:
// the cross-wave combine of each (row, head), then the output (single split)
// or the split's record of each row; every thread combines its head's waves
// itself, with finish()'s arithmetic.
template <int HD, int G, int NR>
__device__ __forceinline__ void finish_rows(const AttnParams& P,
                                            float (&s_o)[kWaves][NR * G][HD],
                                            float (&s_ml)[kWaves][NR * G][2], int split, int kh,
                                            int row0, int nr) {
  __syncthreads();
  auto combine = [&](int q, float& M, float (&f)[kWaves], float& L) {
    float m[kWaves], l[kWaves];
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      m[i] = s_ml[i][q][0];
      l[i] = s_ml[i][q][1];
    }
    M = kMinit;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) M = fmaxf(M, m[i]);
    L = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      f[i] = fast_exp2(m[i] - M);
      L += l[i] * f[i];
    }
  };
  auto o_of = [&](int q, int d, const float (&f)[kWaves]) {
    float O = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) O += s_o[i][q][d] * f[i];
    return O;
  };
  if (P.direct) {
    for (int idx = threadIdx.x; idx < nr * G * HD; idx += kThreads) {
      const int q = idx / HD, d = idx % HD, r = q / G, g = q % G;
      float M, f[kWaves], L;
      combine(q, M, f, L);
      P.out[((static_cast<size_t>(row0 + r) * P.n_heads + kh * G + g) * HD) + d] = o_of(q, d, f) / L;
    }
    return;
  }
  constexpr int PR = G * HD + 2 * G;  // floats a row's record receives
  for (int idx = threadIdx.x; idx < nr * PR; idx += kThreads) {
    const int r = idx / PR, rem = idx % PR;
    const size_t head_base = static_cast<size_t>(row0 + r) * P.nkv + kh;
    float* orec = P.part + head_base * record_region(P.nsplit, G, HD) +
                  static_cast<size_t>(split) * record_floats(G, HD);
    const int g = rem < G * HD ? rem / HD : (rem - G * HD) >> 1;
    float M, f[kWaves], L;
    combine(r * G + g, M, f, L);
    if (rem < G * HD) {
      __hip_atomic_store(orec + rem, o_of(r * G + g, rem % HD, f), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      const int k = rem - G * HD;  // (m, l) of head k / 2
      __hip_atomic_store(orec + G * HD + k, (k & 1) ? L : M, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// NR: query rows per workgroup (chunk rows: a verify round's rows share
// every K/V byte and its bf16 conversion; decode and the fused step: 1).
template <int HD, int G, bool PROD, int CPW, int NR>
__global__ __launch_bounds__(kThreads) void attn_i8_kernel(const AttnParams P, const AppendArgs A) {
  constexpr int NQ = NR * G;
  using C = MCfg<HD, NQ>;
  constexpr int NBK = C::NBK, QVT = C::QVT, NT = C::NT, LPQ = C::LPQ;
  constexpr int KL = C::KL, NTV = C::NTV, VL = C::VL;
  constexpr int NT2 = C::NT2, KS = C::KS, NQS = C::NQS;
  constexpr int CHUNK = kKGroup;
  constexpr int NB = NBK;

  static_assert(NR == 1 || !PROD, "raw projections: decode (one row) only");
  constexpr bool kFuse = NR == 1;  // the fused decode step (one row) only
  __shared__ float s_o[kWaves][NQ][HD];
  __shared__ float s_ml[kWaves][NQ][2];
  __shared__ int s_slice[NR];
  // q~ digits: the int8 QK^T A operand of row tile T2, k-step jp, lane
  // group g, row m (lane m + 16 g reads [T2][jp][g][m]: 16 consecutive
  // bytes per lane, no bank conflicts)
  __shared__ __align__(16) uint4 s_qd[kWaves][NT2][KS][4][16];
  __shared__ float s_qsc[kWaves][NT2 * 4];       // 2^-S of each query's digits
  __shared__ __align__(16) float s_p[kWaves][NQS][32];  // chunk weights (masked: -1)
  __shared__ float s_al[kWaves][NQS];            // rescale factor of each query
  // fused step stages (the single head group's)
  __shared__ __align__(16) AppStage s_stage;
  __shared__ __align__(16) float s_row[PROD ? 768 : 256];
  __shared__ __align__(16) float s_raw[kFuse ? kWaves / 2 : 1][kFuse ? kKGroup * HD / (kWaves / 2) : 4];
  __shared__ __align__(16) uint8_t s_kgbuf[kFuse ? sizeof(KGroupStage) : 16];
  KGroupStage& s_kg = *reinterpret_cast<KGroupStage*>(s_kgbuf);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;    // matrix column / row group of this lane
  const int qvl = lane / LPQ, c8 = lane % LPQ;   // q~ layout: query qvl, channels 8*c8..
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int row0 = blockIdx.z * NR;              // this workgroup's rows [row0, row0 + nr)
  const int nr = min(NR, P.rows - row0);
  const int nqv = nr * G;                        // its query vectors (row r, head g: r*G + g)
  const int nkeys = P.pos0 + row0 + nr;          // keys of its last row
  const int nchunks = (nkeys + CHUNK - 1) / CHUNK;
  const int c_end = min((split + 1) * P.chunks_per_split, nchunks);
  const size_t head = static_cast<size_t>(kh) * P.capg;
  const size_t head_el = head * HD;
  const int app_chunk = kFuse && A.slot >= 0 ? A.slot / CHUNK : -1;
  const bool app_here = app_chunk >= split * P.chunks_per_split && app_chunk < c_end;

  const int kv_bytes = P.capg * HD;
  const rsrc_t rk = make_rsrc(P.k8 + head_el, kv_bytes);
  const rsrc_t rv = make_rsrc(P.v8 + head_el, kv_bytes);
  const rsrc_t rks = make_rsrc(P.ks + static_cast<size_t>(kh) * P.ng * HD, P.ng * HD * 4);
  const rsrc_t rvs = make_rsrc(P.vs + head * NB, P.capg * NB * 4);

  using Buf = MBuf<HD, NQ>;
  // one chunk buffer, refilled half by half (issue_k, issue_v) as the
  // chunk's math frees it
  constexpr int NBUF = 1;

  // Every chunk issues the same loads, so the load waits are exact; a chunk
  // past c_end reads from p0 = capg, past the end of every array (reads
  // return 0). The group a fused step requantizes is read as well and
  // replaced from LDS.
  // A chunk's K half (codes, the group's channel scales) and V half (codes,
  // block scales) are issued separately: the next chunk's K goes out as soon
  // as this chunk's QK^T has read its K registers, its V as soon as PV has
  // read V, so a wave always has loads in flight instead of waiting for its
  // whole chunk before requesting the next.
  auto chunk_p0 = [&](int ch) {
    return __builtin_amdgcn_readfirstlane(ch < c_end ? ch * CHUNK : P.capg);
  };
  // Scales go out before codes: loads return in issue order, so the q~
  // digits (q * the group's channel scales) and the PV weights (p * the V
  // block scales) are built while the chunk's codes are still arriving.
  auto issue_k = [&](Buf& b, int ch) {
    const int p0 = chunk_p0(ch);
    const int base = p0 * HD;
    const int so = (p0 / kKGroup) * HD * 4;
    b.ks[0] = load_b128(rks, 32 * c8, so);
    b.ks[1] = load_b128(rks, 32 * c8 + 16, so);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int jp = 0; jp < KL; ++jp)
        b.k[h][jp] = __builtin_bit_cast(uint4, stream_b128(rk, lane * 16, base + (h * KL + jp) * 1024));
  };
  auto issue_v = [&](Buf& b, int ch) {
    const int p0 = chunk_p0(ch);
    const int base = p0 * HD;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      b.vs[s] = load_b32(rvs, ((16 * (s / 4) + 4 * grp + s % 4) * NB + col % NBK) * 4, p0 * NB * 4);
#pragma unroll
    for (int tp = 0; tp < VL; ++tp)
      b.v[tp] = __builtin_bit_cast(uint4, stream_b128(rv, lane * 16, base + tp * 1024));
  };

  // ---- q * scale * log2(e) of this lane's 8 channels of query T*QVT + qvl
  // (padding queries >= nqv are 0)
  float qs[NT][8];
  const bool q_prod = PROD && (P.qb != nullptr || P.qcs != nullptr);  // uniform
  auto load_q = [&]() {
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int qv = min(T * QVT + qvl, nqv - 1);
      const float* qg =
          P.q + (static_cast<size_t>(row0 + qv / G) * P.n_heads + kh * G + qv % G) * HD;
      const float4 a = *reinterpret_cast<const float4*>(qg + 8 * c8);
      const float4 b = *reinterpret_cast<const float4*>(qg + 8 * c8 + 4);
      qs[T][0] = a.x; qs[T][1] = a.y; qs[T][2] = a.z; qs[T][3] = a.w;
      qs[T][4] = b.x; qs[T][5] = b.y; qs[T][6] = b.z; qs[T][7] = b.w;
    }
  };
  // Raw projections: q + qb, then the fp64 rope, as the producer computes
  // each element. Every wave needs the whole of q, and producing it per wave
  // would wait on q's loads before the stream's loads go out (the rope reads
  // them), a round trip ahead of the stream. Instead one rope pair per
  // thread: its raw loads go out first (they return first), the pair is
  // produced after the first chunk's loads are issued, and the waves read q
  // from LDS (one row: query qv is head g).
  constexpr int H2 = HD / 2;
  static_assert(!PROD || NQ * H2 <= kThreads, "one rope pair per thread");
  __shared__ __align__(16) float s_qp[PROD ? NQ * HD : 4];
  const int qp_v = threadIdx.x / H2, qp_j = threadIdx.x % H2;
  const bool qp_on = q_prod && qp_v < nqv;
  float qp_a = 0.0f, qp_b = 0.0f, qp_ba = 0.0f, qp_bb = 0.0f;
  double2 qp_cs = make_double2(1.0, 0.0);
  auto load_q_raw = [&]() {
    if (qp_on) {
      const float* qg = P.q + (static_cast<size_t>(row0) * P.n_heads + kh * G + qp_v) * HD;
      qp_a = qg[qp_j];
      qp_b = qg[qp_j + H2];
      if (P.qb != nullptr) {
        const float* bg = P.qb + (kh * G + qp_v) * HD;
        qp_ba = bg[qp_j];
        qp_bb = bg[qp_j + H2];
      }
      if (P.qcs != nullptr) qp_cs = P.qcs[qp_j];
    }
  };

  // ---- fused decode step (FusedAppend, one head group): the owner wave
  // stages the new row; waves [0, RW) requantize its K group before their
  // own chunk and publish it through an LDS count
  using App = FusedAppend<HD, kI8Dense, PROD>;
  const int app_rel = app_chunk - split * P.chunks_per_split;
  const bool app_owner = app_here && wave == app_rel % kWaves;  // wave-uniform
  const bool app_share = app_here && wave < App::RW;
  float* app_raw = s_raw[wave < App::RW ? wave : 0];
  if (app_here) {  // workgroup-uniform
    if (threadIdx.x == 0) s_kg.done = 0;
    __syncthreads();
  }
  if (q_prod)
    load_q_raw();
  else
    load_q();
  typename App::ShareIn app_knew{};
  typename App::RowIn app_in{};
  if (app_share) App::load_share(A, kh, wave, lane, app_knew);
  if (app_owner) App::load_row(A, kh, lane, app_in);
  // the fp32 sinks' K and V rows (wave 0 of split 0): their loads go out
  // with q, ahead of the stream, and their scores are taken before the
  // wave's chunk, so attending them after the stream waits on no load. A
  // fused step's own sink row comes from the step's inputs.
  constexpr int SB = 4;  // sinks taken at entry (further ones after the stream)
  const int ns = min(P.n_sink, nkeys);  // sinks of the last row (a row r sees pos0 + r + 1 keys)
  const bool sink_wave = split == 0 && wave == 0 && ns > 0;  // wave-uniform
  const bool fresh_sink = kFuse && A.slot >= 0 && A.pos < P.n_sink;
  // Raw projections: the step's own sink row (k + kb roped, v + vb) is
  // produced once per workgroup into LDS with q, not per lane inline (whose
  // loads and fp64 temporaries would set the kernel's register peak).
  const bool fresh_prod = PROD && A.prod && fresh_sink && split == 0 && ns > 0;  // uniform
  __shared__ __align__(16) float s_fresh[PROD ? 2 * HD : 4];
  bool fresh_ready = false;
  auto fresh_row = [&](float (&kx)[8], float (&vx)[8]) {
    const float4 k0 = *reinterpret_cast<const float4*>(&s_fresh[8 * c8]);
    const float4 k1 = *reinterpret_cast<const float4*>(&s_fresh[8 * c8 + 4]);
    const float4 v0 = *reinterpret_cast<const float4*>(&s_fresh[HD + 8 * c8]);
    const float4 v1 = *reinterpret_cast<const float4*>(&s_fresh[HD + 8 * c8 + 4]);
    kx[0] = k0.x; kx[1] = k0.y; kx[2] = k0.z; kx[3] = k0.w;
    kx[4] = k1.x; kx[5] = k1.y; kx[6] = k1.z; kx[7] = k1.w;
    vx[0] = v0.x; vx[1] = v0.y; vx[2] = v0.z; vx[3] = v0.w;
    vx[4] = v1.x; vx[5] = v1.y; vx[6] = v1.z; vx[7] = v1.w;
  };
  // thread t < hd/2: the K pair (t, t + hd/2); hd/2 <= t < 3 hd/2: V element
  // t - hd/2 (produced<HD>() element by element)
  float fr_a = 0.0f, fr_b = 0.0f, fr_ba = 0.0f, fr_bb = 0.0f;
  double2 fr_cs = make_double2(1.0, 0.0);
  auto load_fresh_raw = [&]() {
    const int t = threadIdx.x;
    if (t < H2) {
      fr_a = A.k[kh * HD + t];
      fr_b = A.k[kh * HD + t + H2];
      if (A.kb != nullptr) {
        fr_ba = A.kb[kh * HD + t];
        fr_bb = A.kb[kh * HD + t + H2];
      }
      if (A.kcs != nullptr) fr_cs = A.kcs[t];
    } else if (t < H2 + HD) {
      fr_a = A.v[kh * HD + t - H2];
      if (A.vb != nullptr) fr_ba = A.vb[kh * HD + t - H2];
    }
  };
  auto produce_fresh = [&]() {
    const int t = threadIdx.x;
    if (t < H2) {
      float a = fr_a, b = fr_b;
      if (A.kb != nullptr) {
        a += fr_ba;
        b += fr_bb;
      }
      if (A.kcs != nullptr) rope_pair(a, b, fr_cs);
      s_fresh[t] = a;
      s_fresh[t + H2] = b;
    } else if (t < H2 + HD) {
      s_fresh[HD + t - H2] = A.vb != nullptr ? fr_a + fr_ba : fr_a;
    }
  };
  auto produce_q = [&]() {  // workgroup-uniform (q_prod or fresh_prod)
    if (qp_on) {
      float u = qp_a, w = qp_b;
      if (P.qb != nullptr) {
        u += qp_ba;
        w += qp_bb;
      }
      if (P.qcs != nullptr) rope_pair(u, w, qp_cs);
      s_qp[qp_v * HD + qp_j] = u;
      s_qp[qp_v * HD + qp_j + H2] = w;
    }
    if (fresh_prod) produce_fresh();
    __syncthreads();
    if (q_prod) {
#pragma unroll
      for (int T = 0; T < NT; ++T) {
        const int qv = min(T * QVT + qvl, nqv - 1);
        const float4 a = *reinterpret_cast<const float4*>(&s_qp[qv * HD + 8 * c8]);
        const float4 b = *reinterpret_cast<const float4*>(&s_qp[qv * HD + 8 * c8 + 4]);
        qs[T][0] = a.x; qs[T][1] = a.y; qs[T][2] = a.z; qs[T][3] = a.w;
        qs[T][4] = b.x; qs[T][5] = b.y; qs[T][6] = b.z; qs[T][7] = b.w;
      }
    }
  };
  auto sink_rows = [&](int p, float (&kx)[8], float (&vx)[8]) {
    const float* ksb = P.ksink + static_cast<size_t>(kh) * P.n_sink * HD;
    const float* vsb = P.vsink + static_cast<size_t>(kh) * P.n_sink * HD;
    const float4* ks4 = reinterpret_cast<const float4*>(ksb + p * HD + 8 * c8);
    const float4* vs4 = reinterpret_cast<const float4*>(vsb + p * HD + 8 * c8);
    const float4 k0 = ks4[0], k1 = ks4[1], v0 = vs4[0], v1 = vs4[1];
    kx[0] = k0.x; kx[1] = k0.y; kx[2] = k0.z; kx[3] = k0.w;
    kx[4] = k1.x; kx[5] = k1.y; kx[6] = k1.z; kx[7] = k1.w;
    vx[0] = v0.x; vx[1] = v0.y; vx[2] = v0.z; vx[3] = v0.w;
    vx[4] = v1.x; vx[5] = v1.y; vx[6] = v1.z; vx[7] = v1.w;
    if (fresh_sink && p == A.pos) {  // uniform
      if (PROD && A.prod) {
        // produced once per workgroup (s_fresh): read from there once it is
        // ready, patched in after the production for the entry sinks
        if (fresh_ready) fresh_row(kx, vx);
      } else {
        const float* kin = A.k + kh * HD;
        const float* vin = A.v + kh * HD;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kx[e] = kin[8 * c8 + e];
          vx[e] = vin[8 * c8 + e];
        }
      }
    }
  };
  // a sink's score for this lane's query: q (scaled) . k over the LPQ lanes
  // of the query (hd 128: a 16-lane row); -inf past the row's sinks
  auto sink_dot = [&](const float (&qv8)[8], const float (&kx)[8], bool seen) {
    float sdot = qv8[0] * kx[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) sdot += qv8[e] * kx[e];
    if constexpr (LPQ == 16) sdot += dpp<kX8>(sdot);
    sdot += dpp<kX7>(sdot);
    sdot += dpp<kX2>(sdot);
    sdot += dpp<kX1>(sdot);
    return seen ? sdot : -INFINITY;
  };
  float skx[SB][8], svx[SB][8];
  if (fresh_prod) load_fresh_raw();
  if (sink_wave) {
#pragma unroll
    for (int u = 0; u < SB; ++u) sink_rows(min(u, ns - 1), skx[u], svx[u]);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int ch0 = split * P.chunks_per_split + wave;  // chunk t of this wave: ch0 + t * 8
  Buf RA;
  // every wave's K half of its first chunk goes out before any V half: a
  // CU's loads are served roughly in issue order, so the waves that issue
  // last would otherwise get their whole chunk last and do all of its math
  // after the stream; this way all K arrives in the first part of the
  // stream, QK^T and the softmax overlap the V half, and only PV follows it
  issue_k(RA, ch0);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  issue_v(RA, ch0);
  __builtin_amdgcn_sched_barrier(0);
  if (q_prod || fresh_prod) {  // workgroup-uniform
    produce_q();
    fresh_ready = true;
    if (fresh_prod && sink_wave) {
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (min(u, ns - 1) == A.pos) fresh_row(skx[u], svx[u]);  // uniform
    }
  }
  if (app_share) App::requant_share(A, wave, lane, app_knew, app_raw, s_kg);
#pragma unroll
  for (int T = 0; T < NT; ++T)
#pragma unroll
    for (int e = 0; e < 8; ++e) qs[T][e] = T * QVT + qvl < nqv ? qs[T][e] * P.qscale : 0.0f;
  float ssd[NT][SB];  // the first SB sinks' scores
  if (sink_wave) {
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int qv = T * QVT + qvl;
      const int nsq = min(P.n_sink, P.pos0 + row0 + (qv < nqv ? qv / G : 0) + 1);
#pragma unroll
      for (int u = 0; u < SB; ++u) ssd[T][u] = sink_dot(qs[T], skx[u], u < nsq);
    }
  }

  // running state: per QK^T row tile, the max and the lane's partial sum of
  // the query of its lane group (query 4 T2 + grp), and the PV accumulators
  // (row (query, block), column = channel of tile t)
  float M[NT2], l[NT2];
  f32x4 o[NT][NTV];
#pragma unroll
  for (int T2 = 0; T2 < NT2; ++T2) {
    M[T2] = kMinit;
    l[T2] = 0.0f;
  }
#pragma unroll
  for (int T = 0; T < NT; ++T)
#pragma unroll
    for (int t = 0; t < NTV; ++t) o[T][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // the owner's V chunk block with the new row patched in, kept for the
  // flush (the producer instance above 4 query heads writes the row's bytes
  // instead: its registers are full)
  constexpr bool kKeepV = !PROD || NQ <= 4;
  uint4 app_v[kKeepV ? VL : 1];
  // next >= 0: the chunk whose loads go into b as this chunk frees it
  auto compute = [&](Buf& b, const int ch, const bool first, const int next) {
    // products feeding split3 are rounded to fp32 first (q * ks, as the
    // reference rounds it; p * vs): no contraction into the split's subtraction
#pragma clang fp contract(off)
    const int p0 = ch * CHUNK;

    // ---- the fused step's chunk: its K group and the new V row from LDS
    if (kFuse && ch == app_chunk) {  // uniform
      App::put_row(A, app_in, lane, s_row);
      if (PROD && A.prod) App::produce_row(A, lane, s_row);
      App::stage_row(A, lane, s_stage, s_row);
      App::await_shares(s_kg);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int jp = 0; jp < KL; ++jp) b.k[h][jp] = s_kg.kchunk[(h * KL + jp) * 64 + lane];
      b.ks[0] = *reinterpret_cast<const float4*>(&s_kg.ks[8 * c8]);
      b.ks[1] = *reinterpret_cast<const float4*>(&s_kg.ks[8 * c8 + 4]);
      const int pc = A.slot - p0;  // the row's position in the chunk
      const int sg = (pc & 15) >> 2, ss = 4 * (pc >> 4) + (pc & 3);
      if (grp == sg && A.pos >= A.n_sink) {  // (a sink row is masked in the stream)
        const uint8_t* v8s = reinterpret_cast<const uint8_t*>(s_stage.v8row);
#pragma unroll
        for (int tp = 0; tp < VL; ++tp) {
          uint32_t w[4] = {b.v[tp].x, b.v[tp].y, b.v[tp].z, b.v[tp].w};
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const uint32_t code = v8s[16 * (2 * tp + tt) + col];
            const int bi = 8 * tt + ss, sh = 8 * (bi & 3);
#pragma unroll
            for (int c4 = 2 * tt; c4 < 2 * tt + 2; ++c4)
              w[c4] = c4 == (bi >> 2) ? (w[c4] & ~(0xFFu << sh)) | (code << sh) : w[c4];
          }
          b.v[tp] = make_uint4(w[0], w[1], w[2], w[3]);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) b.vs[s] = s == ss ? s_stage.vs[col % NBK] : b.vs[s];
      }
      // every lane's part of the patched V block, for the flush
      if constexpr (kKeepV) {
#pragma unroll
        for (int tp = 0; tp < VL; ++tp) app_v[tp] = b.v[tp];
      }
    }

    // ---- q~ of this chunk's K group as exact base-256 digits, into LDS.
    // Per query, X = trunc(q~ * 2^S) with S fitting |X| < 2^30, and
    // X = sum_i 256^i D_i with balanced digits D_i in [-128, 127] (the
    // bytes of (X + 0x80808080) ^ 0x80808080). Digit i of query q is row
    // 4 (q % 4) + i of row tile q / 4; the lane's 8 channels are 8 bytes of
    // one A operand (channel 64 jp + 32 j2 + 8 g + e at byte 8 j2 + e, the
    // order of the K codes in the B operand).
    {
      const float ks8[8] = {b.ks[0].x, b.ks[0].y, b.ks[0].z, b.ks[0].w,
                            b.ks[1].x, b.ks[1].y, b.ks[1].z, b.ks[1].w};
      const int jp = c8 / 8, j2 = (c8 / 4) % 2, gq = c8 % 4;
#pragma unroll
      for (int T = 0; T < NT; ++T) {
        const int qv = T * QVT + qvl;
        float x[8], mx = 0.0f, nf = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] = qs[T][e] * ks8[e];
          mx = fmaxf(mx, fabsf(x[e]));
          nf += x[e];
        }
        // the query's max over its LPQ lanes; nf becomes NaN when any of its
        // q~ is not finite (the digits cannot carry it: the scale below does)
        nf *= 0.0f;
        mx = fmaxf(mx, dpp<kX1>(mx));
        nf += dpp<kX1>(nf);
        mx = fmaxf(mx, dpp<kX2>(mx));
        nf += dpp<kX2>(nf);
        mx = fmaxf(mx, dpp<kX7>(mx));
        nf += dpp<kX7>(nf);
        if constexpr (LPQ == 16) {
          mx = fmaxf(mx, dpp<kX8>(mx));
          nf += dpp<kX8>(nf);
        }
        const int ex = __builtin_amdgcn_frexp_expf(mx);  // mx < 2^ex
        const float up = __builtin_amdgcn_ldexpf(1.0f, 30 - ex);
        uint32_t d[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          d[e] = (static_cast<uint32_t>(static_cast<int>(x[e] * up)) + 0x80808080u) ^ 0x80808080u;
        uint32_t lo[4], hi[4];
        byte_planes({d[0], d[1], d[2], d[3]}, lo);
        byte_planes({d[4], d[5], d[6], d[7]}, hi);
        if (qv < NT2 * 4) {
          uint8_t* rowb = reinterpret_cast<uint8_t*>(&s_qd[wave][qv / 4][jp][gq][0]) + 8 * j2;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint2*>(rowb + 16 * (4 * (qv % 4) + i)) = make_uint2(lo[i], hi[i]);
          if (c8 == 0) s_qsc[wave][qv] = __builtin_amdgcn_ldexpf(1.0f, ex - 30) + nf;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- QK^T on the int8 matrix cores: row 4 g + i of tile T2 = digit i
    // of query 4 T2 + g, column = position 16 h + col; every product and
    // sum is exact in int32. The score combines the digits in fp32.
    float sc[2][NT2];
    {
      i32x4 acc[2][NT2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int T2 = 0; T2 < NT2; ++T2) acc[h][T2] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int jp = 0; jp < KS; ++jp)
#pragma unroll
        for (int T2 = 0; T2 < NT2; ++T2) {
          const i32x4 a = __builtin_bit_cast(i32x4, s_qd[wave][T2][jp][grp][col]);
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[h][T2] = mfma_i8(a, b.k[h][jp], acc[h][T2]);
        }
#pragma unroll
      for (int T2 = 0; T2 < NT2; ++T2) {
        const float down = s_qsc[wave][4 * T2 + grp];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const i32x4 a = acc[h][T2];
          float t = static_cast<float>(a[3]);
          t = fmaf(t, 256.0f, static_cast<float>(a[2]));
          t = fmaf(t, 256.0f, static_cast<float>(a[1]));
          t = fmaf(t, 256.0f, static_cast<float>(a[0]));
          sc[h][T2] = t * down;
        }
      }
    }

    if (next >= 0) {  // uniform: this chunk's K registers are read
      __builtin_amdgcn_sched_barrier(0);
      issue_k(b, next);
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- online softmax per query (its 16 lanes hold the chunk's 32
    // positions, two each); the weights go to LDS for the PV A operand
#pragma unroll
    for (int T2 = 0; T2 < NT2; ++T2) {
      const int qv = 4 * T2 + grp;
      // keys of this query's row (causal: row r attends [0, pos0 + r])
      const int nk = qv < nqv ? P.pos0 + row0 + qv / G + 1 : 0;
      float sv[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int p = p0 + 16 * h + col;
        sv[h] = p < nk && p >= P.n_sink ? sc[h][T2] : -INFINITY;
      }
      const float mn = fmaxf(M[T2], row16_max(fmaxf(sv[0], sv[1])));
      const float alpha = first ? 0.0f : fast_exp2(M[T2] - mn);
      M[T2] = mn;
      const float p0w = fast_exp2(sv[0] - mn), p1w = fast_exp2(sv[1] - mn);
      l[T2] = first ? p0w + p1w : fmaf(l[T2], alpha, p0w + p1w);
      // masked slots: -1, weighed exactly 0 (their stale V scales may be anything)
      s_p[wave][qv][col] = sv[0] != -INFINITY ? p0w : -1.0f;
      s_p[wave][qv][16 + col] = sv[1] != -INFINITY ? p1w : -1.0f;
      if (col == 0) s_al[wave][qv] = alpha;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- PV: A = weight x V block scale in three bf16 parts, row (query,
    // block) = col, k = the lane's 8 positions 16 (s / 4) + 4 grp + s % 4
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int qv = T * QVT + col / NBK;
      const float4 pa = *reinterpret_cast<const float4*>(&s_p[wave][qv][4 * grp]);
      const float4 pb = *reinterpret_cast<const float4*>(&s_p[wave][qv][16 + 4 * grp]);
      const float pk[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      float w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = pk[k] >= 0.0f ? pk[k] * b.vs[k] : 0.0f;
      uint4 aw[3];
      split3(w, aw);
      // the rescale of output rows 4 grp + i: query T QVT + (4 grp + i) / NBK
      if (!first) {
        if constexpr (NBK == 4) {
          const float ar = s_al[wave][T * QVT + grp];
#pragma unroll
          for (int t = 0; t < NTV; ++t) o[T][t][t / 2] *= ar;
        } else {
          const float a0 = s_al[wave][T * QVT + 2 * grp];
          const float a1 = s_al[wave][T * QVT + 2 * grp + 1];
#pragma unroll
          for (int t = 0; t < NTV; ++t) {
            o[T][t][t / 2] *= a0;
            o[T][t][2 + t / 2] *= a1;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NTV; ++t) {
        const uint4 vw = b.v[t / 2];
        const bf16x8 bv = (t & 1) ? codes_bf16(vw.z, vw.w) : codes_bf16(vw.x, vw.y);
#pragma unroll
        for (int a = 0; a < 3; ++a) o[T][t] = mfma(aw[a], bv, o[T][t]);
      }
    }
    if (next >= 0) {  // uniform: this chunk's V registers are read
      __builtin_amdgcn_sched_barrier(0);
      issue_v(b, next);
    }
    __builtin_amdgcn_wave_barrier();
  };

  static_assert(NBUF == 1, "the next chunk's loads reuse the one buffer");
  if constexpr (CPW > 0) {
#pragma unroll
    for (int t = 0; t < CPW; ++t) {
      const int cht = ch0 + t * kWaves;
      if (cht < c_end) compute(RA, cht, t == 0, t + 1 < CPW ? cht + kWaves : -1);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    int ch = ch0;
    bool first = true;
    while (ch < c_end) {
      compute(RA, ch, first, ch + kWaves);
      first = false;
      __builtin_amdgcn_sched_barrier(0);
      ch += kWaves;
    }
  }

  // ---- wave state to LDS: (m, l) by the lanes of block-0 columns of row
  // group 0, o by the lane holding (query, channel) (row 4*grp + i of tile t
  // is query (4*grp + i) / NBK at block (4*grp + i) % NBK; kept when that is
  // the tile's block t / 2). A wave without a chunk writes (kMinit, 0, 0).
#pragma unroll
  for (int T2 = 0; T2 < NT2; ++T2) {
    const float lt = row16_sum(l[T2]);
    const int qv = 4 * T2 + grp;
    if (col == 0 && qv < NQ) {
      s_ml[wave][qv][0] = M[T2];
      s_ml[wave][qv][1] = lt;
    }
  }
#pragma unroll
  for (int T = 0; T < NT; ++T) {
#pragma unroll
    for (int t = 0; t < NTV; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * grp + i, q = T * QVT + r / NBK;
        if (r % NBK == t / 2 && q < NQ) s_o[wave][q][16 * t + col] = o[T][t][i];
      }
  }

  // ---- the fp32 sinks (positions < n_sink, model.cpp:612-626), folded into
  // wave 0's record of split 0 (q~ layout: lane = query qvl, channels
  // 8*c8..): the first SB from the scores and V rows taken at entry
  if (sink_wave) {  // wave-uniform
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int qv = T * QVT + qvl;
      const bool real = qv < nqv;
      const int nsq = min(P.n_sink, P.pos0 + row0 + (real ? qv / G : 0) + 1);  // this row's sinks
      float Ms = real ? s_ml[0][qv][0] : kMinit, Ls = real ? s_ml[0][qv][1] : 0.0f, os[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) os[e] = real ? s_o[0][qv][8 * c8 + e] : 0.0f;
      auto update = [&](float sdot, const float (&vx)[8]) {
        const float mn = fmaxf(Ms, sdot);
        const float al = fast_exp2(Ms - mn), pw = fast_exp2(sdot - mn);
        Ms = mn;
        Ls = fmaf(Ls, al, pw);
#pragma unroll
        for (int e = 0; e < 8; ++e) os[e] = fmaf(os[e], al, pw * vx[e]);
      };
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (u < ns) update(ssd[T][u], svx[u]);  // uniform
      // further blocks of SB sinks, every load of a block in flight at once
      for (int pb = SB; pb < ns; pb += SB) {
        float kx[SB][8], vx[SB][8];
#pragma unroll
        for (int u = 0; u < SB; ++u) sink_rows(min(pb + u, ns - 1), kx[u], vx[u]);
#pragma unroll
        for (int u = 0; u < SB; ++u)
          if (pb + u < ns) update(sink_dot(qs[T], kx[u], pb + u < nsq), vx[u]);  // uniform
      }
      if (real) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[0][qv][8 * c8 + e] = os[e];
        if (c8 == 0) {
          s_ml[0][qv][0] = Ms;
          s_ml[0][qv][1] = Ls;
        }
      }
    }
  }

  finish_rows<HD, G, NR>(P, s_o, s_ml, split, kh, row0, nr);
  if (!P.direct) {
    // this thread's record stores have reached the coherence point
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    arrive_and_merge<HD, G, NR>(P, kh, row0, nr, wave, lane, s_slice);
  }
  if (kFuse && app_owner)
    App::flush(A, kh, lane, s_stage, &s_kg, s_row, kKeepV ? app_v : nullptr);
}

// The largest rows-per-workgroup a (hd, G) instance serves: its query
// vectors fill at most three 16-column tiles (registers), and at most 4 rows.
__host__ __device__ constexpr int i8_max_rows(int HD, int G) {
  return (3 * (16 / (HD / kBlock))) / G < 4 ? (3 * (16 / (HD / kBlock))) / G : 4;
}

// CPW: chunks per wave of the plan (1, 2, 4 unrolled; 0 a runtime loop).
template <int HD, int G, bool PROD, int NR>
void* i8_kernel_cpw(int cpw) {
  if constexpr (NR > i8_max_rows(HD, G) || (PROD && NR > 1)) {
    return nullptr;
  } else {
    switch (cpw) {
      case 1: return reinterpret_cast<void*>(&attn_i8_kernel<HD, G, PROD, 1, NR>);
      case 2: return reinterpret_cast<void*>(&attn_i8_kernel<HD, G, PROD, 2, NR>);
      case 4: return reinterpret_cast<void*>(&attn_i8_kernel<HD, G, PROD, 4, NR>);
      default: return reinterpret_cast<void*>(&attn_i8_kernel<HD, G, PROD, 0, NR>);
    }
  }
}

template <int HD, bool PROD, int NR>
void* pick_i8(int G, int cpw) {
  switch (G) {
    case 1: return i8_kernel_cpw<HD, 1, PROD, NR>(cpw);
    case 2: return i8_kernel_cpw<HD, 2, PROD, NR>(cpw);
    case 3: return i8_kernel_cpw<HD, 3, PROD, NR>(cpw);
    case 4: return i8_kernel_cpw<HD, 4, PROD, NR>(cpw);
    case 5: return i8_kernel_cpw<HD, 5, PROD, NR>(cpw);
    case 6: return i8_kernel_cpw<HD, 6, PROD, NR>(cpw);
    case 7: return i8_kernel_cpw<HD, 7, PROD, NR>(cpw);
    case 8: return i8_kernel_cpw<HD, 8, PROD, NR>(cpw);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace dbi
