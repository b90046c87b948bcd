// GQA attention kernel over the three cache layouts (model.cpp:567-728)
// and the causal chunk rows of decode_layer_chunk (model.cpp:956-981).
// Instantiated by attn_inst_*.hip (one translation unit per layout and
// producer flag, compiled in parallel); dispatched by attention.hip.
//
// Design (CDNA4, wave64):
//  - Grid (split, kv_head, query_row), 8 waves per workgroup. A workgroup
//    streams one contiguous range of key positions of ONE kv head and serves
//    all G = gqa query heads of that head from the same bytes, so K/V cross
//    HBM once per kv head (the reference re-reads them per query head,
//    model.cpp:575-596).
//  - A wave handles 32-position chunks (16 for the ring and for wide fp32
//    groups), chunk t -> wave t % 8, in the granule layout of
//    kv_internal.hpp: every load instruction reads 64 lanes x 8 elements,
//    contiguous. A "lane row" of LPR = hd/8 lanes holds one position; RPW =
//    64/LPR rows per instruction.
//  - QK: each lane keeps the partial dots of its 8 dims for the NSG slots of
//    a granule. K's slot order is permuted per lane (kslot_xor) so that the
//    16-lane (hd 128) or 8-lane (hd 64) reduction is a transposing one: three
//    DPP adds halve the slots and sum across lanes at once, and every lane
//    ends up holding ONE position's full score (each position in 4 lanes).
//    Softmax then runs once per position instead of once per lane row.
//  - Softmax: wave-uniform running max (DPP row max, row_bcast15/31,
//    readlane), exp2 with scale*log2(e) folded into q; weights go through a
//    per-wave LDS buffer to the PV lane mapping (lane = 8 consecutive V dims
//    of one position row).
//  - Loads: K of the next chunk is issued right after QK, V of the next
//    chunk right after PV, so one of them is always in flight.
//  - Split-K: each split writes (o[G][HD], m[G], l[G]) of its range with
//    agent-coherent stores, waits for them, and counts itself in a per
//    (row, kv head) counter with one device-scope atomic. The split that
//    arrives last merges every split (and the sinks) and resets the counter,
//    so no second launch, no fence (an agent-scope fence is a whole-L2
//    writeback on this multi-XCD part) and no memset between launches.
//  - int8 dense: a 32-position chunk is exactly one K group, so the
//    per-channel K scale folds into q once per chunk (the reference's
//    (q_i * ks_i) * k8_i); codes are signed bytes, converted with one
//    sign-extending SDWA v_cvt_f32_i32 each. The fp32 sinks (pos < n_sink)
//    are attended in the merge as further entries.
//  - Fused decode step (dbi_kv_decode): the append of the new row runs
//    inside the launch (FusedAppend), staged in LDS for the wave that
//    attends its chunk.
//  - ring: keys are stored un-roped; each resident key is dequantized (int8:
//    per-block scale) and roped at its cache-relative position from an fp32
//    cos/sin table, q at n_res - 1 (model.cpp:662-700). K lanes hold dims d
//    and d + hd/2 together, so the rotation is lane-local.
#pragma once

#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "kv_internal.hpp"
#include "quant.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSplits = 64;  // one split per lane in the merge
// split-arrival counters sit 256 bytes apart: the atomics of different
// (row, kv head) pairs never share a cache line
constexpr int kCounterStride = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMinit = -1.0e30f;  // finite: exp2(kMinit - kMinit) == 1, no NaN
// Lazy reference maximum of the chunk-rows kernels' softmax: it moves only
// when a score passes it by more than 2^kLazyLog2 (so every weight is at
// most 2^kLazyLog2, exact in the three-part splits and far from fp32's
// range); otherwise alpha is exactly 1 and the rescale is skipped.
constexpr float kLazyLog2 = 8.0f;
__device__ __forceinline__ float lazy_max(float m, float cm) { return cm > m + kLazyLog2 ? cm : m; }

enum Kind { kF32Dense = 0, kI8Dense = 1, kF32Ring = 2, kI8Ring = 3 };

struct AttnParams {
  const float* kf;
  const float* vf;
  const uint8_t* k8;
  const uint8_t* v8;
  const float* ks;
  const float* vs;
  const float* ksink;
  const float* vsink;
  const float2* rope;
  int rope_rows;
  const float* q;
  // decode from raw projections (rows == 1): q bias [n_heads*hd] or null, and
  // the (cos, sin) row of the decode position for a dense rope, or null
  const float* qb;
  const double2* qcs;
  float* out;
  float* part;
  unsigned* cnt;  // split arrivals per (row, kv head), zero between launches
  int capg, ng, n_sink, nkv, n_heads;
  int rows, pos0;
  int ring_nres, ring_s, ring_W, ring_base;
  int nsplit;  // splits (partial records) per (row, kv head)
  int direct;  // 1: single split and no sinks, write the output directly;
               // 0: write a partial record, the last split to arrive merges
  int chunks_per_split;
  float qscale;
};

// ---------------------------------------------------------------------------
// cross-lane helpers

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// DPP controls: lane ^ 8 within a 16-lane row (row_ror:8), lane ^ 7 within
// 8 lanes (row_half_mirror), lane ^ 2 and lane ^ 1 (quad_perm).
constexpr int kX8 = 0x128, kX7 = 0x141, kX2 = 0x4E, kX1 = 0xB1;

// Row-broadcast step of a wave reduction: rows in ROWMASK combine with the
// last lane of the row(s) before them, the other rows with `idle`.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float bcast(float x, float idle) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, idle), __builtin_bit_cast(int, x),
                                         CTRL, ROWMASK, 0xF, false));
}

__device__ __forceinline__ float lane63(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Wave-uniform max / sum of one value per lane.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kX8>(v));
  v = fmaxf(v, dpp<kX7>(v));
  v = fmaxf(v, dpp<kX2>(v));
  v = fmaxf(v, dpp<kX1>(v));
  v = fmaxf(v, bcast<0x142, 0xA>(v, v));  // row_bcast:15
  v = fmaxf(v, bcast<0x143, 0xC>(v, v));  // row_bcast:31
  return lane63(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kX8>(v);
  v += dpp<kX7>(v);
  v += dpp<kX2>(v);
  v += dpp<kX1>(v);
  v += bcast<0x142, 0xA>(v, 0.0f);
  v += bcast<0x143, 0xC>(v, 0.0f);
  return lane63(v);
}

// gfx950 permlane swaps, emitted through asm (the compiler's builtins fold
// the two results into one when both are used). swap32(a, b): lanes 0-31
// end with {own a, a of lane + 32}, lanes 32-63 with {b of lane - 32, own
// b}; swap16 does the same between even and odd 16-lane rows. a + b after
// the swap is therefore a's pair sum in the lower half and b's in the upper.
__device__ __forceinline__ float swap32_sum(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}
// Raw v_exp_f32 (2^x). Softmax weights below 2^-126 are far under the
// output tolerance, so the denormal-range handling of exp2f is not needed.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// tensor::rope's fp64 NeoX rotation of one pair (ops.cpp:31-34): products
// and sums rounded one by one, as the reference's scalar code does
__device__ __forceinline__ void rope_pair(float& a, float& b, double2 cs) {
#pragma clang fp contract(off)
  const double x = static_cast<double>(a) * cs.x - static_cast<double>(b) * cs.y;
  const double y = static_cast<double>(b) * cs.x + static_cast<double>(a) * cs.y;
  a = static_cast<float>(x);
  b = static_cast<float>(y);
}

// Element d of one head row as the reference's host code hands it to the
// cache (model.cpp:747-763): x + bias (one fp32 add; no add without a
// bias), then, with a (cos, sin) row, the rope of its pair (d, d +- hd/2).
template <int HD>
__device__ __forceinline__ float produced(const float* x, const float* bias, const double2* cs,
                                          int d) {
  constexpr int H2 = HD / 2;
  const int j = d % H2;
  float a = x[j], b = x[j + H2];
  if (bias != nullptr) {
    a += bias[j];
    b += bias[j + H2];
  }
  if (cs != nullptr) rope_pair(a, b, cs[j]);
  return d < H2 ? a : b;
}

// Raw buffer resources (gfx9 descriptor word 3 = 0x00020000: 32-bit raw
// data, bounds-checked against num_records bytes; reads past it return 0).
using rsrc_t = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}
__device__ __forceinline__ float4 load_b128(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float2 load_b64(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ float load_b32(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
// K/V rows are read once per call: non-temporal (gfx940+ cache policy NT)
constexpr int kNT = 2;
__device__ __forceinline__ float4 stream_b128(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNT));
}

// 8 int8 codes -> float (one sign-extending SDWA v_cvt_f32_i32 each)
__device__ __forceinline__ void cvt8(const uint2 w, float* f) {
#pragma unroll
  for (int b = 0; b < 4; ++b) f[b] = static_cast<float>(static_cast<int8_t>(w.x >> (8 * b)));
#pragma unroll
  for (int b = 0; b < 4; ++b) f[4 + b] = static_cast<float>(static_cast<int8_t>(w.y >> (8 * b)));
}

template <int HD, int G, int KIND>
struct Cfg {
  static constexpr bool kInt8 = (KIND == kI8Dense || KIND == kI8Ring);
  static constexpr bool kRing = (KIND == kF32Ring || KIND == kI8Ring);
  static constexpr int LPR = HD / 8;            // lanes per position row
  static constexpr int RPW = 64 / LPR;          // rows per load instruction
  static constexpr int NSG = kGranule / RPW;    // slots per granule
  static constexpr int NGC = 1;                 // granules per chunk
  static constexpr int CHUNK = kGranule * NGC;
  static constexpr int NS = NSG * NGC;          // slots per chunk
  // every wave holds q and o of all G heads (up to 8 x 16 registers each):
  // each chunk is streamed, and for a ring roped, once per kv head
  static constexpr int NHG = 1;
  static constexpr int GW = (G + NHG - 1) / NHG;  // query heads per wave
  static constexpr int WPG = kWaves / NHG;        // waves per head group
  static constexpr int GP = GW <= 4 ? 4 : 8;      // padded heads of an LDS weight row
  static constexpr int DUP = LPR / NSG;         // lanes holding one position's score
  static constexpr int NB = HD / kBlock;
  static_assert(HD == 64 || HD == 128, "head dim");
  // dense int8 runs on the matrix-core kernel (attn_mfma.hpp)
  static_assert(KIND != kI8Dense, "dense int8: attn_i8_kernel");
};

// Reduces the NSG per-slot partial dots of a lane row to full scores, one
// position per lane (lane c of the row ends with granule slot kslot_xor(c)).
template <int HD>
__device__ __forceinline__ float treduce(const float* a) {
  float t;
  if constexpr (HD == 128) {
    const float s0 = a[0] + dpp<kX8>(a[2]);
    const float s1 = a[1] + dpp<kX8>(a[3]);
    t = s0 + dpp<kX7>(s1);
  } else {
    t = a[0] + dpp<kX7>(a[1]);
  }
  t += dpp<kX2>(t);
  t += dpp<kX1>(t);
  return t;
}

// Fused decode step (Model::decode_layer's kv.append then attend,
// model.cpp:759-771): the row of one position, appended by the workgroup
// whose split holds its storage chunk (FusedAppend below).
struct AppendArgs {
  const float* k;  // new row, device [nkv][hd]; nullptr: no append
  const float* v;
  // raw-projection step: the row is k + kb roped by kcs (dense) and v + vb;
  // each may be null (no bias / no rope); prod = any of them set
  const float* kb;
  const float* vb;
  const double2* kcs;
  int prod;
  int slot;        // storage row (dense: pos; ring: slot_for(pos)); -1: no append
  int pos;
  int nkv, n_sink, capg, ng;
  float* kf;       // this layer's arrays, writable
  float* vf;
  uint8_t* k8;
  uint8_t* v8;
  float* ks;
  float* vs;
  float* k_raw;    // dense int8 staging [32][nkv*hd]
  float* ksink;
  float* vsink;
};

// One split's record: o [G][HD], then (m, l) [G] in a 128-byte tail of
// its own (records written by workgroups on different XCDs share no cache
// line), 16-byte aligned throughout for the merge's loads.
__host__ __device__ constexpr int record_floats(int G, int HD) { return G * HD + 32; }
// Floats of one (row, kv head)'s records, [nsplit] of them.
__host__ __device__ constexpr size_t record_region(int nsplit, int G, int HD) {
  return static_cast<size_t>(nsplit) * record_floats(G, HD);
}

// Cross-wave combine of (m, l, o) in LDS, then either the final output
// (single split) or this split's partial record. Head g was handled by the
// WPG waves of head group g / GW, at their local head index g % GW. Every
// thread derives its head's combined max and wave factors itself from the
// waves' (m, l) (broadcast LDS reads), so one barrier orders the whole step.
template <int HD, int G, int GW, int WPG>
__device__ __forceinline__ void finish(const AttnParams& P, float (&s_o)[kWaves][GW][HD],
                                       float (&s_ml)[kWaves][GW][2], int split, int kh,
                                       int qrow) {
  __syncthreads();
  // head g: combined max M, weight f[i] of wave i, combined sum L
  auto combine = [&](int g, float& M, float (&f)[WPG], float& L) {
    const int w0 = (g / GW) * WPG, gl = g % GW;
    float m[WPG], l[WPG];
#pragma unroll
    for (int i = 0; i < WPG; ++i) {
      m[i] = s_ml[w0 + i][gl][0];
      l[i] = s_ml[w0 + i][gl][1];
    }
    M = kMinit;
#pragma unroll
    for (int i = 0; i < WPG; ++i) M = fmaxf(M, m[i]);
    L = 0.0f;
#pragma unroll
    for (int i = 0; i < WPG; ++i) {
      f[i] = fast_exp2(m[i] - M);
      L += l[i] * f[i];
    }
  };
  auto o_of = [&](int g, int d, const float (&f)[WPG]) {
    const int w0 = (g / GW) * WPG, gl = g % GW;
    float O = 0.0f;
#pragma unroll
    for (int i = 0; i < WPG; ++i) O += s_o[w0 + i][gl][d] * f[i];
    return O;
  };
  const size_t head_base = static_cast<size_t>(qrow) * P.nkv + kh;
  if (P.direct) {
    float* out_base = P.out + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
      const int g = idx / HD, d = idx % HD;
      float M, f[WPG], L;
      combine(g, M, f, L);
      out_base[idx] = o_of(g, d, f) / L;
    }
    return;
  }
  // this split's records: o [G][HD] in the region's o part, (m, l) [G] in
  // its (m, l) part; written through to the device coherence point (the
  // merging workgroup may run on another XCD, behind another L2)
  float* orec = P.part + head_base * record_region(P.nsplit, G, HD) +
                static_cast<size_t>(split) * record_floats(G, HD);
  float* mlrec = orec + G * HD;
  for (int idx = threadIdx.x; idx < G * HD + 2 * G; idx += kThreads) {
    const int g = idx < G * HD ? idx / HD : (idx - G * HD) >> 1;
    float M, f[WPG], L;
    combine(g, M, f, L);
    if (idx < G * HD) {
      __hip_atomic_store(orec + idx, o_of(g, idx % HD, f), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      const int r = idx - G * HD;  // (m, l) of head r / 2
      __hip_atomic_store(mlrec + r, (r & 1) ? L : M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The split merge of one (row, kv head), run by the workgroup whose split
// arrived last (each split counts itself in P.cnt after its record stores
// completed; the last one resets the count for the next launch). Wave g
// merges query head g: the (m, l) of split s in lane s give the split weights
// (DPP max / sum); the o records are read 16 bytes per lane, HD / 4 lanes
// per record, so one load instruction covers 64 / (HD / 4) splits, every
// load of the merge in one round. Records are read at device coherence.
// SINKS: the dense int8 fp32 sinks (positions < n_sink, model.cpp:612-626)
// of this row are attended here too (the rows kernels leave them to the
// merge): their scores join the split maxima, their V rows the sum.
// MAXS (32 or 64) bounds nsplit: the loads and sums are straight-line over
// MAXS splits (splits past nsplit reload the last record and weigh 0), and
// each lane fetches the weight of its split from the split's lane with an
// independent ds_bpermute; a per-split branch and readlane chain, with its
// SGPR hazards, cost ~1.2 us per merge at 32 splits.
template <int HD, int G, bool SINKS = false, int MAXS = kMaxSplits>
__device__ __forceinline__ void merge_head(const AttnParams& P, int kh, int qrow, int g, int lane) {
  constexpr int kSC1 = 16;  // cache policy: agent-coherent load
  constexpr int LPH = HD / 4;       // lanes per record of one head
  constexpr int SPI = 64 / LPH;     // splits per load instruction
  constexpr int NI = MAXS / SPI;
  static_assert(MAXS <= kMaxSplits, "split bound");
  const size_t head_base = static_cast<size_t>(qrow) * P.nkv + kh;
  constexpr int RF = record_floats(G, HD);
  const float* region = P.part + head_base * record_region(P.nsplit, G, HD);
  const rsrc_t ro = make_rsrc(region, P.nsplit * RF * 4);
  const bool on = lane < P.nsplit;
  const float2 ml = __builtin_bit_cast(
      float2, __builtin_amdgcn_raw_buffer_load_b64(ro, (min(lane, P.nsplit - 1) * RF + G * HD + 2 * g) * 4,
                                                   0, kSC1));
  const int sub = lane / LPH, dl = lane % LPH;  // split within an instruction, dims 4dl..
  float4 ov[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int sp = min(k * SPI + sub, P.nsplit - 1);
    ov[k] = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(ro, (sp * RF + g * HD + 4 * dl) * 4, 0,
                                                      kSC1));
  }
  // the sinks' scores (uniform): q * scale * log2 e (as the kernels scale it)
  // against each sink's K row, dims lane and lane + 64 of each lane
  constexpr int SB = 4;  // sinks whose loads go out together and stay in registers
  constexpr int DPL = HD / 64;
  const int nsq = SINKS ? min(P.n_sink, P.pos0 + qrow + 1) : 0;  // this row's sinks
  const float* ksb = SINKS ? P.ksink + static_cast<size_t>(kh) * P.n_sink * HD : nullptr;
  const float* vsb = SINKS ? P.vsink + static_cast<size_t>(kh) * P.n_sink * HD : nullptr;
  float Ms = kMinit;
  float qd[DPL];
  float sd0[SB];   // scores of the first SB sinks (uniform), their V rows (dims 4 lane ..)
  float4 vx0[SB];
  auto sink_dot = [&](const float (&kx)[DPL]) {
    float sd = qd[0] * kx[0];
#pragma unroll
    for (int u = 1; u < DPL; ++u) sd += qd[u] * kx[u];
    return wave_sum(sd);
  };
  if constexpr (SINKS) {
    const float* qp = P.q + (static_cast<size_t>(qrow) * P.n_heads + kh * G + g) * HD;
#pragma unroll
    for (int u = 0; u < DPL; ++u) qd[u] = qp[lane + 64 * u] * P.qscale;
    float kx[SB][DPL];
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      const int p = min(b, nsq - 1);
#pragma unroll
      for (int u = 0; u < DPL; ++u) kx[b][u] = ksb[p * HD + lane + 64 * u];
      vx0[b] = *reinterpret_cast<const float4*>(vsb + p * HD + 4 * (lane % LPH));
    }
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      sd0[b] = sink_dot(kx[b]);
      if (b < nsq) Ms = fmaxf(Ms, sd0[b]);
    }
    for (int pb = SB; pb < nsq; ++pb) {  // further sinks (uniform), one at a time
      float ky[DPL];
#pragma unroll
      for (int u = 0; u < DPL; ++u) ky[u] = ksb[pb * HD + lane + 64 * u];
      Ms = fmaxf(Ms, sink_dot(ky));
    }
  }
  const float M = fmaxf(wave_max(on ? ml.x : kMinit), Ms);
  const float w = on ? fast_exp2(ml.x - M) : 0.0f;  // splits past nsplit weigh 0
  float L = wave_sum(on ? ml.y * w : 0.0f);
  float4 acc[2] = {make_float4(0.0f, 0.0f, 0.0f, 0.0f), make_float4(0.0f, 0.0f, 0.0f, 0.0f)};
  // weight of this lane's split of instruction k, from lane k * SPI + sub
  // (0 past nsplit); the fetches are independent of each other
  float ws[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k)
    ws[k] = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute(4 * (k * SPI + sub), __builtin_bit_cast(int, w)));
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    float4& a = acc[k & 1];
    a.x = fmaf(ws[k], ov[k].x, a.x);
    a.y = fmaf(ws[k], ov[k].y, a.y);
    a.z = fmaf(ws[k], ov[k].z, a.z);
    a.w = fmaf(ws[k], ov[k].w, a.w);
  }
  float o4[4] = {acc[0].x + acc[1].x, acc[0].y + acc[1].y, acc[0].z + acc[1].z,
                 acc[0].w + acc[1].w};
  // the SPI lane groups hold other splits of the same dims: sum them
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o4[e] = swap32_sum(o4[e], o4[e]);
    if constexpr (SPI == 4) o4[e] = swap16_sum(o4[e], o4[e]);
  }
  if constexpr (SINKS) {
    // the sinks' weights against M, and their V rows (dims 4 lane .. of the
    // lanes holding the output)
    auto add_sink = [&](float sd, const float4& v) {
      const float pw = fast_exp2(sd - M);
      L += pw;
      o4[0] = fmaf(pw, v.x, o4[0]);
      o4[1] = fmaf(pw, v.y, o4[1]);
      o4[2] = fmaf(pw, v.z, o4[2]);
      o4[3] = fmaf(pw, v.w, o4[3]);
    };
#pragma unroll
    for (int b = 0; b < SB; ++b)
      if (b < nsq) add_sink(sd0[b], vx0[b]);
    for (int pb = SB; pb < nsq; ++pb) {  // further sinks: scores recomputed as above
      float ky[DPL];
#pragma unroll
      for (int u = 0; u < DPL; ++u) ky[u] = ksb[pb * HD + lane + 64 * u];
      add_sink(sink_dot(ky), *reinterpret_cast<const float4*>(vsb + pb * HD + 4 * (lane % LPH)));
    }
  }
  if (lane < LPH) {
    const size_t h = static_cast<size_t>(qrow) * P.n_heads + kh * G + g;
    const float inv = 1.0f / L;
    *reinterpret_cast<float4*>(P.out + h * HD + 4 * lane) =
        make_float4(o4[0] * inv, o4[1] * inv, o4[2] * inv, o4[3] * inv);
  }
}
// merge_head with the split bound of the plan (uniform choice)
template <int HD, int G, bool SINKS = false>
__device__ __forceinline__ void merge_split(const AttnParams& P, int kh, int qrow, int g,
                                            int lane) {
  if (P.nsplit <= 32)
    merge_head<HD, G, SINKS, 32>(P, kh, qrow, g, lane);
  else
    merge_head<HD, G, SINKS, kMaxSplits>(P, kh, qrow, g, lane);
}

// Re-reads of a counter before a waiting merger gives up (a bound only: the
// arrival it waits for belongs to a workgroup that is already running and
// waits on nothing).
constexpr int kSpinLimit = 1 << 22;

// Records a single merging workgroup reads before the merge is spread over
// several: its CU fetches them at ~64 bytes per clock plus a round trip
// (~1 us for C3's 3 heads x 32 records), while handing slices to other
// workgroups costs a round trip of its own (measured slower at C3).
constexpr int kOneMergerBytes = 96 << 10;

// Split arrival and merge of the decode kernels, after this workgroup's
// records have reached the coherence point; thread r < nr counts row
// row0 + r. A (row, kv head) counter holds (epoch << 8) | arrivals. The
// last D arrivals each merge one slice of the query heads (slice m: heads
// m, m + D, ..): D = 1 unless the records exceed kOneMergerBytes (a C4 ring
// call: 7 heads x 33 records), then D = min(G, nsplit), so the records are
// read by D workgroups on D CUs. The last arrival moves the counter to the
// next epoch (arrivals back to 0, with no wait) and merges its slice; the
// other mergers wait until the epoch moves, which the last arrival does
// right after its own count: every record was acknowledged before its
// split was counted, so all of them are at the coherence point by then.
template <int HD, int G, int NR>
__device__ __forceinline__ void arrive_and_merge(const AttnParams& P, int kh, int row0, int nr,
                                                 int wave, int lane, int (&s_slice)[NR]) {
  const int D = P.nsplit * G * HD * 4 > kOneMergerBytes ? min(G, P.nsplit) : 1;
  if (static_cast<int>(threadIdx.x) < nr) {
    unsigned* cnt =
        P.cnt + (static_cast<size_t>(row0 + threadIdx.x) * P.nkv + kh) * kCounterStride;
    const unsigned before =
        __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int a = static_cast<int>(before & 0xFFu);
    const int slice = a - (P.nsplit - D);
    if (a == P.nsplit - 1) {
      (void)__hip_atomic_fetch_add(cnt, 256u - static_cast<unsigned>(P.nsplit), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    } else if (slice >= 0) {
      const unsigned epoch = before >> 8;
      for (int it = 0; it < kSpinLimit &&
                       (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 8) == epoch;
           ++it)
        __builtin_amdgcn_s_sleep(1);
    }
    s_slice[threadIdx.x] = slice;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int slice = r < nr ? s_slice[r] : -1;  // uniform
    const int g = slice + wave * D;
    if (slice >= 0 && g < G) merge_split<HD, G>(P, kh, row0 + r, g, lane);
  }
}


// LDS stage of a fused step's new values, in the layouts the attention
// reads them in, for the wave that processes the appended chunk.
struct AppStage {
  float ks[4];                       // ring int8: the new row's K block scales
  float vs[4];                       // int8: the new row's V block scales
  float krow[128];                   // fp32: the new K row
  float vrow[128];                   // fp32: the new V row
  uint32_t k8row[32];                // ring int8: the new K codes
  uint32_t v8row[32];                // int8: the new V codes
};

// Dense int8: the requantized 32-token group of the fused step, shared by
// the head groups of the workgroup.
struct KGroupStage {
  uint4 kchunk[kKGroup * 128 / 16];  // the group's codes, dense int8 layout
  float ks[128];                     // its channel scales
  unsigned done;                     // requantizing waves done (zeroed at launch)
};

// One kv head's part of KVCache::append (model.cpp:357-404) inside the
// attention kernel, with the arithmetic of the append kernels (quant.hpp):
// fp32 rows are copied; int8 ring rows are block-quantized (a 32-element
// block spans 16 lanes, two elements per lane); dense int8 stages the raw K
// row and requantizes its 32-token group per channel, and block-quantizes
// V, or stores both as fp32 sinks when pos < n_sink. New values go to LDS
// stages in the layouts the attention reads, and to global memory only
// after the writing wave's last load (a store in flight would hold back its
// next wait on loads).
//
// Work split: the wave (of each head group) that attends the new row's
// chunk, the owner, stages the row itself. The dense int8 group
// requantization (32 codes per channel, far too long for one wave's
// critical path) is shared by the first RW waves of the workgroup, CPW
// channels each, before their own chunk: their loads go out first, so the
// shares are done by the time the owner (usually a later wave) reaches the
// new row's chunk. They publish through an LDS counter that only the owners
// wait on; no other wave waits. (Measured: all 8 waves sharing, or the 4
// waves just before the owner, made the step slower.)
//
// Loads are ordinary 16-byte vector loads into registers (the compiler's
// load waits stay exact), written to LDS where they are consumed: the new K
// and V rows into `row` ([0, HD) and [HD, 2 HD) of 256 floats; k_dev and
// v_dev are 16-byte aligned) and a wave's channels of the group's 32 staged
// raw rows into its `raw` share ([32][CPW]).
template <int HD, int KIND, bool PROD>
struct FusedAppend {
  static constexpr bool kInt8 = (KIND == kI8Dense || KIND == kI8Ring);
  static constexpr int NB = HD / kBlock;
  static constexpr int RW = kWaves / 2;       // dense int8: requantizing waves
  static constexpr int CPW = HD / RW;         // channels per requantizing wave
  static constexpr int RPL = kKGroup * CPW / 64;  // raw rows per lane of a share

  __device__ __forceinline__ static void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // The owner's inputs, 16 bytes per lane, loaded into registers ahead and
  // written to the LDS row where they are consumed (ordinary loads: the
  // compiler's load waits stay exact): the K row in lanes [0, HD/4), the V
  // row in [HD/4, HD/2) (hd 64: lanes past HD/2 repeat them into row[2 HD,
  // 4 HD)); raw projections add the (cos, sin) row and the K / V biases.
  // (native vectors: copies into LDS stay register stores)
  using v4f = float __attribute__((ext_vector_type(4)));
  struct RowIn {
    v4f kv, cs, bias;
  };
  __device__ __forceinline__ static void load_row(const AppendArgs& A, int kh, int lane,
                                                  RowIn& in) {
    constexpr int Q = HD / 4;         // lanes per row
    const int hl = lane % (2 * Q);
    in.kv = *reinterpret_cast<const v4f*>((hl < Q ? A.k : A.v) + kh * HD + (hl % Q) * 4);
    if (PROD && A.prod) {  // raw projections: the (cos, sin) row and the biases too
      if (A.kcs != nullptr)
        in.cs = *reinterpret_cast<const v4f*>(A.kcs + lane % (HD / 2));
      if (A.kb != nullptr || A.vb != nullptr) {  // a missing one is loaded but not added
        const float* kb = A.kb != nullptr ? A.kb : A.vb;
        const float* vb = A.vb != nullptr ? A.vb : A.kb;
        in.bias = *reinterpret_cast<const v4f*>((hl < Q ? kb : vb) + kh * HD + (hl % Q) * 4);
      }
    }
  }
  // the row into LDS (K [0, HD), V [HD, 2 HD); raw projections: [256, 512)
  // the (cos, sin) row, [512, 768) the biases)
  __device__ __forceinline__ static void put_row(const AppendArgs& A, const RowIn& in, int lane,
                                                 float* row) {
    reinterpret_cast<v4f*>(row)[lane] = in.kv;
    if (PROD && A.prod) {
      reinterpret_cast<v4f*>(row + 256)[lane] = in.cs;
      reinterpret_cast<v4f*>(row + 512)[lane] = in.bias;
    }
    wave_sync();
  }

  // raw projections, owner wave, after put_row(): the row in LDS becomes
  // k + kb roped and v + vb, exactly as produced() computes each element
  __device__ __forceinline__ static void produce_row(const AppendArgs& A, int lane, float* row) {
    constexpr int H2 = HD / 2;
    const float* bias = row + 512;  // kb [0, HD), vb [HD, 2 HD)
    if (lane < H2) {
      float a = row[lane], b = row[lane + H2];
      if (A.kb != nullptr) {
        a += bias[lane];
        b += bias[lane + H2];
      }
      if (A.kcs != nullptr) rope_pair(a, b, reinterpret_cast<const double2*>(row + 256)[lane]);
      row[lane] = a;
      row[lane + H2] = b;
    }
    if (A.vb != nullptr && 2 * lane < HD) {
      row[HD + 2 * lane] += bias[HD + 2 * lane];
      row[HD + 2 * lane + 1] += bias[HD + 2 * lane + 1];
    }
    wave_sync();
  }

  // the loaded inputs of a share's channel of the new K row: the value
  // (raw projections: the pair's raw values and biases and its (cos, sin),
  // combined only after the wait, so no wait stalls the share's loads)
  static constexpr int LPRW = CPW / 4, RPI = 64 / LPRW;  // lanes per share row, rows per load
  struct ShareIn {
    float x0, x1, b0, b1;
    double2 cs;
    v4f raw[kKGroup / RPI];  // the share's raw rows, 16 bytes per lane per load
  };
  __device__ __forceinline__ static float share_value(const AppendArgs& A, const ShareIn& in,
                                                      int d) {
    if constexpr (PROD) {
      if (A.prod) {
        float a = in.x0, b = in.x1;
        if (A.kb != nullptr) {
          a += in.b0;
          b += in.b1;
        }
        if (A.kcs != nullptr) rope_pair(a, b, in.cs);
        return d % HD < HD / 2 ? a : b;
      }
    }
    return in.x0;
  }

  // dense int8, wave < RW: its share of the group's raw rows (into
  // registers) and its channel of the new K row (lane l holds channel
  // l % CPW of the share)
  __device__ __forceinline__ static void load_share(const AppendArgs& A, int kh, int wave,
                                                    int lane, ShareIn& in) {
    const size_t P_ = static_cast<size_t>(A.nkv) * HD;
    const float* src = A.k_raw + static_cast<size_t>(lane / LPRW) * P_ + kh * HD + wave * CPW +
                       (lane % LPRW) * 4;
#pragma unroll
    for (int m = 0; m < kKGroup / RPI; ++m)
      in.raw[m] = *reinterpret_cast<const v4f*>(src + m * RPI * P_);
    const int d = wave * CPW + lane % CPW;
    if (PROD && A.prod) {
      const int j = d % (HD / 2);
      const float* x = A.k + kh * HD;
      in.x0 = x[j];
      in.x1 = x[j + HD / 2];
      if (A.kb != nullptr) {
        in.b0 = A.kb[kh * HD + j];
        in.b1 = A.kb[kh * HD + j + HD / 2];
      }
      if (A.kcs != nullptr) in.cs = A.kcs[j];
    } else {
      in.x0 = A.k[kh * HD + d];
    }
  }

  // dense int8, wave < RW: requantize_kgroup
  // (model.cpp:329-355) of the wave's CPW channels over raw rows
  // [0, within] that are not sinks (row `within` is the new one). Lane l
  // takes channel l % CPW over RPL rows; the channel max combines its lanes
  // by xor shuffles. Rows outside the range count |x| * 0 (0, or a NaN that
  // max_f skips as it skips NaN inputs) and their codes are neither
  // attended (masked positions) nor flushed.
  __device__ __forceinline__ static void requant_share(const AppendArgs& A, int wave, int lane,
                                                       const ShareIn& in, float* raw,
                                                       KGroupStage& kg) {
    const int within = A.pos % kKGroup, first = A.pos - within;
    const int c = lane % CPW, rb = lane / CPW;
#pragma unroll
    for (int m = 0; m < kKGroup / RPI; ++m)
      reinterpret_cast<v4f*>(raw + m * RPI * CPW)[lane] = in.raw[m];
    const float knew = share_value(A, in, wave * CPW + c);
    wave_sync();
    if (lane < CPW) raw[within * CPW + c] = knew;
    wave_sync();
    float x[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) x[i] = raw[(rb * RPL + i) * CPW + c];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int w = rb * RPL + i;
      m = max_f(m, fabsf(x[i]) * ((w <= within && first + w >= A.n_sink) ? 1.0f : 0.0f));
    }
#pragma unroll
    for (int off = CPW; off < 64; off <<= 1) m = max_f(m, __shfl_xor(m, off));
    const float sc = m / 127.0f;
    const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
    uint8_t* kc = reinterpret_cast<uint8_t*>(kg.kchunk);
    const int d = wave * CPW + c;
#pragma unroll
    for (int i = 0; i < RPL; ++i)
      kc[k_off_i8d(HD, rb * RPL + i, d)] = static_cast<uint8_t>(quant_code(x[i], inv));
    if (lane < CPW) kg.ks[d] = sc;
    // publish (the release orders the stage writes before the count)
    if (lane == 0) __hip_atomic_fetch_add(&kg.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  // dense int8 owner: wait until all RW shares are published
  __device__ __forceinline__ static void await_shares(const KGroupStage& kg) {
    while (__hip_atomic_load(&kg.done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           static_cast<unsigned>(RW))
      __builtin_amdgcn_s_sleep(1);
  }

  // quant_head of a 32-element block held two per lane by 16 lanes
  __device__ __forceinline__ static float block_scale(float2 x) {
    float m = max_f(fabsf(x.x), fabsf(x.y));
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) m = max_f(m, __shfl_xor(m, off, 16));
    return m / 127.0f;
  }
  __device__ __forceinline__ static uint32_t codes2(float2 x, float s) {
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    const uint32_t a = static_cast<uint8_t>(quant_code(x.x, inv));
    const uint32_t b = static_cast<uint8_t>(quant_code(x.y, inv));
    return a | (b << 8);
  }

  // owner wave, after put_row(): the row's own values into its stage
  // (dense int8: V only; the K group is requant_share's)
  __device__ __forceinline__ static void stage_row(const AppendArgs& A, int lane, AppStage& st,
                                                   const float* row) {
    const bool on = 2 * lane < HD;
    const int d = 2 * lane;
    const float2 kx = on ? *reinterpret_cast<const float2*>(row + d) : float2{};
    const float2 vx = on ? *reinterpret_cast<const float2*>(row + HD + d) : float2{};
    uint16_t* k8s = reinterpret_cast<uint16_t*>(st.k8row);
    uint16_t* v8s = reinterpret_cast<uint16_t*>(st.v8row);
    if constexpr (!kInt8) {
      if (on) {
        *reinterpret_cast<float2*>(&st.krow[d]) = kx;
        *reinterpret_cast<float2*>(&st.vrow[d]) = vx;
      }
    } else if constexpr (KIND == kI8Ring) {
      const float sk = block_scale(kx), sv = block_scale(vx);
      if (on) {
        k8s[lane] = static_cast<uint16_t>(codes2(kx, sk));
        v8s[lane] = static_cast<uint16_t>(codes2(vx, sv));
        if (d % kBlock == 0) {
          st.ks[d / kBlock] = sk;
          st.vs[d / kBlock] = sv;
        }
      }
    } else if (A.pos < A.n_sink) {
      if (on) {
        v8s[lane] = 0;  // a sink position is masked in the stream; keep the stage finite
        if (d % kBlock == 0) st.vs[d / kBlock] = 0.0f;
      }
    } else {
      const float sv = block_scale(vx);
      if (on) {
        v8s[lane] = static_cast<uint16_t>(codes2(vx, sv));
        if (d % kBlock == 0) st.vs[d / kBlock] = sv;
      }
    }
    wave_sync();
  }

  // The stages to global memory in whole contiguous pieces, by one wave per
  // kv head, after its last load.
  // (kg: the dense int8 group stage; null for the other layouts)
  // vblock (dense int8, optional): the new row's whole V chunk block as the
  // owner holds it, 16 bytes per lane per 1 KiB piece (the chunk's V loads
  // with the row's codes patched in); written back in whole lines instead of
  // the row's bytes scattered one per 16-byte unit
  __device__ __forceinline__ static void flush(const AppendArgs& A, int kh, int lane,
                                               const AppStage& st, const KGroupStage* kg,
                                               const float* row,
                                               const uint4* vblock = nullptr) {
    const bool on = 2 * lane < HD;
    const int d = 2 * lane;
    const size_t hel = static_cast<size_t>(kh) * A.capg * HD;
    constexpr int LPR = HD / 8, RPW = 64 / LPR;
    const int pg = A.slot & 15, rr = pg % RPW, ii = pg / RPW;  // the row's granule slot
    if constexpr (KIND == kI8Dense) {
      const int pos = A.pos, grp = pos / kKGroup, within = pos % kKGroup, first = pos - within;
#pragma unroll 4
      for (int m = 0; m < kKGroup * HD / 8 / 64; ++m) {  // one 8-byte piece per lane each
        // (a piece is 8 channels of one position: 1 KiB block o / 1024 of
        // granule block / (hd / 64), position n of lane (o % 1024) / 16)
        const int o = (m * 64 + lane) * 8;
        const int w = kGranule * ((o / 1024) / (HD / 64)) + ((o % 1024) / 16) % 16;
        if (w <= within && first + w >= A.n_sink)  // later rows and sinks keep their memory
          *reinterpret_cast<uint2*>(A.k8 + hel + static_cast<size_t>(first) * HD + o) =
              *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(kg->kchunk) + o);
      }
      if (on) {
        const float2 kx = *reinterpret_cast<const float2*>(row + d);
        *reinterpret_cast<float2*>(A.ks + (static_cast<size_t>(kh) * A.ng + grp) * HD + d) =
            *reinterpret_cast<const float2*>(&kg->ks[d]);
        *reinterpret_cast<float2*>(A.k_raw + static_cast<size_t>(within) * A.nkv * HD + kh * HD +
                                   d) = kx;
        if (pos < A.n_sink) {
          const size_t at = (static_cast<size_t>(kh) * A.n_sink + pos) * HD + d;
          *reinterpret_cast<float2*>(A.ksink + at) = kx;
          *reinterpret_cast<float2*>(A.vsink + at) = *reinterpret_cast<const float2*>(row + HD + d);
        }
      }
      if (pos >= A.n_sink) {
        if (vblock != nullptr) {  // the chunk's V block, HD / 32 pieces of 1 KiB
          uint8_t* vb = A.v8 + hel + static_cast<size_t>(pos / kKGroup) * kKGroup * HD;
#pragma unroll
          for (int tp = 0; tp < HD / 32; ++tp)
            *reinterpret_cast<uint4*>(vb + tp * 1024 + lane * 16) = vblock[tp];
        } else if (on) {  // V row: one byte per channel (channels d, d + 1 of this lane)
          const uint8_t* v8s = reinterpret_cast<const uint8_t*>(st.v8row);
          A.v8[hel + v_off_i8d(HD, pos, d)] = v8s[d];
          A.v8[hel + v_off_i8d(HD, pos, d + 1)] = v8s[d + 1];
        }
        if (lane < NB) A.vs[(static_cast<size_t>(kh) * A.capg + pos) * NB + lane] = st.vs[lane];
      }
    } else if constexpr (KIND == kI8Ring) {
      if (lane < LPR) {
        const int c = lane, j = ii ^ kslot_xor(HD, c);
        *reinterpret_cast<uint2*>(A.k8 + hel + granule_off(HD, true, A.slot, j, rr * LPR + c, 0)) =
            make_uint2(st.k8row[c], st.k8row[HD / 8 + c]);
        *reinterpret_cast<uint2*>(A.v8 + hel + granule_off(HD, true, A.slot, ii, rr * LPR + c, 0)) =
            make_uint2(st.v8row[2 * c], st.v8row[2 * c + 1]);
      }
      if (lane < NB) {
        const size_t srow = static_cast<size_t>(kh) * A.capg + A.slot;
        A.ks[srow * NB + lane] = st.ks[lane];
        A.vs[srow * NB + lane] = st.vs[lane];
      }
    } else {
      if (lane < LPR) {
        const int c = lane, j = ii ^ kslot_xor(HD, c);
        float* kdst = A.kf + hel + granule_off(HD, false, A.slot, j, rr * LPR + c, 0);
        *reinterpret_cast<float4*>(kdst) = *reinterpret_cast<const float4*>(&row[4 * c]);
        *reinterpret_cast<float4*>(kdst + 256) =
            *reinterpret_cast<const float4*>(&row[HD / 2 + 4 * c]);
        float* vdst = A.vf + hel + granule_off(HD, false, A.slot, ii, rr * LPR + c, 0);
        *reinterpret_cast<float4*>(vdst) = *reinterpret_cast<const float4*>(&row[HD + 8 * c]);
        *reinterpret_cast<float4*>(vdst + 256) =
            *reinterpret_cast<const float4*>(&row[HD + 8 * c + 4]);
      }
    }
  }
};

// The registers one chunk's loads land in: K (and for a ring its rope
// (cos, sin) and int8 block scales), the dense int8 channel scales of its K
// group, V and the int8 V block scales.
template <int HD, int KIND>
struct ChunkBuf {
  using C = Cfg<HD, 1, KIND>;
  static constexpr int NS = C::NS;
  static constexpr bool kInt8 = C::kInt8, kRing = C::kRing;
  uint2 kq[kInt8 ? NS : 1], vq[kInt8 ? NS : 1];
  float4 kf[kInt8 ? 1 : NS][2], vf[kInt8 ? 1 : NS][2];
  float ksc[KIND == kI8Ring ? NS : 1][2];  // ring int8 K block scales
  float vsc[kInt8 ? NS : 1];               // int8 V block scales
  float4 cs[kRing ? NS : 1][2];            // ring rope cos/sin of the lane's 4 pairs
  // VGPRs the buffer holds
  static constexpr int kVgprs = (kInt8 ? 4 * NS + NS : 16 * NS) +
                                (KIND == kI8Ring ? 2 * NS : 0) + (kRing ? 8 * NS : 0);
};

// CPW: chunks per wave, unrolled (exact load waits); 0: a runtime loop for
// splits longer than the unrolled instances serve
template <int HD, int G, int KIND, bool PROD, int CPW>
__global__ __launch_bounds__(kThreads) void attn_kernel(const AttnParams P, const AppendArgs A) {
  using C = Cfg<HD, G, KIND>;
  constexpr int LPR = C::LPR, RPW = C::RPW, NSG = C::NSG, NGC = C::NGC;
  constexpr int CHUNK = C::CHUNK, GP = C::GP, NB = C::NB;
  constexpr int GW = C::GW, WPG = C::WPG;
  constexpr bool kInt8 = C::kInt8, kRing = C::kRing;

  __shared__ float s_o[kWaves][GW][HD];
  __shared__ float s_ml[kWaves][GW][2];
  __shared__ int s_slice[1];
  __shared__ __align__(16) float s_w[kWaves][CHUNK][GP];
  __shared__ __align__(16) AppStage s_stage[C::NHG];
  // dense int8 fused step: each head group's copy of the group's raw K rows
  // fused step inputs, per head group: the new K and V rows, and (dense
  // int8) the group's raw K rows
  // ([0, 256): K and V rows; raw projections: [256, 512) the (cos, sin)
  // row, [512, 768) the K and V biases)
  __shared__ __align__(16) float s_row[C::NHG][PROD ? 768 : 256];

  const int lane = threadIdx.x & 63;
  // wave index as a provably uniform value: buffer-load SGPR offsets derive
  // from it (a divergent one would turn every load into a waterfall loop)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g0 = (wave / WPG) * GW;  // first query head of this wave's head group
  const int wl = wave % WPG;         // wave index inside the head group
  const int c = lane % LPR;
  const int r = lane / LPR;
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int qrow = blockIdx.z;
  const int nkeys = kRing ? P.ring_nres : P.pos0 + qrow + 1;

  const int nchunks = (nkeys + CHUNK - 1) / CHUNK;
  const int c_end = min((split + 1) * P.chunks_per_split, nchunks);
  const size_t head = static_cast<size_t>(kh) * P.capg;  // first row of this kv head
  const size_t head_el = head * HD;
  const int kx_slot = kslot_xor(HD, c);  // granule slot of this lane's scores
  const int app_chunk = A.slot >= 0 ? A.slot / CHUNK : -1;
  const bool app_here =
      app_chunk >= split * P.chunks_per_split && app_chunk < c_end;  // workgroup-uniform

  // ---- one chunk's loads go into a ChunkBuf; two of them (the chunk being
  // computed and the next one in flight) where the registers allow
  using Buf = ChunkBuf<HD, KIND>;
  constexpr int NBUF = (!kRing && 16 * GW + 2 * Buf::kVgprs <= 208) ? 2 : 1;

  auto rope_pos = [&](int slot) {
    if (slot < P.ring_s) return slot;
    int t = slot - P.ring_s - P.ring_base;
    t += t < 0 ? P.ring_W : 0;
    return P.ring_s + t;
  };

  // Buffer resources of this kv head's arrays: every load is a raw buffer
  // load with a wave-uniform SGPR offset (chunk and slot) and one per-lane
  // VGPR offset, so no 64-bit address registers are held per load.
  constexpr int ES = kInt8 ? 1 : 4;  // bytes per K/V element
  const int kv_bytes = P.capg * HD * ES;
  const rsrc_t rk = make_rsrc(kInt8 ? static_cast<const void*>(P.k8 + head_el)
                                    : static_cast<const void*>(P.kf + head_el), kv_bytes);
  const rsrc_t rv = make_rsrc(kInt8 ? static_cast<const void*>(P.v8 + head_el)
                                    : static_cast<const void*>(P.vf + head_el), kv_bytes);
  // (arrays a layout lacks get an empty resource: every read returns 0)
  const rsrc_t rks =
      KIND == kI8Ring ? make_rsrc(P.ks + head * NB, P.capg * NB * 4)
                        : make_rsrc(P.q, 0);
  const rsrc_t rvs = kInt8 ? make_rsrc(P.vs + head * NB, P.capg * NB * 4) : make_rsrc(P.q, 0);
  const int cs_bytes = P.rope_rows * (HD / 2) * 8;
  const rsrc_t rcs = kRing ? make_rsrc(P.rope, cs_bytes) : make_rsrc(P.q, 0);

  // K (with a ring's rope rows and block scales), the K group's channel
  // scales, then V and its scales, of chunk ch. Every chunk issues the same
  // loads, so the compiler's load waits are exact: a chunk past c_end reads
  // from p0 = capg, past the end of every array (the reads return 0 and
  // fetch nothing). The group a fused step requantizes is read as well and
  // replaced from LDS.
  auto issue = [&](Buf& b, int ch) {
    const bool live = ch < c_end;
    const int p0 = __builtin_amdgcn_readfirstlane(live ? ch * CHUNK : P.capg);
#pragma unroll
    for (int gs = 0; gs < NGC; ++gs)
#pragma unroll
      for (int j = 0; j < NSG; ++j) {
        const int sl = gs * NSG + j;
        const int so = (p0 + gs * kGranule) * HD * ES + j * 512 * ES;
        if constexpr (kInt8) {
          if ((j & 1) == 0) {  // one 16-byte load per lane covers slots j, j + 1
            const uint4 t = __builtin_bit_cast(uint4, stream_b128(rk, lane * 16, so));
            b.kq[sl] = make_uint2(t.x, t.y);
            b.kq[sl + 1] = make_uint2(t.z, t.w);
          }
        } else {
          b.kf[sl][0] = stream_b128(rk, lane * 16, so);
          b.kf[sl][1] = stream_b128(rk, lane * 16, so + 1024);
        }
        if constexpr (kRing) {
          const int p = min(p0 + gs * kGranule + (j ^ kx_slot) * RPW + r, nkeys - 1);
          const int co = live ? rope_pos(p) * (HD / 2) * 8 + 32 * c : cs_bytes;
          b.cs[sl][0] = load_b128(rcs, co, 0);
          b.cs[sl][1] = load_b128(rcs, co + 16, 0);
          if constexpr (KIND == kI8Ring) {
            // the position's block scales in one load: the lane's dims 4c..
            // and hd/2 + 4c.. sit in blocks c / 8 and NB / 2 + c / 8
            const int ko = (live ? p : P.capg) * NB * 4;
            if constexpr (HD == 128) {
              const float4 t = load_b128(rks, ko, 0);
              b.ksc[sl][0] = c >= 8 ? t.y : t.x;
              b.ksc[sl][1] = c >= 8 ? t.w : t.z;
            } else {
              const float2 t = load_b64(rks, ko, 0);
              b.ksc[sl][0] = t.x;
              b.ksc[sl][1] = t.y;
            }
          }
        }
      }
#pragma unroll
    for (int gs = 0; gs < NGC; ++gs)
#pragma unroll
      for (int i = 0; i < NSG; ++i) {
        const int sl = gs * NSG + i;
        const int pb = p0 + gs * kGranule + i * RPW;  // position of row 0
        const int so = (p0 + gs * kGranule) * HD * ES + i * 512 * ES;
        if constexpr (kInt8) {
          if ((i & 1) == 0) {
            const uint4 t = __builtin_bit_cast(uint4, stream_b128(rv, lane * 16, so));
            b.vq[sl] = make_uint2(t.x, t.y);
            b.vq[sl + 1] = make_uint2(t.z, t.w);
          }
          b.vsc[sl] = load_b32(rvs, (r * NB + (8 * c) / kBlock) * 4, pb * NB * 4);
        } else {
          b.vf[sl][0] = stream_b128(rv, lane * 16, so);
          b.vf[sl][1] = stream_b128(rv, lane * 16, so + 1024);
        }
      }
  };

  // ---- q of this lane's K dims (4c..4c+3, hd/2+4c..), in the log2 domain;
  // the ring ropes it at n_res - 1 (model.cpp:669-671). Its loads go out
  // before the first chunk's: vector loads return in order, so q issued last
  // would hold QK back until the whole chunk (V included) had arrived.
  float4 qa[GW], qc[GW], cq[2];
  // Raw projections (PROD, decode): the q bias of the lane's dims and the
  // (cos, sin) of its 4 pairs load with q and are applied with the scaling
  // below (bias, then the fp64 rope of every head the lane holds)
  float4 qba[GW], qbc[GW];
  double2 qt[4];
  const bool q_bias = PROD && P.qb != nullptr, q_rope = PROD && !kRing && P.qcs != nullptr;
  if (q_bias) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const float* bg = P.qb + (kh * G + min(g0 + g, G - 1)) * HD;
      qba[g] = *reinterpret_cast<const float4*>(bg + 4 * c);
      qbc[g] = *reinterpret_cast<const float4*>(bg + HD / 2 + 4 * c);
    }
  }
  if (q_rope) {
#pragma unroll
    for (int t = 0; t < 4; ++t) qt[t] = P.qcs[4 * c + t];
  }
  {
    const float* qb = P.q + (static_cast<size_t>(qrow) * P.n_heads + kh * G) * HD;
    if constexpr (kRing) {
      const float4* t = reinterpret_cast<const float4*>(
          P.rope + static_cast<size_t>(P.ring_nres - 1) * (HD / 2) + 4 * c);
      cq[0] = t[0];
      cq[1] = t[1];
    }
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const float* qg = qb + min(g0 + g, G - 1) * HD;
      qa[g] = *reinterpret_cast<const float4*>(qg + 4 * c);
      qc[g] = *reinterpret_cast<const float4*>(qg + HD / 2 + 4 * c);
    }
  }
  // fused decode step (FusedAppend): the owner wave of each head group
  // stages the new row and takes its values from the stage for that chunk,
  // so no global read-after-write happens inside the kernel. The row's
  // inputs load ahead of the owner's first chunk when that chunk is the new
  // row's, else right behind it (vector loads return in order, so they then
  // hold back nothing before that chunk), and are staged on reaching the
  // chunk.
  AppStage& s_app = s_stage[wave / WPG];
  const int app_rel = app_chunk - split * P.chunks_per_split;
  const bool app_owner = app_here && wl == app_rel % WPG;  // wave-uniform
  using App = FusedAppend<HD, KIND, PROD>;
  float* app_row = s_row[wave / WPG];
  // (loaded ahead of the chunks, the oldest loads in flight: a register
  // reused later never waits on them longer than on the chunk loads)
  typename App::RowIn app_in{};
  if (app_owner) App::load_row(A, kh, lane, app_in);
  __builtin_amdgcn_sched_barrier(0);
  const int ch0 = split * P.chunks_per_split + wl;  // chunk t of this wave: ch0 + t * WPG
  Buf RA, RB;
  issue(RA, ch0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NBUF == 2 && CPW != 1) issue(RB, ch0 + WPG);
  __builtin_amdgcn_sched_barrier(0);
  float qv[GW][8];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    // a head group's padding head (odd G) gets q = 0 and is never stored
    const bool hv = g0 + g < G;
    float x[8] = {qa[g].x, qa[g].y, qa[g].z, qa[g].w, qc[g].x, qc[g].y, qc[g].z, qc[g].w};
    if (q_bias) {
      const float b[8] = {qba[g].x, qba[g].y, qba[g].z, qba[g].w,
                          qbc[g].x, qbc[g].y, qbc[g].z, qbc[g].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] += b[e];
    }
    if (q_rope) {
#pragma unroll
      for (int t = 0; t < 4; ++t) rope_pair(x[t], x[4 + t], qt[t]);
    }
    if constexpr (kRing) {
      const float cv[4] = {cq[0].x, cq[0].z, cq[1].x, cq[1].z};
      const float sv[4] = {cq[0].y, cq[0].w, cq[1].y, cq[1].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float u = x[t], w = x[4 + t];
        // explicit fused forms: every instance rounds the same way
        x[t] = fmaf(u, cv[t], -(w * sv[t]));
        x[4 + t] = fmaf(w, cv[t], u * sv[t]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[g][e] = hv ? x[e] * P.qscale : 0.0f;
  }

  float M[GW], l[GW], o[GW][8];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    M[g] = kMinit;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  auto compute = [&](Buf& b, const int ch) {
    const int p0 = ch * CHUNK;

    // ---- the appended row (fused step): take its new values from the stage
    const bool app_now = ch == app_chunk;  // uniform
    const int app_pc = A.slot - p0;        // its position inside the chunk
    const int app_r = (app_pc & 15) % RPW, app_i = (app_pc & 15) / RPW, app_gs = app_pc >> 4;
    if (app_now) {
      App::put_row(A, app_in, lane, app_row);
      if (PROD && A.prod) App::produce_row(A, lane, app_row);
      App::stage_row(A, lane, s_app, app_row);
      {
        const bool mine = r == app_r;
#pragma unroll
        for (int gs = 0; gs < NGC; ++gs)
#pragma unroll
          for (int j = 0; j < NSG; ++j) {
            const int sl = gs * NSG + j;
            if (mine && gs == app_gs && (j ^ kx_slot) == app_i) {
              if constexpr (kInt8) {
                b.kq[sl] = make_uint2(s_app.k8row[c], s_app.k8row[HD / 8 + c]);
                b.ksc[sl][0] = s_app.ks[(4 * c) / kBlock];
                b.ksc[sl][1] = s_app.ks[(HD / 2 + 4 * c) / kBlock];
              } else {
                b.kf[sl][0] = *reinterpret_cast<const float4*>(&s_app.krow[4 * c]);
                b.kf[sl][1] = *reinterpret_cast<const float4*>(&s_app.krow[HD / 2 + 4 * c]);
              }
            }
          }
      }
    }

    // ---- q for this chunk
    float qt[GW][8];
#pragma unroll
    for (int g = 0; g < GW; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) qt[g][e] = qv[g][e];

    // ---- QK: per granule, NSG slot partials -> one score per lane
    float sc[NGC][GW];
#pragma unroll
    for (int gs = 0; gs < NGC; ++gs) {
      float acc[GW][NSG];
#pragma unroll
      for (int j = 0; j < NSG; ++j) {
        const int sl = gs * NSG + j;
        float kx[8];
        if constexpr (kInt8) {
          cvt8(b.kq[sl], kx);
          if constexpr (KIND == kI8Ring) {
            // dequantize (code * block scale, model.cpp:689-690)
#pragma unroll
            for (int e = 0; e < 8; ++e) kx[e] = b.ksc[sl][e >> 2] * kx[e];
          }
        } else {
          kx[0] = b.kf[sl][0].x; kx[1] = b.kf[sl][0].y; kx[2] = b.kf[sl][0].z; kx[3] = b.kf[sl][0].w;
          kx[4] = b.kf[sl][1].x; kx[5] = b.kf[sl][1].y; kx[6] = b.kf[sl][1].z; kx[7] = b.kf[sl][1].w;
        }
        if constexpr (kRing) {
          const float cv[4] = {b.cs[sl][0].x, b.cs[sl][0].z, b.cs[sl][1].x, b.cs[sl][1].z};
          const float sv[4] = {b.cs[sl][0].y, b.cs[sl][0].w, b.cs[sl][1].y, b.cs[sl][1].w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float a = kx[t], b = kx[4 + t];
            kx[t] = fmaf(a, cv[t], -(b * sv[t]));
            kx[4 + t] = fmaf(b, cv[t], a * sv[t]);
          }
        }
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          float a = qt[g][0] * kx[0];
#pragma unroll
          for (int e = 1; e < 8; ++e) a += qt[g][e] * kx[e];
          acc[g][j] = a;
        }
      }
      const int p = p0 + gs * kGranule + kx_slot * RPW + r;
      const bool valid = p < nkeys;
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const float s = treduce<HD>(acc[g]);
        sc[gs][g] = valid ? s : -INFINITY;
      }
    }

    // ---- online softmax with a wave-uniform running max
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      float mx = sc[0][g];
#pragma unroll
      for (int gs = 1; gs < NGC; ++gs) mx = fmaxf(mx, sc[gs][g]);
      const float mn = fmaxf(M[g], wave_max(mx));
      const float alpha = fast_exp2(M[g] - mn);
      M[g] = mn;
      float ls = l[g] * alpha;
#pragma unroll
      for (int gs = 0; gs < NGC; ++gs) {
        const float w = fast_exp2(sc[gs][g] - mn);
        sc[gs][g] = w;
        ls += w;
      }
      l[g] = ls;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
    }

    // ---- weights to the PV mapping through this wave's LDS rows
    if ((c & 3) == 0) {
#pragma unroll
      for (int gs = 0; gs < NGC; ++gs) {
        float* wr = &s_w[wave][gs * kGranule + kx_slot * RPW + r][0];
#pragma unroll
        for (int gq = 0; gq < GP; gq += 4) {
          float4 w4;
          w4.x = gq + 0 < GW ? sc[gs][gq + 0 < GW ? gq + 0 : 0] : 0.0f;
          w4.y = gq + 1 < GW ? sc[gs][gq + 1 < GW ? gq + 1 : 0] : 0.0f;
          w4.z = gq + 2 < GW ? sc[gs][gq + 2 < GW ? gq + 2 : 0] : 0.0f;
          w4.w = gq + 3 < GW ? sc[gs][gq + 3 < GW ? gq + 3 : 0] : 0.0f;
          *reinterpret_cast<float4*>(wr + gq) = w4;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    if (app_now && r == app_r) {
#pragma unroll
      for (int gs = 0; gs < NGC; ++gs)
#pragma unroll
        for (int i = 0; i < NSG; ++i) {
          const int sl = gs * NSG + i;
          if (gs == app_gs && i == app_i) {
            if constexpr (kInt8) {
              b.vq[sl] = make_uint2(s_app.v8row[2 * c], s_app.v8row[2 * c + 1]);
              b.vsc[sl] = s_app.vs[(8 * c) / kBlock];
            } else {
              b.vf[sl][0] = *reinterpret_cast<const float4*>(&s_app.vrow[8 * c]);
              b.vf[sl][1] = *reinterpret_cast<const float4*>(&s_app.vrow[8 * c + 4]);
            }
          }
        }
    }

    // ---- PV: lane (row r, dims 8c..8c+7), slot i -> position i*RPW + r.
    // Rows past the last key have weight 0; in the final partial chunk their
    // (stale) V and scales are zeroed as well, so nothing non-finite enters.
    const bool full = p0 + CHUNK <= nkeys;  // uniform
#pragma unroll
    for (int gs = 0; gs < NGC; ++gs)
#pragma unroll
      for (int i = 0; i < NSG; ++i) {
        const int sl = gs * NSG + i;
        const float* wr = &s_w[wave][gs * kGranule + i * RPW + r][0];
        float wv[GP];
#pragma unroll
        for (int gq = 0; gq < GP; gq += 4) {
          const float4 w4 = *reinterpret_cast<const float4*>(wr + gq);
          wv[gq] = w4.x;
          wv[gq + 1] = w4.y;
          wv[gq + 2] = w4.z;
          wv[gq + 3] = w4.w;
        }
        float vx[8];
        float vsl = 0.0f;
        if constexpr (kInt8) {
          cvt8(b.vq[sl], vx);
          vsl = b.vsc[sl];
        } else {
          vx[0] = b.vf[sl][0].x; vx[1] = b.vf[sl][0].y; vx[2] = b.vf[sl][0].z; vx[3] = b.vf[sl][0].w;
          vx[4] = b.vf[sl][1].x; vx[5] = b.vf[sl][1].y; vx[6] = b.vf[sl][1].z; vx[7] = b.vf[sl][1].w;
        }
        if (!full) {
          const bool ok = p0 + gs * kGranule + i * RPW + r < nkeys;
#pragma unroll
          for (int e = 0; e < 8; ++e) vx[e] = ok ? vx[e] : 0.0f;
          vsl = ok ? vsl : 0.0f;
        }
        if constexpr (kInt8) {
#pragma unroll
          for (int g = 0; g < GW; ++g) wv[g] *= vsl;
        }
#pragma unroll
        for (int g = 0; g < GW; ++g)
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] += wv[g] * vx[e];
      }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- the chunks of this wave, in a software pipeline: chunk t + NBUF is
  // issued into the buffer chunk t used as soon as chunk t is consumed
  if constexpr (CPW > 0) {
#pragma unroll
    for (int t = 0; t < CPW; ++t) {
      Buf& X = (NBUF == 2 && (t & 1)) ? RB : RA;
      const int cht = ch0 + t * WPG;
      if (cht < c_end) compute(X, cht);
      __builtin_amdgcn_sched_barrier(0);
      if (t + NBUF < CPW) issue(X, ch0 + (t + NBUF) * WPG);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    int ch = ch0;
    while (ch < c_end) {
      compute(RA, ch);
      __builtin_amdgcn_sched_barrier(0);
      issue(RA, ch + NBUF * WPG);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NBUF == 2) {
        if (ch + WPG >= c_end) break;
        compute(RB, ch + WPG);
        __builtin_amdgcn_sched_barrier(0);
        issue(RB, ch + 3 * WPG);
        __builtin_amdgcn_sched_barrier(0);
      }
      ch += NBUF * WPG;
    }
  }


  // ---- wave epilogue: l over lanes, o over the RPW lane rows (transposing
  // permlane swaps: lane ends with values K = k + 2GW * (lane / 16), k < 2GW)
#pragma unroll
  for (int g = 0; g < GW; ++g) l[g] = wave_sum(l[g]) * (1.0f / C::DUP);
  float v1[4 * GW], v2[2 * GW];
#pragma unroll
  for (int k = 0; k < 4 * GW; ++k)
    v1[k] = swap32_sum(o[k / 8][k % 8], o[(k + 4 * GW) / 8][(k + 4 * GW) % 8]);
#pragma unroll
  for (int k = 0; k < 2 * GW; ++k) v2[k] = swap16_sum(v1[k], v1[k + 2 * GW]);
  if constexpr (HD == 64) {
#pragma unroll
    for (int k = 0; k < 2 * GW; ++k) v2[k] += dpp<kX8>(v2[k]);
  }
  if (HD == 128 || (lane & 8) == 0) {
    const int q4 = lane >> 4;
#pragma unroll
    for (int k = 0; k < 2 * GW; ++k) {
      const int K = k + 2 * GW * q4;
      s_o[wave][K / 8][8 * c + K % 8] = v2[k];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      s_ml[wave][g][0] = M[g];
      s_ml[wave][g][1] = l[g];
    }
  }
  finish<HD, G, GW, WPG>(P, s_o, s_ml, split, kh, qrow);
  if (!P.direct) {
    // this thread's record stores have reached the coherence point
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    arrive_and_merge<HD, G, 1>(P, kh, qrow, 1, wave, lane, s_slice);
  }
  if (app_owner && g0 == 0) App::flush(A, kh, lane, s_app, nullptr, app_row);
}

}  // namespace
}  // namespace dbi

// ---------------------------------------------------------------------------
// instance selection (used by the attn_inst_*.hip translation units)
namespace dbi {
namespace {

// CPW: chunks per wave of the plan (1, 2, 4 unrolled; 0 a runtime loop).
template <int HD, int G, int KIND, bool PROD>
void* kernel_cpw(int cpw) {
  switch (cpw) {
    case 1: return reinterpret_cast<void*>(&attn_kernel<HD, G, KIND, PROD, 1>);
    case 2: return reinterpret_cast<void*>(&attn_kernel<HD, G, KIND, PROD, 2>);
    case 4: return reinterpret_cast<void*>(&attn_kernel<HD, G, KIND, PROD, 4>);
    default: return reinterpret_cast<void*>(&attn_kernel<HD, G, KIND, PROD, 0>);
  }
}

template <int HD, int KIND, bool PROD>
void* pick_g(int G, int cpw) {
  switch (G) {
    case 1: return kernel_cpw<HD, 1, KIND, PROD>(cpw);
    case 2: return kernel_cpw<HD, 2, KIND, PROD>(cpw);
    case 3: return kernel_cpw<HD, 3, KIND, PROD>(cpw);
    case 4: return kernel_cpw<HD, 4, KIND, PROD>(cpw);
    case 5: return kernel_cpw<HD, 5, KIND, PROD>(cpw);
    case 6: return kernel_cpw<HD, 6, KIND, PROD>(cpw);
    case 7: return kernel_cpw<HD, 7, KIND, PROD>(cpw);
    case 8: return kernel_cpw<HD, 8, KIND, PROD>(cpw);
    default: return nullptr;
  }
}

}  // namespace

// one per layout and producer flag, each in its own translation unit
void* attn_instance_0_0(int hd, int G, int cpw);
void* attn_instance_0_1(int hd, int G, int cpw);
// dense int8 (matrix-core kernel, one query row per workgroup)
void* attn_instance_1_0(int hd, int G, int cpw);
void* attn_instance_1_1(int hd, int G, int cpw);
// dense int8 chunk rows (matrix-core kernel): nvt 16-vector tiles per workgroup
void* attn_instance_i8_rows(int hd, int G, int nvt);
// dense fp32 chunk rows (matrix-core kernel): nvt 16-vector tiles per workgroup
void* attn_instance_f32_rows(int hd, int G, int nvt);
void* attn_instance_f32_rows_merge(int hd, int G);
void* attn_instance_2_0(int hd, int G, int cpw);
void* attn_instance_2_1(int hd, int G, int cpw);
void* attn_instance_3_0(int hd, int G, int cpw);
void* attn_instance_3_1(int hd, int G, int cpw);

}  // namespace dbi
