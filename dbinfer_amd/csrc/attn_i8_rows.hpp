// Dense int8 GQA attention of a few query rows at once on the matrix cores
// (attend_dense_int8's arithmetic, model.cpp:600-661, for the causal chunk
// rows of decode_layer_chunk, model.cpp:956-981: a speculative verify
// round's k + 1 rows, speculative.cpp:64). Instantiated by
// attn_inst_i8_rows.hip.
//
// Design (CDNA4, wave64, v_mfma_f32_16x16x32_bf16, exact bf16 products as
// attn_mfma.hpp: codes are exact in bf16, fp32 factors are split into three
// bf16 parts):
//  - Grid (split, kv head, row group), 8 waves per workgroup, 32-position
//    chunks (one K group each), chunk t -> wave t % 8. A workgroup serves
//    NQ = 16 * NVT query vectors (row r, head g: r * G + g) of up to
//    NR = NQ / G rows, so a C5 verify round (5 rows x 4 heads) streams the
//    cache once.
//  - Matrix columns are query vectors (the decode kernel's columns are
//    (query, V block) pairs, which fill a tile with its few queries but
//    repeat each one per block): QK^T has A = the chunk's K codes (rows:
//    positions), B = q~ = (q * scale * log2 e) * ks in three parts, built by
//    each lane for exactly its own operand (query lane % 16, channels
//    32 j + 8 (lane / 16) + e) from the scaled q in LDS.
//  - Softmax on the scores as they leave the matrix core (lane n + 16 g holds
//    query n at positions 16 h + 4 g + i, a column's max and sum are lane-
//    local plus two permlane swaps); those 8 positions are exactly the lane's
//    PV A operand, so the weight of each V block b, w_b = p * vs[pos][b], is
//    built in place (three parts) and multiplies the V codes of the two
//    16-channel tiles of block b.
//  - PV output: lane (channel n, group g) holds queries 4 g .. 4 g + 3; their
//    rescale factors come from the QK lanes of those columns (ds_bpermute).
//  - Remainder tile (REM): a group of 16 + r vectors, r <= 16 / (hd / 32),
//    runs one 16-column tile and one of (query, channel block) columns:
//    column (q, c) splits q~ of block c only and enters QK^T in k-step c
//    alone, so it sums block c's partial score; the partials of a query
//    (neighbouring lanes) add up by DPP. PV runs transposed there, O^T = V^T
//    W^T: the V codes as loaded are the A operand and the column's weights
//    of block c the B operand, so column (q, c) keeps the output tiles of
//    block c. Its rescale is lane-local. A 16-column tile would split and
//    exponentiate all 16 columns for r of them.
//  - The fp32 sinks (positions < n_sink, model.cpp:612-626) are masked in
//    the stream and attended by the rows merge launch (attn_rows.hpp), which
//    merges the split records; with sinks there is always a merge launch.
#pragma once

#include "attn_rows.hpp"

namespace dbi {
namespace {

template <int HD, int G, int NVT, bool REM = false>
struct I8RCfg {
  static constexpr int NQ = 16 * NVT;       // query vectors per workgroup (padded)
  static constexpr int NJ = HD / 32;        // QK k-steps (32 channels) = V blocks
  static constexpr int QR = 16 / NJ;        // REM: vectors of the remainder tile
  static constexpr int NR = REM ? (16 + QR) / G : NQ / G;  // rows per workgroup
  static constexpr int NBK = HD / kBlock;   // V blocks per head
  static constexpr int KL = HD / 64;        // K loads per granule (two k-steps each)
  static constexpr int NTV = HD / 16;       // PV channel tiles
  static constexpr int VL = HD / 32;        // V loads per chunk (two tiles each)
  static constexpr int OP = HD + 4;         // LDS row pitch of a wave's outputs
  static_assert(HD == 64 || HD == 128, "head dim");
  static_assert(G >= 1 && G <= NQ, "query heads per kv head");
  static_assert(NBK == NJ && (!REM || NVT == 2), "remainder tile: one column per (query, block)");
};

template <int HD, int G, int NVT, bool REM>
__global__ __launch_bounds__(kThreads) void attn_i8_rows_kernel(const AttnParams P) {
  using C = I8RCfg<HD, G, NVT, REM>;
  constexpr int NQ = C::NQ, NR = C::NR, NBK = C::NBK, NJ = C::NJ, KL = C::KL;
  constexpr int NTV = C::NTV, VL = C::VL, OP = C::OP, QR = C::QR;
  constexpr int CHUNK = kKGroup;
  constexpr int NT = REM ? 1 : NVT;  // tiles of 16 query columns
  // remainder tile (REM): lane column col = NJ rq + rc serves query 16 + rq
  // and channel block rc (QK k-step rc, V block rc)

  // q * scale * log2 e (0 past the queries); rows padded by 16 bytes: a q~
  // read takes one 16-byte piece of 16 consecutive rows, which a 512-byte
  // pitch would put in the same banks
  __shared__ __align__(16) float s_q[NQ][HD + 4];
  __shared__ __align__(16) float s_o[kWaves][16][OP];
  __shared__ float s_ml[kWaves][16][2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, grp = lane >> 4;  // matrix column / row group of this lane
  const int rq = col / NJ, rc = col % NJ;      // REM: query and channel block of the column
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int row0 = blockIdx.z * NR;            // this workgroup's rows [row0, row0 + nr)
  const int nr = min(NR, P.rows - row0);
  const int nqv = nr * G;                      // its query vectors
  const int nkeys = P.pos0 + row0 + nr;        // keys of its last row
  const int nchunks = (nkeys + CHUNK - 1) / CHUNK;
  const int c_end = min((split + 1) * P.chunks_per_split, nchunks);
  const size_t head = static_cast<size_t>(kh) * P.capg;
  const int kv_bytes = P.capg * HD;
  const rsrc_t rk = make_rsrc(P.k8 + head * HD, kv_bytes);
  const rsrc_t rv = make_rsrc(P.v8 + head * HD, kv_bytes);
  const int ks_bytes = P.ng * HD * 4;
  const rsrc_t rks = make_rsrc(P.ks + static_cast<size_t>(kh) * P.ng * HD, ks_bytes);
  const int vs_bytes = P.capg * NBK * 4;
  const rsrc_t rvs = make_rsrc(P.vs + head * NBK, vs_bytes);

  // ---- the workgroup's queries, scaled, into LDS
  for (int idx = threadIdx.x; idx < NQ * HD / 4; idx += kThreads) {
    const int q = idx / (HD / 4), d4 = idx % (HD / 4);
    float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (q < nqv) {
      x = *reinterpret_cast<const float4*>(
          P.q + (static_cast<size_t>(row0 + q / G) * P.n_heads + kh * G + q % G) * HD + 4 * d4);
      x.x *= P.qscale;
      x.y *= P.qscale;
      x.z *= P.qscale;
      x.w *= P.qscale;
    }
    *reinterpret_cast<float4*>(&s_q[q][4 * d4]) = x;
  }

  // ---- one chunk's loads (K codes and the lane's K channel scales; V codes
  // and the V block scales of the lane's 8 positions). A chunk past c_end
  // reads at offsets past num_records: the reads return 0 and fetch nothing.
  // So do the V scales of sink positions and of positions past the group's
  // last key: their weights are then exactly 0 (the masked scores give p = 0,
  // and a stale scale there may be anything).
  uint4 kc[2][KL], vc[VL];
  float4 ksc[NJ][2];
  float vsc[8][NBK];
  float4 ksr[2];  // REM: the K channel scales of block rc (channels 32 rc + 8 grp + e)
  float vsr[8];   // REM: the V scale of block rc at the lane's 8 positions
  auto issue_k = [&](int ch) {
    const bool live = ch < c_end;
    const int base = live ? ch * CHUNK * HD : kv_bytes;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int jp = 0; jp < KL; ++jp)
        kc[h][jp] = __builtin_bit_cast(uint4, stream_b128(rk, base + lane * 16 + (h * KL + jp) * 1024, 0));
    const int sb = live ? ch * HD * 4 : ks_bytes;  // the chunk's K group row of scales
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      ksc[j][0] = load_b128(rks, sb + (32 * j + 8 * grp) * 4, 0);
      ksc[j][1] = load_b128(rks, sb + (32 * j + 8 * grp + 4) * 4, 0);
    }
    if constexpr (REM) {
      ksr[0] = load_b128(rks, sb + (32 * rc + 8 * grp) * 4, 0);
      ksr[1] = load_b128(rks, sb + (32 * rc + 8 * grp + 4) * 4, 0);
    }
  };
  auto issue_v = [&](int ch) {
    const bool live = ch < c_end;
    const int base = live ? ch * CHUNK * HD : kv_bytes;
#pragma unroll
    for (int tp = 0; tp < VL; ++tp)
      vc[tp] = __builtin_bit_cast(uint4, stream_b128(rv, base + lane * 16 + tp * 1024, 0));
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int p = ch * CHUNK + 16 * (s / 4) + 4 * grp + s % 4;
      const int vo = live && p >= P.n_sink && p < nkeys ? p * NBK * 4 : vs_bytes;
      if constexpr (NBK == 4) {
        const float4 t = load_b128(rvs, vo, 0);
        vsc[s][0] = t.x;
        vsc[s][1] = t.y;
        vsc[s][2] = t.z;
        vsc[s][3] = t.w;
      } else {
        const float2 t = load_b64(rvs, vo, 0);
        vsc[s][0] = t.x;
        vsc[s][1] = t.y;
      }
      // (vo = vs_bytes for a masked position: the read lands past num_records, 0)
      if constexpr (REM) vsr[s] = load_b32(rvs, vo + rc * 4, 0);
    }
  };

  const int ch0 = split * P.chunks_per_split + wave;  // chunk t of this wave: ch0 + 8 t
  issue_k(ch0);
  issue_v(ch0);
  __syncthreads();  // s_q

  float M[NT], l[NT];
  f32x4 o[NT][NTV];
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    M[T] = kMinit;
    l[T] = 0.0f;
#pragma unroll
    for (int t = 0; t < NTV; ++t) o[T][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // REM: the remainder tile's state; its output lane (column (rq, rc), row
  // group grp) holds O^T[channel 16 t + 4 grp + i][column], kept where rc is
  // the block of tile t
  float MR = kMinit, lR = 0.0f;
  f32x4 oR[REM ? NTV : 1];
#pragma unroll
  for (int t = 0; t < (REM ? NTV : 1); ++t) oR[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int ch = ch0; ch < c_end; ch += kWaves) {
    // products feeding split3 are rounded to fp32 first (q * ks, as the
    // reference rounds it; p * vs): no contraction into the split's subtraction
#pragma clang fp contract(off)
    const int p0 = ch * CHUNK;
    // ---- QK^T: scores of query T * 16 + col at positions 16 h + 4 grp + i
    f32x4 sc[2][NT], scr[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int T = 0; T < NT; ++T) sc[h][T] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      scr[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // REM: the column's q~ of block rc only (it enters k-step rc alone, so
    // the column sums the partial score of its block)
    uint4 ptr[3];
    if constexpr (REM) {
      const float4 qa = *reinterpret_cast<const float4*>(&s_q[16 + rq][32 * rc + 8 * grp]);
      const float4 qb = *reinterpret_cast<const float4*>(&s_q[16 + rq][32 * rc + 8 * grp + 4]);
      const float x[8] = {qa.x * ksr[0].x, qa.y * ksr[0].y, qa.z * ksr[0].z, qa.w * ksr[0].w,
                          qb.x * ksr[1].x, qb.y * ksr[1].y, qb.z * ksr[1].z, qb.w * ksr[1].w};
      split3(x, ptr);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      bf16x8 ak[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 w = kc[h][j / 2];
        ak[h] = (j & 1) ? codes_bf16(w.z, w.w) : codes_bf16(w.x, w.y);
      }
      const float ks8[8] = {ksc[j][0].x, ksc[j][0].y, ksc[j][0].z, ksc[j][0].w,
                            ksc[j][1].x, ksc[j][1].y, ksc[j][1].z, ksc[j][1].w};
#pragma unroll
      for (int T = 0; T < NT; ++T) {
        const float4 qa = *reinterpret_cast<const float4*>(&s_q[T * 16 + col][32 * j + 8 * grp]);
        const float4 qb = *reinterpret_cast<const float4*>(&s_q[T * 16 + col][32 * j + 8 * grp + 4]);
        const float q8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = q8[e] * ks8[e];
        uint4 pt[3];
        split3(x, pt);
#pragma unroll
        for (int a = 0; a < 3; ++a)
#pragma unroll
          for (int h = 0; h < 2; ++h) sc[h][T] = mfma(ak[h], pt[a], sc[h][T]);
      }
      if constexpr (REM) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int a = 0; a < 3; ++a) {
          const uint4 b = rc == j ? ptr[a] : z;
#pragma unroll
          for (int h = 0; h < 2; ++h) scr[h] = mfma(ak[h], b, scr[h]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_k(ch + kWaves);
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax per column, then the block weights (PV A operands)
    float pk[NT][8];
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      // keys of this column's row (causal: row r attends [0, pos0 + r]); the
      // sinks (positions < n_sink) are attended from their fp32 copies
      const int nk = P.pos0 + row0 + min(T * 16 + col, nqv - 1) / G + 1;
      float s[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int p = p0 + 16 * (k / 4) + 4 * grp + k % 4;
        const bool valid = p < nk && p >= P.n_sink;
        s[k] = valid ? sc[k / 4][T][k % 4] : -INFINITY;
      }
      float mx = s[0];
#pragma unroll
      for (int k = 1; k < 8; ++k) mx = fmaxf(mx, s[k]);
      const float mn = lazy_max(M[T], col_max(mx));
      const float alpha = fast_exp2(M[T] - mn);
      M[T] = mn;
      float ls = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        pk[T][k] = fast_exp2(s[k] - mn);
        ls += pk[T][k];
      }
      l[T] = fmaf(l[T], alpha, ls);
      // rescale of the output rows (queries 4 grp + i of this tile): the
      // factor of column 4 grp + i, from that column's lane; skipped while
      // every reference maximum holds
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ar = __builtin_bit_cast(
              float, __builtin_amdgcn_ds_bpermute(4 * (4 * grp + i), __builtin_bit_cast(int, alpha)));
#pragma unroll
          for (int t = 0; t < NTV; ++t) o[T][t][i] *= ar;
        }
      }
    }
    // REM: the NJ block partials of a query sit in NJ neighbouring lanes (a
    // DPP quad); their sum is the score, equal in all of them
    float pkr[8];
    if constexpr (REM) {
      const int nk = P.pos0 + row0 + min(16 + rq, nqv - 1) / G + 1;
      float s[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float x = scr[k / 4][k % 4];
        x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
        if constexpr (NJ == 4)
          x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
        const int p = p0 + 16 * (k / 4) + 4 * grp + k % 4;
        s[k] = p < nk && p >= P.n_sink ? x : -INFINITY;
      }
      float mx = s[0];
#pragma unroll
      for (int k = 1; k < 8; ++k) mx = fmaxf(mx, s[k]);
      const float mn = lazy_max(MR, col_max(mx));
      const float alpha = fast_exp2(MR - mn);
      MR = mn;
      float ls = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        pkr[k] = fast_exp2(s[k] - mn);
        ls += pkr[k];
      }
      lR = fmaf(lR, alpha, ls);
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int t = 0; t < NTV; ++t) oR[t] *= alpha;  // (the lane's own column)
      }
    }
    // ---- PV per V block: w_b = p * vs[pos][b] (masked slots: p = 0, and
    // outside the group's keys vs = 0), three parts, against the V codes of
    // the block's two channel tiles; each tile's codes are converted once
    // and serve every vector tile
    // REM: B = W^T of the column (the weights of block rc at the lane's 8
    // positions), against A = V^T: the tile's codes as loaded
    uint4 pbr[3];
    if constexpr (REM) {
      float w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = pkr[k] * vsr[k];
      split3(w, pbr);
    }
#pragma unroll
    for (int b = 0; b < NBK; ++b) {
      uint4 aw[NT][3];
#pragma unroll
      for (int T = 0; T < NT; ++T) {
        float w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) w[k] = pk[T][k] * vsc[k][b];
        split3(w, aw[T]);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * b + tt;
        const uint4 vw = vc[t / 2];
        const bf16x8 bv = (t & 1) ? codes_bf16(vw.z, vw.w) : codes_bf16(vw.x, vw.y);
#pragma unroll
        for (int T = 0; T < NT; ++T)
#pragma unroll
          for (int a = 0; a < 3; ++a) o[T][t] = mfma(aw[T][a], bv, o[T][t]);
        if constexpr (REM) {
#pragma unroll
          for (int a = 0; a < 3; ++a) oR[t] = mfma(bv, pbr[a], oR[t]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_v(ch + kWaves);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- per query tile: wave states to LDS, then the cross-wave combine of
  // the tile (local query ql = query q0 + ql) and the output (single split,
  // no sinks) or the records
  auto emit = [&](int q0, int nq) {
    auto combine = [&](int ql, float& Mx, float (&f)[kWaves], float& L) {
      float m[kWaves], lw[kWaves];
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        m[i] = s_ml[i][ql][0];
        lw[i] = s_ml[i][ql][1];
      }
      Mx = kMinit;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) Mx = fmaxf(Mx, m[i]);
      L = 0.0f;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        f[i] = fast_exp2(m[i] - Mx);
        L += lw[i] * f[i];
      }
    };
    // one thread per (query, 4 dims): the combine once per thread, float4
    // reads of the wave states and float4 stores (the records are read by
    // the merge launch, after this kernel)
    constexpr int D4 = HD / 4;
    const size_t row_stride = static_cast<size_t>(P.nkv) * record_region(P.nsplit, G, HD);
    float* const rbase = P.part + (static_cast<size_t>(row0) * P.nkv + kh) * record_region(P.nsplit, G, HD) +
                         static_cast<size_t>(split) * record_floats(G, HD);
    for (int idx = threadIdx.x; idx < nq * D4; idx += kThreads) {
      const int ql = idx / D4, d4 = idx % D4, q = q0 + ql, r = q / G, g = q % G;
      float Mx, f[kWaves], L;
      combine(ql, Mx, f, L);
      float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        const float4 x = *reinterpret_cast<const float4*>(&s_o[i][ql][4 * d4]);
        O.x += x.x * f[i];
        O.y += x.y * f[i];
        O.z += x.z * f[i];
        O.w += x.w * f[i];
      }
      if (P.direct) {
        *reinterpret_cast<float4*>(
            P.out + (static_cast<size_t>(row0 + r) * P.n_heads + kh * G + g) * HD + 4 * d4) =
            make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
      } else {
        float* orec = rbase + static_cast<size_t>(r) * row_stride;
        *reinterpret_cast<float4*>(orec + g * HD + 4 * d4) = O;
        if (d4 == 0) *reinterpret_cast<float2*>(orec + G * HD + 2 * g) = make_float2(Mx, L);
      }
    }
  };
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    const float lt = col_sum(l[T]);
    if (grp == 0) {
      s_ml[wave][col][0] = M[T];
      s_ml[wave][col][1] = lt;
    }
    // lane holds query 4 grp + i at channel 16 t + col
#pragma unroll
    for (int t = 0; t < NTV; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_o[wave][4 * grp + i][16 * t + col] = o[T][t][i];
    __syncthreads();
    emit(T * 16, min(16, nqv - T * 16));
    __syncthreads();  // s_o / s_ml are rewritten by the next query tile
  }
  if constexpr (REM) {
    // the remainder tile: column (rq, rc) keeps output tile t where rc is
    // the block of t (channels 16 t + 4 grp + i)
    const float lt = col_sum(lR);
    if (grp == 0 && rc == 0) {
      s_ml[wave][rq][0] = MR;
      s_ml[wave][rq][1] = lt;
    }
#pragma unroll
    for (int t = 0; t < NTV; ++t)
      if (rc == t / 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_o[wave][rq][16 * t + 4 * grp + i] = oR[t][i];
      }
    __syncthreads();
    emit(16, min(QR, nqv - 16));
  }
}

template <int HD, int NVT, bool REM = false>
void* pick_i8_rows_g(int G) {
  switch (G) {
    case 1: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 1, NVT, REM>);
    case 2: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 2, NVT, REM>);
    case 3: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 3, NVT, REM>);
    case 4: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 4, NVT, REM>);
    case 5: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 5, NVT, REM>);
    case 6: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 6, NVT, REM>);
    case 7: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 7, NVT, REM>);
    case 8: return reinterpret_cast<void*>(&attn_i8_rows_kernel<HD, 8, NVT, REM>);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace dbi
