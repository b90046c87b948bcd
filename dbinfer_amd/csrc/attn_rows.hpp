// Dense fp32 GQA attention of a few query rows at once on the matrix cores:
// the causal chunk rows of decode_layer_chunk (model.cpp:956-981) for chunks
// too short for the prefill kernel, e.g. a speculative verify round (k + 1
// rows, speculative.cpp:64). Instantiated by attn_inst_f32_rows*.hip.
//
// Design (CDNA4, wave64, v_mfma_f32_16x16x4_f32: fp32 products, so every
// score and output is an fp32 accumulation of exact products, well inside
// the reference's fp32 tolerance):
//  - Grid (split, kv head, row group), 8 waves per workgroup. A workgroup
//    serves NV = 16 * NVT (NVT 3: 20) query vectors (row r, head g: r * G + g) of up to
//    NR = NV / G rows, so every K/V byte of the kv head crosses HBM once per
//    row group (one group for a C5 verify round: 5 rows x 4 heads = 20).
//  - Keys in 16-position tiles (one granule of the layout of
//    kv_internal.hpp), tile t -> wave t % 8 of the split; each tile's K and V
//    are loaded once into registers and serve all NVT vector tiles.
//  - S^T = K Q^T: A = K (16 keys x 4 dims), B = Q^T (4 dims x 16 vectors).
//    The dims of instruction (h, a, e) are permuted per lane group kk so that
//    a lane's operand is one 16-byte unit of the granule layout: dims
//    4 (4a + kk) + e + h hd/2 (the unit of K lane column c = 4a + kk, half h).
//    The result holds S[vector lane % 16][key 4 (lane / 16) + v] in lane l.
//  - O^T += V^T P^T: A = V^T (16 dims x 4 keys, dims VD i + tt of key
//    4 kk + j, VD = hd / 16 contiguous floats of one V unit pair), B = P^T
//    straight from the score registers (element j of lane group kk is key
//    4 kk + j). A lane's output is then hd/4 contiguous dims of its vector.
//  - Online softmax per vector (lane % 16): a lane's 4 keys, then the four
//    lane groups through two permlane swaps.
//  - Remainder tile (NVT 3, e.g. 5 rows x 4 heads = 16 + 4 vectors): the 4
//    vectors past the first 16 on v_mfma_f32_4x4x1_16b_f32, 16 blocks of
//    4 x 4 instead of a 16-column tile three quarters padding. QK^T: block
//    l / 4 takes keys 4 (n / 4) .. + 3 (rows, the lane's own K operand) and
//    vectors 16 .. 19 (columns: q of vector 16 + n % 4) over the lane
//    group's dims; the four lane groups' partial scores sum by two permlane
//    swaps. PV: block l / 4 takes key 4 kk + j (its weights fetched from
//    the lane that holds them) and dims VD (4 (n / 4) + r) + tt (rows, the
//    lane's own V operand); the lane groups' partial outputs (disjoint keys)
//    sum once, at the end. A quarter of the 16-column tile's matrix cycles.
//  - Split-K records as attn_kernel; the records are merged by a second
//    launch (attn_rows_merge), one workgroup per (row, head).
#pragma once

#include "attn_mfma.hpp"

namespace dbi {
namespace {

constexpr int kR4 = 0x124;  // DPP row_ror:4 (lane n of a row reads n - 4 mod 16)

// NVT 1 / 2: one / two 16-vector tiles; 3: one 16-vector tile and a
// remainder tile of 4 vectors on v_mfma_f32_4x4x1_16b_f32 (see the kernel)
template <int HD, int G, int NVT>
struct RCfg {
  static constexpr bool REM = NVT == 3;
  static constexpr int NTL = REM ? 2 : NVT;           // vector tiles held
  static constexpr int NV = REM ? 20 : 16 * NVT;      // query vectors per workgroup (padded)
  static constexpr int NR = NV / G;    // rows per workgroup
  static constexpr int NA = HD / 32;   // K units per half per lane (lane columns 4a + kk)
  static constexpr int VD = HD / 16;   // V dims per lane per key
  static constexpr int VU = VD / 4;    // V units per key per lane
  static constexpr int NT = HD / 16;   // PV output tiles
  static constexpr int OP = HD + 4;    // LDS row pitch of a wave's outputs (bank spread)
  static_assert(HD == 64 || HD == 128, "head dim");
  static_assert(G >= 1 && G <= NV, "query heads per kv head");
};

template <int HD, int G, int NVT>
__global__ __launch_bounds__(kThreads) void attn_rows_kernel(const AttnParams P) {
  using C = RCfg<HD, G, NVT>;
  constexpr int NA = C::NA, VD = C::VD, VU = C::VU, NT = C::NT, NR = C::NR, OP = C::OP;
  constexpr int NTL = C::NTL;
  constexpr bool REM = C::REM;
  constexpr int TILE = kGranule;
  constexpr int NCH = NTL == 1 ? 4 : 2;

  __shared__ __align__(16) float s_o[kWaves][16][OP];
  __shared__ float s_ml[kWaves][16][2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kk = lane >> 4;  // matrix column (vector / V dim row), lane group
  const int split = blockIdx.x;
  const int kh = blockIdx.y;
  const int row0 = blockIdx.z * NR;         // this workgroup's rows [row0, row0 + nr)
  const int nr = min(NR, P.rows - row0);
  const int nv = nr * G;                    // its query vectors
  const int nkeys = P.pos0 + row0 + nr;     // keys of its last row
  const int ntiles = (nkeys + TILE - 1) / TILE;
  const int t_end = min((split + 1) * P.chunks_per_split, ntiles);
  const size_t head_el = static_cast<size_t>(kh) * P.capg * HD;
  const int kv_bytes = P.capg * HD * 4;
  const rsrc_t rk = make_rsrc(P.kf + head_el, kv_bytes);
  const rsrc_t rv = make_rsrc(P.vf + head_el, kv_bytes);

  // byte offsets of this lane's operand units inside a granule
  int koff[2][NA], voff[4][VU];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int a = 0; a < NA; ++a)
      koff[h][a] = static_cast<int>(k_off_tiled(HD, false, n, 4 * (4 * a + kk) + (HD / 2) * h)) * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int u = 0; u < VU; ++u)
      voff[j][u] = static_cast<int>(v_off_tiled(HD, false, 4 * kk + j, VD * n + 4 * u)) * 4;

  // ---- q operands of the lane's vectors, dims 4 (4a + kk) + h hd/2 .. + 3,
  // in the log2 domain; padding vectors (>= nv) are 0
  // (the remainder tile: vector 16 + lane % 4, see below)
  float4 qv[NTL][2][NA];
  int lim[NTL];  // last key of each of the lane's vectors (causal)
  auto vec_of = [&](int vt) { return REM && vt == 1 ? 16 + (n & 3) : vt * 16 + n; };
#pragma unroll
  for (int vt = 0; vt < NTL; ++vt) {
    const int q = min(vec_of(vt), nv - 1);
    lim[vt] = P.pos0 + row0 + q / G;
    const float* qp =
        P.q + (static_cast<size_t>(row0 + q / G) * P.n_heads + kh * G + q % G) * HD + 4 * kk;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int a = 0; a < NA; ++a)
        qv[vt][h][a] = *reinterpret_cast<const float4*>(qp + 16 * a + (HD / 2) * h);
  }

  // ---- one tile's K and V units; a tile past t_end reads at the array's
  // end (the per-lane offset past num_records: the reads return 0, fetch
  // nothing)
  float4 kb[2][NA], vb[4][VU];
  auto tile_base = [&](int t) { return t < t_end ? t * TILE * HD * 4 : kv_bytes; };
  auto issue_k = [&](int t) {
    const int base = tile_base(t);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int a = 0; a < NA; ++a) kb[h][a] = stream_b128(rk, base + koff[h][a], 0);
  };
  auto issue_v = [&](int t) {
    const int base = tile_base(t);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < VU; ++u) vb[j][u] = stream_b128(rv, base + voff[j][u], 0);
  };

  // (q's loads go out first: vector loads return in order)
  __builtin_amdgcn_sched_barrier(0);
  int t = split * P.chunks_per_split + wave;
  issue_k(t);
  issue_v(t);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int vt = 0; vt < NTL; ++vt) {
    const float fq = vec_of(vt) < nv ? P.qscale : 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int a = 0; a < NA; ++a) qv[vt][h][a] *= fq;
  }

  float M[NTL], l[NTL];
  f32x4 acc[NTL][NT];
#pragma unroll
  for (int vt = 0; vt < NTL; ++vt) {
    M[vt] = kMinit;
    l[vt] = 0.0f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) acc[vt][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  for (; t < t_end; t += kWaves) {
    const int k0 = t * TILE;  // first key of the tile
    // ---- S^T in NCH independent chains per vector tile (4 independent
    // chains in all keep the matrix core's dependent issue covered)
    f32x4 sc[NTL][NCH];
#pragma unroll
    for (int vt = 0; vt < NTL; ++vt)
#pragma unroll
      for (int e = 0; e < NCH; ++e) sc[vt][e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const float4 x = kb[h][a];
        const float xe[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int vt = 0; vt < NTL; ++vt) {
          const float4 y = qv[vt][h][a];
          const float ye[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sc[vt][e % NCH] =
                REM && vt == 1
                    ? __builtin_amdgcn_mfma_f32_4x4x1f32(xe[e], ye[e], sc[vt][e % NCH], 0, 0, 0)
                    : __builtin_amdgcn_mfma_f32_16x16x4f32(xe[e], ye[e], sc[vt][e % NCH], 0, 0, 0);
        }
      }
    __builtin_amdgcn_sched_barrier(0);
    issue_k(t + kWaves);
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax per vector (lane % 16)
    float pw[NTL][4];
#pragma unroll
    for (int vt = 0; vt < NTL; ++vt) {
      const bool rem = REM && vt == 1;
      f32x4 s4 = sc[vt][0];
#pragma unroll
      for (int e = 1; e < NCH; ++e) s4 += sc[vt][e];
      // the remainder tile: lane l holds the partial sums of block l / 4 (the
      // lane group's dims) at keys 4 (n / 4) + v; the four lane groups sum
      // to the scores of vector 16 + n % 4
      if (rem) {
#pragma unroll
        for (int v = 0; v < 4; ++v) s4[v] = col_sum(s4[v]);
      }
      const int kq = rem ? 4 * (n >> 2) : 4 * kk;  // the lane's first key in the tile
      float s[4], mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        s[v] = k0 + kq + v <= lim[vt] ? s4[v] : -INFINITY;
        mx = fmaxf(mx, s[v]);
      }
      // (remainder: the max over the lanes n, n ^ 4, n ^ 8, n ^ 12 of a row)
      const float cm = rem ? fmaxf(fmaxf(mx, dpp<kR4>(mx)), dpp<kX8>(fmaxf(mx, dpp<kR4>(mx))))
                           : col_max(mx);
      const float mn = lazy_max(M[vt], cm);
      const float alpha = fast_exp2(M[vt] - mn);
      M[vt] = mn;
      float ls = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        pw[vt][v] = fast_exp2(s[v] - mn);
        ls += pw[vt][v];
      }
      l[vt] = fmaf(l[vt], alpha, ls);
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {  // (the maxima moved)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) acc[vt][tt] *= alpha;
      }
    }

    // ---- O^T += V^T P^T; keys past the group's last key weigh 0, and in
    // the final tile their (stale) V is zeroed so nothing non-finite enters
    const bool ragged = k0 + TILE > nkeys;  // uniform
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vd[VD];
#pragma unroll
      for (int u = 0; u < VU; ++u) {
        vd[4 * u + 0] = vb[j][u].x;
        vd[4 * u + 1] = vb[j][u].y;
        vd[4 * u + 2] = vb[j][u].z;
        vd[4 * u + 3] = vb[j][u].w;
      }
      if (ragged) {
        const bool ok = k0 + 4 * kk + j < nkeys;
#pragma unroll
        for (int d = 0; d < VD; ++d) vd[d] = ok ? vd[d] : 0.0f;
      }
#pragma unroll
      for (int vt = 0; vt < NTL; ++vt) {
        if (REM && vt == 1) {
          // block l / 4 takes key 4 kk + j: the weight of vector 16 + n % 4
          // there, from the lane whose scores hold it (lane 4 kk + n % 4)
          const float pr = __shfl(pw[1][j], 4 * kk + (n & 3));
#pragma unroll
          for (int tt = 0; tt < NT; ++tt)
            acc[1][tt] = __builtin_amdgcn_mfma_f32_4x4x1f32(vd[tt], pr, acc[1][tt], 0, 0, 0);
        } else {
#pragma unroll
          for (int tt = 0; tt < NT; ++tt)
            acc[vt][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[tt], pw[vt][j], acc[vt][tt], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_v(t + kWaves);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- per vector tile: wave states to LDS, the cross-wave combine, then
  // the output (single split) or this split's record of each row
#pragma unroll
  for (int vt = 0; vt < NTL; ++vt) {
    if (REM && vt == 1) {
      // lane l: the sums of its 4 keys (vector 16 + n % 4), the same in every
      // lane group; O^T partials over the lane group's keys at dims
      // VD (4 (n / 4) + v) + tt
      float lt = l[1] + dpp<kR4>(l[1]);
      lt += dpp<kX8>(lt);
      if (lane < 4) {
        s_ml[wave][lane][0] = M[1];
        s_ml[wave][lane][1] = lt;
      }
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[1][tt][v] = col_sum(acc[1][tt][v]);
      if (kk == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int u = 0; u < VU; ++u)
            *reinterpret_cast<float4*>(&s_o[wave][n & 3][VD * (4 * (n >> 2) + v) + 4 * u]) =
                make_float4(acc[1][4 * u][v], acc[1][4 * u + 1][v], acc[1][4 * u + 2][v],
                            acc[1][4 * u + 3][v]);
      }
    } else {
      const float lt = col_sum(l[vt]);
      if (kk == 0) {
        s_ml[wave][n][0] = M[vt];
        s_ml[wave][n][1] = lt;
      }
      // lane holds O^T[dim VD (4 kk + v) + tt][vector n]
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int u = 0; u < VU; ++u)
          *reinterpret_cast<float4*>(&s_o[wave][n][VD * (4 * kk + v) + 4 * u]) =
              make_float4(acc[vt][4 * u][v], acc[vt][4 * u + 1][v], acc[vt][4 * u + 2][v],
                          acc[vt][4 * u + 3][v]);
    }
    __syncthreads();
    const int q0 = vt * 16;
    const int nq = min(16, nv - q0);  // vectors of this tile (uniform)
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
    float* const rbase = P.part +
                         (static_cast<size_t>(row0) * P.nkv + kh) * record_region(P.nsplit, G, HD) +
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
    __syncthreads();  // s_o / s_ml are rewritten by the next vector tile
  }
}

// The split merge of a rows launch, as a second launch: one wave per (row,
// head) pair, merge_head() over the pair's split records (and, dense int8,
// the row's fp32 sinks). The records of a row group come from workgroups on
// every XCD, and one workgroup merging all of them (as the decode kernel's
// last arriver does) is bound by the bandwidth of its single CU; one
// workgroup per pair spreads the reads.
template <int HD, int G>
__global__ __launch_bounds__(64) void attn_rows_merge(const AttnParams P) {
  const int pr = blockIdx.x;  // (row, kv head, head) pair
  const int g = pr % G, kh = (pr / G) % P.nkv, qrow = pr / (G * P.nkv);
  if (P.n_sink > 0)
    merge_split<HD, G, true>(P, kh, qrow, g, threadIdx.x);
  else
    merge_split<HD, G, false>(P, kh, qrow, g, threadIdx.x);
}

template <int HD, int NVT>
void* pick_rows_g(int G) {
  switch (G) {
    case 1: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 1, NVT>);
    case 2: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 2, NVT>);
    case 3: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 3, NVT>);
    case 4: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 4, NVT>);
    case 5: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 5, NVT>);
    case 6: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 6, NVT>);
    case 7: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 7, NVT>);
    case 8: return reinterpret_cast<void*>(&attn_rows_kernel<HD, 8, NVT>);
    default: return nullptr;
  }
}

template <int HD>
void* pick_rows_merge_g(int G) {
  switch (G) {
    case 1: return reinterpret_cast<void*>(&attn_rows_merge<HD, 1>);
    case 2: return reinterpret_cast<void*>(&attn_rows_merge<HD, 2>);
    case 3: return reinterpret_cast<void*>(&attn_rows_merge<HD, 3>);
    case 4: return reinterpret_cast<void*>(&attn_rows_merge<HD, 4>);
    case 5: return reinterpret_cast<void*>(&attn_rows_merge<HD, 5>);
    case 6: return reinterpret_cast<void*>(&attn_rows_merge<HD, 6>);
    case 7: return reinterpret_cast<void*>(&attn_rows_merge<HD, 7>);
    case 8: return reinterpret_cast<void*>(&attn_rows_merge<HD, 8>);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace dbi
