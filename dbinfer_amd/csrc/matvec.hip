// Quantized matvecs of the layer offload and of the o_proj seam:
// matvec_q8_0_scalar / matvec_q4_0_scalar (matmul.cpp:56-99) of one
// activation row quantized with quantize_row_q8_0 (dequant.cpp:80-97), with
// the steps that Model::decode_layer runs around them on the same row fused
// into the launch:
//
//   rmsnorm in front (ops.cpp:7-17; model.cpp:738, 777, 913): every
//     workgroup sums the squares of the raw row itself and quantizes
//     x[i] * scale * w[i], so no normalized row is written or re-read;
//   up to three matrices over the same activation in one launch, their rows
//     concatenated (matvec_quant_fused of wq, wk, wv, model.cpp:740-745,
//     matmul.cpp:283);
//   a gate/up pair with silu(gate) * up as the epilogue (model.cpp:779-785);
//   the residual add as the epilogue (model.cpp:773-774, 786-787).
//
// Rows of in / 32 blocks with in a multiple of 64: a row is a whole number of
// block pairs (68 bytes Q8_0, 36 bytes Q4_0) and, with the weights 4-byte
// aligned, every pair starts 4-byte aligned. So a lane reads a pair as
// contiguous dwords; the first block's codes sit 2 bytes into their dword
// (one fixed funnel shift each) and the second block's codes are aligned.
//
// Work: a task is kNR row dot products (kNR consecutive rows, or kNR/2 rows
// each of gate and up); a unit is one chunk of 64 pairs of every row of a
// task, one pair per lane. Each workgroup takes a contiguous, balanced range
// of tasks and its waves deal the units round-robin. A wave requests its
// next unit row by row as it finishes summing the current one (the registers
// of row r are refilled as soon as row r is summed), so every wave keeps
// about kNR rows in flight; a wave that waits for all of a unit before
// requesting the next would move in lockstep rounds with every other wave,
// leaving HBM idle for a latency between rounds. The first unit is requested
// before the activation prologue when the row is short enough to be held in
// registers (its loads are issued first, since vector loads return in order).
// Rows of one chunk finish in their wave; longer rows (the down projection)
// are split over waves and summed in chunk order from LDS.
//
// Per block the integer dot product is exact (v_dot4_i32_i8) and its term is
// (f16(dw) * f16(dx)) * sumi in fp32, the reference's expression; terms are
// summed per lane and then across the wave, so a row agrees with the
// reference's sequential sum to the rounding of a dot product.
// HBM-bound: rows * in / 32 * (34 or 18) bytes per matrix.
#include "kv_internal.hpp"
#include "quant.hpp"

namespace dbi {
namespace {

constexpr int kMvThreads = 512;
constexpr int kMvWaves = kMvThreads / 64;
constexpr int kNR = 4;  // row dot products per task
constexpr int kWgPerCu = 2;

struct MvArgs {
  const float* x;   // activation row [in] (raw when nw is set)
  const float* nw;  // rmsnorm weight [in], or null
  float eps;
  int in, nbk, npair;
  const uint8_t* w[3];  // plain: the segments' weights; pair: gate, up
  float* y[3];          // plain: the segments' outputs; pair: y[0]
  int seg_end[3];       // plain: cumulative row ends of the segments
  int rows;             // plain: total rows; pair: rows of each matrix
  int tasks, chunks;    // tasks of kNR row dots; units per task
  int pair, acc;
};

template <bool Q4>
struct Pair {
  static constexpr int kBytes = Q4 ? 36 : 68;  // two blocks
  static constexpr int kDw = kBytes / 4;
};

// Global-address-space views: the weight and row pointers reach the loads
// through selects over the argument struct, where the compiler cannot prove
// their address space and would emit flat loads.
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const float gf32;
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f4v gf4;
typedef __attribute__((address_space(1))) float gf32w;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ inline uint32_t pack4(int8_t a, int8_t b, int8_t c, int8_t d) {
  return static_cast<uint32_t>(static_cast<uint8_t>(a)) |
         (static_cast<uint32_t>(static_cast<uint8_t>(b)) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(c)) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(d)) << 24);
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float dpp_add(float v, int ctrl) {
  // v + v of the lane that the DPP pattern names (row-local patterns only)
  switch (ctrl) {
    case 0xB1:
      return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    case 0x4E:
      return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    case 0x141:
      return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    default:
      return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  }
}

// The row pointers of task t's row dots.
template <bool Q4>
__device__ inline void task_rows(const MvArgs& a, int t, const uint8_t* wrow[kNR]) {
  const size_t row_bytes = static_cast<size_t>(a.npair) * Pair<Q4>::kBytes;
  if (a.pair) {
    constexpr int H = kNR / 2;
#pragma unroll
    for (int r = 0; r < kNR; ++r) {
      const int row = min(t * H + r % H, a.rows - 1);
      wrow[r] = a.w[r / H] + static_cast<size_t>(row) * row_bytes;
    }
  } else {
    const int first = t * kNR;
    const int s = first >= a.seg_end[0] ? (first >= a.seg_end[1] ? 2 : 1) : 0;
    const int start = s ? a.seg_end[s - 1] : 0;
#pragma unroll
    for (int r = 0; r < kNR; ++r) {
      const int row = min(first + r, a.seg_end[s] - 1) - start;
      wrow[r] = a.w[s] + static_cast<size_t>(row) * row_bytes;
    }
  }
}

// Weight loads of one row of a unit: pair c * 64 + lane of the row (past
// the row's end the last pair is re-read and its terms skipped).
template <bool Q4>
__device__ __forceinline__ void load_row(uint32_t wd[Pair<Q4>::kDw], const uint8_t* wrow, int c,
                                         int npair, int lane) {
  const int p = min(c * 64 + lane, npair - 1);
  gu32* base = (gu32*)(wrow + static_cast<size_t>(p) * Pair<Q4>::kBytes);
#pragma unroll
  for (int i = 0; i < Pair<Q4>::kDw; ++i) wd[i] = base[i];
}

// The activation pair a lane's weights meet in chunk c. LDS holds the row as
// s_code[block][8] code dwords and s_dx[block] = f16(d) as float (and, for
// Q4_0, s_sum[block] its code sum as the nibble offset's factor).
struct ActPair {
  uint32_t xa[8], xb[8];
  float dxa, dxb;
  int sa, sb;
  bool valid;
};

template <bool Q4>
__device__ __forceinline__ void load_act(ActPair& x, int c, int npair, int lane,
                                         const uint32_t* s_code, const float* s_dx,
                                         const int* s_sum) {
  const int p0 = c * 64 + lane;
  x.valid = p0 < npair;
  const int p = min(p0, npair - 1);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x.xa[i] = s_code[(2 * p) * 8 + i];
    x.xb[i] = s_code[(2 * p + 1) * 8 + i];
  }
  x.dxa = s_dx[2 * p];
  x.dxb = s_dx[2 * p + 1];
  x.sa = x.sb = 0;
  if constexpr (Q4) {
    x.sa = s_sum[2 * p];
    x.sb = s_sum[2 * p + 1];
  }
}

// One row's two block terms added to acc.
template <bool Q4>
__device__ __forceinline__ void sum_row(const uint32_t w[Pair<Q4>::kDw], const ActPair& x,
                                        float& acc) {
  // block A: scale in the low half of dword 0, data from byte 2;
  // block B: scale in the high half of dword kDw/2, data from dword kDw/2 + 1
  constexpr int HB = Pair<Q4>::kDw / 2;
  const float dwa =
      static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[0] & 0xffffu)));
  const float dwb =
      static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[HB] >> 16)));
  int ia = 0, ib = 0;
  if constexpr (Q4) {
    // element j: low nibble of byte j; element j + 16: its high nibble
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t ca = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
      const uint32_t cb = w[HB + 1 + i];
      ia = __builtin_amdgcn_sdot4(static_cast<int>(ca & 0x0F0F0F0Fu), static_cast<int>(x.xa[i]), ia, false);
      ia = __builtin_amdgcn_sdot4(static_cast<int>((ca >> 4) & 0x0F0F0F0Fu), static_cast<int>(x.xa[4 + i]), ia, false);
      ib = __builtin_amdgcn_sdot4(static_cast<int>(cb & 0x0F0F0F0Fu), static_cast<int>(x.xb[i]), ib, false);
      ib = __builtin_amdgcn_sdot4(static_cast<int>((cb >> 4) & 0x0F0F0F0Fu), static_cast<int>(x.xb[4 + i]), ib, false);
    }
    ia -= 8 * x.sa;
    ib -= 8 * x.sb;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t ca = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
      ia = __builtin_amdgcn_sdot4(static_cast<int>(ca), static_cast<int>(x.xa[i]), ia, false);
      ib = __builtin_amdgcn_sdot4(static_cast<int>(w[HB + 1 + i]), static_cast<int>(x.xb[i]), ib, false);
    }
  }
  const float t = acc + (dwa * x.dxa) * static_cast<float>(ia);
  acc = x.valid ? t + (dwb * x.dxb) * static_cast<float>(ib) : acc;
}

// A unit's kNR lane sums, reduced together: two halving steps leave lane l
// with a partial of row l >> 4, four in-row DPP steps finish it; lane 16r
// returns row r's sum.
__device__ inline float reduce_unit(const float acc[kNR], int lane) {
  const bool h5 = lane >= 32, h4 = (lane & 16) != 0;
  const float b0 = (h5 ? acc[2] : acc[0]) + __shfl_xor(h5 ? acc[0] : acc[2], 32);
  const float b1 = (h5 ? acc[3] : acc[1]) + __shfl_xor(h5 ? acc[1] : acc[3], 32);
  float v = (h4 ? b1 : b0) + __shfl_xor(h4 ? b0 : b1, 16);
  v = dpp_add(v, 0xB1);   // quad_perm [1,0,3,2]
  v = dpp_add(v, 0x4E);   // quad_perm [2,3,0,1]
  v = dpp_add(v, 0x141);  // row_half_mirror
  return dpp_add(v, 0x140);  // row_mirror
}

// Row r of task t: plain rows go into their segment (y = v or y += v, two
// roundings as proj then x + proj); pair tasks write silu(gate) * up for
// r < kNR / 2 (gate row r, up row r + kNR / 2).
__device__ inline void put_row(const MvArgs& a, int t, int r, float v, float up) {
  if (a.pair) {
    constexpr int H = kNR / 2;
    const int row = t * H + r;
    if (r < H && row < a.rows) ((gf32w*)a.y[0])[row] = (v / (1.0f + expf(-v))) * up;
  } else {
    const int first = t * kNR;
    const int s = first >= a.seg_end[0] ? (first >= a.seg_end[1] ? 2 : 1) : 0;
    const int start = s ? a.seg_end[s - 1] : 0;
    const int row = first + r;
    if (row < a.seg_end[s]) {
      gf32w* y = (gf32w*)(a.y[s] + (row - start));
      *y = a.acc ? *y + v : v;
    }
  }
}

// Row r of task t from its chunk partials, summed in chunk order (so the
// result does not depend on which wave ran which chunk).
__device__ inline void finish_row(const MvArgs& a, int t, int r, const float* part, int C) {
  auto row_sum = [&](int rr) {
    float v = 0.0f;
    for (int c = 0; c < C; ++c) v += part[c * kNR + rr];
    return v;
  };
  put_row(a, t, r, row_sum(r), a.pair && r < kNR / 2 ? row_sum(r + kNR / 2) : 0.0f);
}

template <typename F>
__device__ __forceinline__ float dpp8(float v, F op) {
  // op over the 8 lanes of an aligned group: quad_perm [1,0,3,2], [2,3,0,1],
  // then row_half_mirror (lane i with 7 - i)
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  return op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
}

__device__ __forceinline__ int dpp8_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  return v + __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
}

// Elements 4f .. 4f + 3 of the activation row (float4 f; thread f % kMvThreads
// of the workgroup, so the 8 float4 of a block sit in 8 adjacent lanes):
// quantize_row_q8_0's arithmetic with the block max over the 8 lanes
// (max|x| is order-free), d = amax / 127, id = 1 / d, the stored scale
// f16(d), codes clamp(lround(x * id), +-127). Lane f % 8 writes code dword
// f % 8 of block f / 8; the block's first lane its scale (and, for Q4_0, the
// block's code sum). Every lane of the group calls it (live == false: a
// float4 past the row, which only ever fills whole groups).
template <bool Q4>
__device__ __forceinline__ void quantize4(f4v t, int f, bool live, uint32_t* s_code, float* s_dx,
                                          int* s_sum) {
  float m = max_f(max_f(fabsf(t.x), fabsf(t.y)), max_f(fabsf(t.z), fabsf(t.w)));
  m = dpp8(m, [](float a, float b) { return max_f(a, b); });
  const float d = m / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const int8_t c0 = quant_code(t.x, id), c1 = quant_code(t.y, id);
  const int8_t c2 = quant_code(t.z, id), c3 = quant_code(t.w, id);
  int sum = 0;
  if constexpr (Q4) sum = dpp8_sum(c0 + c1 + c2 + c3);
  if (live) {
    s_code[f] = pack4(c0, c1, c2, c3);
    if ((f & 7) == 0) {
      s_dx[f >> 3] = static_cast<float>(static_cast<_Float16>(d));
      if constexpr (Q4) s_sum[f >> 3] = sum;
    }
  }
}

// float4s of the row each thread holds through the prologue (rows up to
// kHold * 4 * kMvThreads elements are read once, before the weights)
constexpr int kHold = 2;

struct RowHold {
  f4v x[kHold], w[kHold];
};

// The held part of the activation row (and of the norm weight), loaded
// before the first unit's weights so that the prologue's wait on it does not
// wait on them (vector loads return in order).
__device__ __forceinline__ void hold_row(const MvArgs& a, RowHold& h) {
  const int n4 = a.in / 4;
#pragma unroll
  for (int k = 0; k < kHold; ++k) {
    const int f = min(static_cast<int>(threadIdx.x) + k * kMvThreads, n4 - 1);
    h.x[k] = ((gf4*)a.x)[f];
    if (a.nw != nullptr) h.w[k] = ((gf4*)a.nw)[f];
  }
}

// The activation row into LDS as Q8_0 blocks; with nw the row is rmsnorm'd
// first (scale = 1 / sqrt(sumsq / in + eps), x[i] * scale * w[i]; the sum of
// squares is a tree over the workgroup).
template <bool Q4>
__device__ inline void prologue(const MvArgs& a, const RowHold& h, uint32_t* s_code, float* s_dx,
                                int* s_sum, float* s_red) {
  const int n4 = a.in / 4;
  const bool held = n4 <= kHold * kMvThreads;
  float scale = 1.0f;
  if (a.nw != nullptr) {
    float ss = 0.0f;
    if (held) {
#pragma unroll
      for (int k = 0; k < kHold; ++k) {
        if (static_cast<int>(threadIdx.x) + k * kMvThreads < n4) {
          const f4v t = h.x[k];
          ss += t.x * t.x;
          ss += t.y * t.y;
          ss += t.z * t.z;
          ss += t.w * t.w;
        }
      }
    } else {
      for (int f = threadIdx.x; f < n4; f += kMvThreads) {
        const f4v t = ((gf4*)a.x)[f];
        ss += t.x * t.x;
        ss += t.y * t.y;
        ss += t.z * t.z;
        ss += t.w * t.w;
      }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
    lds_barrier();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kMvWaves; ++i) tot += s_red[i];
    scale = 1.0f / sqrtf(tot / static_cast<float>(a.in) + a.eps);
  }
  auto normed = [&](f4v t, f4v g) {
    if (a.nw != nullptr) {
      t.x = t.x * scale * g.x;
      t.y = t.y * scale * g.y;
      t.z = t.z * scale * g.z;
      t.w = t.w * scale * g.w;
    }
    return t;
  };
  if (held) {
#pragma unroll
    for (int k = 0; k < kHold; ++k) {
      const int f = static_cast<int>(threadIdx.x) + k * kMvThreads;
      if (k * kMvThreads < n4)  // whole groups live or not
        quantize4<Q4>(normed(h.x[k], h.w[k]), f, f < n4, s_code, s_dx, s_sum);
    }
  } else {
    // longer rows stream through in groups of 4 float4 per thread
    for (int f0 = 0; f0 < n4; f0 += 4 * kMvThreads) {
      f4v xs[4], ws[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int f = min(f0 + static_cast<int>(threadIdx.x) + k * kMvThreads, n4 - 1);
        xs[k] = ((gf4*)a.x)[f];
        if (a.nw != nullptr) ws[k] = ((gf4*)a.nw)[f];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int f = f0 + static_cast<int>(threadIdx.x) + k * kMvThreads;
        if (f0 + k * kMvThreads < n4) quantize4<Q4>(normed(xs[k], ws[k]), f, f < n4, s_code, s_dx, s_sum);
      }
    }
  }
  lds_barrier();
}

// Work of a workgroup: a contiguous, balanced range of tasks, taken in
// batches of at most kBatchUnits units (task, chunk) that the waves deal
// round-robin. Rows of one chunk finish in the wave that summed them; longer
// rows park each unit's kNR row sums in LDS and, after a barrier, the
// workgroup's threads finish the batch's rows.
constexpr int kBatchUnits = 512;

template <bool Q4>
__global__ __launch_bounds__(kMvThreads) void matvec_q_kernel(const MvArgs a) {
  extern __shared__ uint32_t s_lds[];  // s_code [nbk][8], s_dx [nbk], s_sum [nbk]
  uint32_t* s_code = s_lds;
  float* s_dx = reinterpret_cast<float*>(s_lds + a.nbk * 8);
  int* s_sum = reinterpret_cast<int*>(s_lds + a.nbk * 9);
  __shared__ float s_red[kMvWaves];
  __shared__ float s_part[kBatchUnits * kNR];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = a.chunks;
  const int t0 = static_cast<int>(static_cast<long long>(a.tasks) * blockIdx.x / gridDim.x);
  const int t1 = static_cast<int>(static_cast<long long>(a.tasks) * (blockIdx.x + 1) / gridDim.x);
  const int bt = max(1, kBatchUnits / C);  // tasks per batch
  RowHold h;
  hold_row(a, h);
  uint32_t wd[kNR][Pair<Q4>::kDw];
  const uint8_t* wr[kNR];
  // A wave's units in order: (batch tb, unit u) then u + kMvWaves, or the
  // next batch's unit `wave` (only the last batch can be short of it). The
  // loads run one unit ahead, row by row: as soon as row r of a unit is
  // summed, row r of the wave's next unit is requested into the same
  // registers, so every wave keeps about kNR rows in flight without a second
  // register set. The first unit is requested before the activation
  // prologue.
  auto batch_units = [&](int tb) { return min(bt, t1 - tb) * C; };
  int ltb = t0, lu = wave;  // the unit in flight
  auto next = [&]() {  // false: the wave has no further unit
    if (lu + kMvWaves < batch_units(ltb)) {
      lu += kMvWaves;
      return true;
    }
    if (ltb + bt < t1 && wave < batch_units(ltb + bt)) {
      ltb += bt;
      lu = wave;
      return true;
    }
    return false;
  };
  auto first_load = [&]() {
    if (wave < batch_units(t0)) {
      const int k = lu / C;
      task_rows<Q4>(a, ltb + k, wr);
#pragma unroll
      for (int r = 0; r < kNR; ++r) load_row<Q4>(wd[r], wr[r], lu - k * C, a.npair, lane);
    }
  };
  if (a.in / 4 <= kHold * kMvThreads) {
    // the row is held: its loads are already ahead of the weights
    first_load();
    prologue<Q4>(a, h, s_code, s_dx, s_sum, s_red);
  } else {
    // a longer row streams through the prologue first (its loads would
    // otherwise queue behind the weights')
    prologue<Q4>(a, h, s_code, s_dx, s_sum, s_red);
    first_load();
  }
#pragma unroll 1
  for (int tb = t0; tb < t1; tb += bt) {
    const int nu = batch_units(tb);
#pragma unroll 1
    for (int u = wave; u < nu; u += kMvWaves) {
      ActPair x;
      load_act<Q4>(x, u % C, a.npair, lane, s_code, s_dx, s_sum);
      const bool more = next();  // wave-uniform
      const int nk = lu / C, nc = lu - nk * C;
      task_rows<Q4>(a, ltb + nk, wr);
      float acc[kNR];
#pragma unroll
      for (int r = 0; r < kNR; ++r) {
        acc[r] = 0.0f;
        sum_row<Q4>(wd[r], x, acc[r]);
        if (more) load_row<Q4>(wd[r], wr[r], nc, a.npair, lane);
      }
      const float v = reduce_unit(acc, lane);
      if (C == 1) {
        // a unit is a whole task: lane 16r holds row r (for pairs, up row r
        // sits in lane 16r + 32)
        const float up = __shfl_down(v, 32);
        if ((lane & 15) == 0) put_row(a, tb + u, lane >> 4, v, up);
      } else if ((lane & 15) == 0) {
        s_part[u * kNR + (lane >> 4)] = v;
      }
    }
    if (C > 1) {
      lds_barrier();
      for (int i = threadIdx.x; i < nu / C * kNR; i += kMvThreads) {
        const int k = i / kNR;
        finish_row(a, tb + k, i - k * kNR, s_part + k * C * kNR, C);
      }
      lds_barrier();
    }
  }
}

int cu_count() {
  static int n[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (n[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        c <= 0)
      c = 256;
    n[dev] = c;
  }
  return n[dev];
}

}  // namespace

int matvec_rows_per_task() { return kNR; }

hipError_t launch_matvec_q(const MatvecCall& c, hipStream_t st) {
  if (c.in <= 0 || c.in % 64 != 0) return hipErrorInvalidValue;
  MvArgs a{};
  a.x = c.x;
  a.nw = c.norm_w;
  a.eps = c.eps;
  a.in = c.in;
  a.nbk = c.in / 32;
  a.npair = c.in / 64;
  a.pair = c.pair ? 1 : 0;
  a.acc = c.acc ? 1 : 0;
  int end = 0;
  for (int s = 0; s < 3; ++s) {
    const bool real = s < c.nseg;
    a.w[s] = static_cast<const uint8_t*>(real ? c.w[s] : c.w[0]);
    a.y[s] = real ? c.y[s] : c.y[0];
    end += real && !c.pair ? c.rows[s] : 0;
    a.seg_end[s] = end;
  }
  if (c.pair) {
    a.rows = c.rows[0];
    a.tasks = (a.rows + kNR / 2 - 1) / (kNR / 2);
  } else {
    a.rows = end;
    a.tasks = (end + kNR - 1) / kNR;
  }
  a.chunks = (a.npair + 63) / 64;
  if (a.tasks == 0) return hipSuccess;
  // one unit per wave where the units allow it, every CU busy while there
  // are tasks for it; at most two workgroups per CU for rows of one chunk,
  // one for longer rows (each workgroup re-quantizes the whole activation)
  const int ncu = cu_count();
  const long long units = static_cast<long long>(a.tasks) * a.chunks;
  const int grid = static_cast<int>(
      min(static_cast<long long>((a.chunks > 1 ? 1 : kWgPerCu) * ncu),
          max(static_cast<long long>(min(ncu, a.tasks)), (units + kMvWaves - 1) / kMvWaves)));
  const size_t lds = static_cast<size_t>(a.nbk) * (c.q4 ? 10 : 9) * sizeof(uint32_t);
  if (c.q4)
    hipLaunchKernelGGL(matvec_q_kernel<true>, dim3(grid), dim3(kMvThreads), lds, st, a);
  else
    hipLaunchKernelGGL(matvec_q_kernel<false>, dim3(grid), dim3(kMvThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace dbi
