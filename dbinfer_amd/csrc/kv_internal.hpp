// Internal state of a dbi_kv handle and the kernel launchers shared by the
// translation units of libdbi_kv.so.
//
// Device storage is head-major, so the keys of one kv head are one contiguous
// stream for decode attention (the reference stores [slot][kv_head][hd],
// model.hpp:108-214; dbi_kv_export converts back):
//   fp32 (dense, ring)  k, v          [L][nkv][capg*hd]   fp32, granule layout
//   int8                k8, v8        [L][nkv][capg*hd]   int8 codes, granule layout
//                       v_scale       [L][nkv][capg][nb]  fp32
//   ring int8           k_scale       [L][nkv][capg][nb]  fp32 (per 32-block)
//   dense int8          k_scale       [L][nkv][ng][hd]    fp32 (per channel, per 32-token group)
//                       k_raw         [L][32][nkv*hd]     fp32 (reference order)
//                       k_sink,v_sink [L][nkv][ns][hd]    fp32
//   ring                rope_cs       [cap][hd/2]         float2 (cos, sin)
//   dense (producer)    rope_dd       [cap][hd/2]         double2 (cos, sin), built on
//                                                         the producer's first call
// capg is the capacity rounded up to a multiple of 64 positions (the reads of
// the attention and prefill kernels are whole 32- / 64-position pieces).
//
// Dense int8 (head dims 64 and 128) uses the matrix-core layout below
// (k_off_i8d / v_off_i8d); fp32 and the int8 ring use the granule layout.
//
// Granule layout (head dims 64 and 128; other head dims are stored row-major
// [pos][hd]): 16 positions per granule, 16*hd elements. A wave reads one
// "slot" of a granule per 64 lanes x 8 elements, each load instruction one
// contiguous KiB: int8 [slot pair][lane][2 slots][8] (one 16-byte load per
// lane covers two slots), fp32 [slot][half][lane][4]. Lane
// l = r*LPR + c, LPR = hd/8 lanes per position row, RPW = 64/LPR rows; slot j
// of row r holds granule position i*RPW + r, with i = j for V and
// i = j ^ kslot_xor(c) for K (the permutation that lets the attention kernel
// reduce 16 lanes' partial dots with one DPP add per position, see
// attention.hip). K lane c holds dims 4c..4c+3 and hd/2+4c..hd/2+4c+3 (rope
// pairs d, d+hd/2 in one lane); V lane c holds dims 8c..8c+7.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "dbi_kv.h"

namespace dbi {

constexpr int kBlock = 32;   // kKvBlock, model.hpp:81
constexpr int kKGroup = 32;  // kKvKGroup, model.hpp:87

struct KvGeom {
  int n_layers, cap, nkv, hd, nb, n_sink, window, ngroups;
  int capg;    // cap rounded up to a multiple of kCapAlign (rows per kv head)
  bool int8, ring;
  bool tiled;  // granule layout (hd 64 / 128); row-major otherwise
};

constexpr int kGranule = 16;
// the attention kernels read whole 32-position chunks, the prefill kernel
// whole 64-position stages
constexpr int kCapAlign = 64;

__host__ __device__ inline int kslot_xor(int hd, int c) {
  return hd == 128 ? ((((c >> 3) & 1) << 1) ^ ((c >> 2) & 1)) : ((c >> 2) & 1);
}

__host__ __device__ inline size_t granule_off(int hd, bool int8, int pos, int j, int l, int e) {
  const size_t base = static_cast<size_t>(pos >> 4) * kGranule * hd + static_cast<size_t>(j) * 512;
  return int8 ? base - (j & 1) * 512 + l * 16 + (j & 1) * 8 + e
              : base + (e >> 2) * 256 + l * 4 + (e & 3);
}

// Offset of element (pos, d) inside one (layer, kv head) K / V array of the
// granule layout (hd 64 or 128).
__host__ __device__ inline size_t k_off_tiled(int hd, bool int8, int pos, int d) {
  const int LPR = hd >> 3, RPW = 64 / LPR, pp = pos & 15, r = pp % RPW, i = pp / RPW;
  const int half = hd >> 1;
  const bool hi = d >= half;
  const int dd = hi ? d - half : d;
  const int c = dd >> 2, e = (dd & 3) + (hi ? 4 : 0);
  return granule_off(hd, int8, pos, i ^ kslot_xor(hd, c), r * LPR + c, e);
}
__host__ __device__ inline size_t v_off_tiled(int hd, bool int8, int pos, int d) {
  const int LPR = hd >> 3, RPW = 64 / LPR, pp = pos & 15, r = pp % RPW, i = pp / RPW;
  return granule_off(hd, int8, pos, i, r * LPR + (d >> 3), d & 7);
}

// Dense int8 matrix-core layout, by 32-position chunks (one K group) of
// 32*hd bytes, so that every 16-byte lane load is a bf16 MFMA operand once
// converted (v_mfma_f32_16x16x32_bf16: lane m + 16*(k/8) holds k % 8 of row /
// column m):
//  K: per granule h (16 positions) hd/64 blocks of 1 KiB, [lane][16 bytes];
//     lane n + 16*g of block jp holds position 16h + n, channels
//     64jp + 32*j2 + 8g + e at byte 8*j2 + e (k-steps 2jp and 2jp + 1).
//  V: hd/32 blocks of 1 KiB, [lane][16 bytes]; lane n + 16*g of block tp
//     holds channel 16*(2tp + tt) + n at bytes 8*tt + s, s = 0..7 the
//     positions 16*(s/4) + 4g + s%4 (the positions the lane's QK^T scores
//     cover, so softmax weights feed the PV product without moving).
__host__ __device__ inline size_t k_off_i8d(int hd, int pos, int d) {
  const int p = pos & 31, h = p >> 4, n = p & 15;
  const int jp = d >> 6, j2 = (d >> 5) & 1, g = (d >> 3) & 3, e = d & 7;
  return static_cast<size_t>(pos >> 5) * 32 * hd + static_cast<size_t>(h * (hd >> 6) + jp) * 1024 +
         (n + 16 * g) * 16 + j2 * 8 + e;
}
__host__ __device__ inline size_t v_off_i8d(int hd, int pos, int d) {
  const int p = pos & 31, h = p >> 4, q = p & 15, g = q >> 2, s = 4 * h + (q & 3);
  const int t = d >> 4, n = d & 15, tp = t >> 1, tt = t & 1;
  return static_cast<size_t>(pos >> 5) * 32 * hd + static_cast<size_t>(tp) * 1024 +
         (n + 16 * g) * 16 + tt * 8 + s;
}

// Offset of element (pos, d) inside one (layer, kv head) K array.
__host__ __device__ inline size_t k_off(const KvGeom& g, int pos, int d) {
  if (!g.tiled) return static_cast<size_t>(pos) * g.hd + d;
  return g.int8 && !g.ring ? k_off_i8d(g.hd, pos, d) : k_off_tiled(g.hd, g.int8, pos, d);
}

// Offset of element (pos, d) inside one (layer, kv head) V array.
__host__ __device__ inline size_t v_off(const KvGeom& g, int pos, int d) {
  if (!g.tiled) return static_cast<size_t>(pos) * g.hd + d;
  return g.int8 && !g.ring ? v_off_i8d(g.hd, pos, d) : v_off_tiled(g.hd, g.int8, pos, d);
}

// Elements of one (layer, kv head) K or V array.
__host__ __device__ inline size_t head_elems(const KvGeom& g) {
  return static_cast<size_t>(g.capg) * g.hd;
}

struct KvStore {
  float* k = nullptr;
  float* v = nullptr;
  int8_t* k8 = nullptr;
  int8_t* v8 = nullptr;
  float* k_scale = nullptr;
  float* v_scale = nullptr;
  float* k_raw = nullptr;
  float* k_sink = nullptr;
  float* v_sink = nullptr;
  float2* rope_cs = nullptr;
  double2* rope_dd = nullptr;
};

// Split-K workspace: partial (o, m, l) of every split of one attention call.
struct Workspace {
  float* part = nullptr;
  size_t part_floats = 0;
  unsigned* counters = nullptr;  // split arrivals per (row, kv head); zero between launches
  size_t counters_n = 0;
  float* staging = nullptr;  // device staging for host-pointer calls
  unsigned char* pinned = nullptr;  // pinned host chunk for prefix-file transfers
  size_t staging_floats = 0;
  float* prod = nullptr;  // producer output: roped q, roped k, biased v rows
  size_t prod_floats = 0;
  // verify round: slice keys, arrival counter and the host variant's token
  // staging, one fixed-size allocation made on first use
  unsigned char* verify = nullptr;
};

// Ring state of one attention call (resident set of n_seen = pos + 1).
struct RingView {
  int n_res;  // resident count
  int s;      // n_sink
  int W;      // window
  int base;   // slot offset of the oldest window token, 0 until the window is full
};

// Parameters of one attention launch (decode: rows == 1).
struct AttnCall {
  int layer;
  int rows;      // query rows (1 for decode, n for chunk)
  int pos0;      // row r attends keys [0, pos0 + r]  (dense); ring: n_res keys
  int n_heads;
  float scale;
  const float* q;  // device [rows][n_heads][hd]
  float* out;      // device [rows][n_heads][hd]
  RingView ring;
  // fused decode step: append this row (device [nkv*hd] each) at position
  // app_pos, storage row app_slot, before attending; app_slot < 0: none
  const float* app_k = nullptr;
  const float* app_v = nullptr;
  int app_slot = -1;
  int app_pos = 0;
  // decode from raw projections (rows == 1): q is the raw q and app_k/app_v
  // the raw k/v; each bias (or null) is added, and with rope_row (the
  // (cos, sin) row of the position, dense layouts) q and k are roped
  const float* q_bias = nullptr;
  const float* k_bias = nullptr;
  const float* v_bias = nullptr;
  const double2* rope_row = nullptr;
};

// Launchers (return a hipError_t of the launch).
hipError_t launch_append(const KvGeom& g, const KvStore& s, int layer, int pos0, int n,
                         const float* k, const float* v, hipStream_t st);
// Returns hipErrorNotSupported for shapes without a kernel instance.
hipError_t launch_attention(const KvGeom& g, const KvStore& s, Workspace& ws,
                            const AttnCall& c, hipStream_t st);
// Number of partial floats one call needs (for workspace sizing).
size_t attention_workspace_need(const KvGeom& g, const AttnCall& c);

// Causal chunks of at least this many rows over the dense fp32 cache run on
// the matrix cores (prefill.hip); shorter ones (verify rounds) through
// launch_attention, whose many small per-wave streams keep more bytes in
// flight than the prefill kernel's one staged stream per workgroup.
constexpr int kPrefillMinRows = 64;
constexpr int kPrefillMaxSplits = 8;  // key splits of one chunk (workspace records)
bool prefill_supported(const KvGeom& g, int n_heads, int rows);
size_t prefill_workspace_need(const KvGeom& g, const AttnCall& c);
hipError_t launch_prefill(const KvGeom& g, const KvStore& s, Workspace& ws, const AttnCall& c,
                          hipStream_t st);
size_t attention_counters_need(const KvGeom& g, const AttnCall& c);
// The largest record floats / counters a one-row decode call of n_heads can
// need at any position (the planner's split cap bounds both).
size_t attention_workspace_bound(const KvGeom& g, int n_heads);
size_t attention_counters_bound(const KvGeom& g);
bool attention_supported(const KvGeom& g, int n_heads);
// Key splits (partial records per query row and kv head) of a call.
int attention_split_count(const KvGeom& g, const AttnCall& c);
int prefill_split_count(const KvGeom& g, const AttnCall& c);

// One producer launch (produce.hip): rows [pos0, pos0 + rows) of raw q/k/v
// projections (device, row-major [rows][heads*hd]) plus optional biases
// become the roped q, roped k and biased v rows the append and attention
// kernels take (a ring: biases only).
struct ProduceCall {
  int rows, pos0, n_heads;
  const float* q;
  const float* k;
  const float* v;
  const float* q_bias;
  const float* k_bias;
  const float* v_bias;
  float* q_out;
  float* k_out;
  float* v_out;
};
hipError_t launch_produce(const KvGeom& g, const double2* rope_dd, const ProduceCall& c,
                          hipStream_t st);
// Host table of (cos, sin) for every position < cap and pair of the head
// dim, [cap][hd/2], with tensor::rope's fp64 expressions (ops.cpp:27-30).
// False for an odd head dim.
bool rope_table_host(const KvGeom& g, float theta, double2* tab);

// Prefix pack/unpack between [L][len][nkv][hd] and the head-major store
// (is_k selects the K or the V granule layout).
hipError_t launch_prefix_pack(const KvGeom& g, const float* src_store, float* dst, int len,
                              bool is_k, hipStream_t st);
hipError_t launch_prefix_unpack(const KvGeom& g, const float* src, float* dst_store, int len,
                                bool is_k, hipStream_t st);
// int8 codes between the granule store and the file's
// [L][len][nkv][hd] (both directions; unpack = file -> store)
hipError_t launch_prefix_codes(const KvGeom& g, int8_t* store, int8_t* file, int len, bool is_k,
                               bool unpack, hipStream_t st);
// store [L][nkv][dev_rows][inner] <-> file [L][rows][nkv][inner] (first rows)
hipError_t launch_rows_pack(float* store, float* file, int n_layers, int nkv, int dev_rows,
                            int rows, int inner, bool unpack, hipStream_t st);

// Speculative verify round, token side (verify.hip): argmax of each of the
// rows = k+1 logit rows, then the merge against the k draft tokens.
constexpr int kMaxVerifyDraft = 64;
constexpr int kMaxVerifyRows = kMaxVerifyDraft + 1;
constexpr int kMaxVerifySlices = 64;  // workgroups per row
struct VerifyCall {
  const float* logits;   // device [rows][vocab]
  const int32_t* draft;  // device [rows - 1]
  int32_t* verified;     // device [rows]
  int32_t* accepted;     // device [1]
  unsigned long long* keys;  // device [kMaxVerifyRows * kMaxVerifySlices]
  unsigned* counter;     // device, zero between calls (the kernel resets it)
  int rows, vocab;
};
hipError_t launch_verify(const VerifyCall& c, hipStream_t st);

// The unfused matvecs of decode_layer (oproj.hip): x[o] += sum_i w[o][i] *
// attn[i] (or x[o] = ... with overwrite), w fp32 or f16 [dim][in] (in % 8 ==
// 0), or Q8_0 / Q4_0 blocks [dim][in/32] with in % 64 == 32 (the even block
// counts run launch_matvec_q).
struct OprojCall {
  const void* w;
  const float* attn;
  float* x;
  int dim, in;
  bool f16, q8, q4;  // else fp32
  bool overwrite;
};
hipError_t launch_oproj(const OprojCall& c, hipStream_t st);
// Quantized matvecs (Q8_0 / Q4_0 weights, the activation quantized to Q8_0
// in each workgroup), optionally with rmsnorm(x, norm_w) in front. Plain:
// nseg matrices of rows[s] rows over the same activation, y[s] = W_s x (or
// y[s] += W_s x with acc); every segment but the last needs a multiple of
// matvec_rows_per_task() rows. Pair: w[0] gate and w[1] up of rows[0] rows,
// y[0] = silu(gate x) * (up x).
struct MatvecCall {
  const float* x;
  const float* norm_w;
  float eps;
  int in;
  bool q4;
  int nseg;
  const void* w[3];
  float* y[3];
  int rows[3];
  bool pair, acc;
};
hipError_t launch_matvec_q(const MatvecCall& c, hipStream_t st);
int matvec_rows_per_task();
// rmsnorm of one row (ops.cpp:7-17) and silu(g) * u in place (model.cpp:781-782)
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int dim,
                          hipStream_t st);
hipError_t launch_silu_mul(float* g, const float* u, int n, hipStream_t st);

}  // namespace dbi
