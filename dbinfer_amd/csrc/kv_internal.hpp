// Internal state of a dbi_kv handle and the kernel launchers shared by the
// translation units of libdbi_kv.so.
//
// Device storage is head-major, so the keys of one kv head are one contiguous
// stream for decode attention (the reference stores [slot][kv_head][hd],
// model.hpp:108-214; dbi_kv_export converts back):
//   fp32 (dense, ring)  k, v          [L][nkv][cap][hd]   fp32
//   int8                k8, v8        [L][nkv][cap][hd]   int8
//                       v_scale       [L][nkv][cap][nb]   fp32
//   ring int8           k_scale       [L][nkv][cap][nb]   fp32 (per 32-block)
//   dense int8          k_scale       [L][nkv][ng][hd]    fp32 (per channel, per 32-token group)
//                       k_raw         [L][32][nkv*hd]     fp32 (reference order)
//                       k_sink,v_sink [L][nkv][ns][hd]    fp32
//   ring                rope_cs       [cap][hd/2]         float2 (cos, sin)
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
  bool int8, ring;
};

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
};

// Split-K workspace: partial (o, m, l) of every split of one attention call.
struct Workspace {
  float* part = nullptr;
  size_t part_floats = 0;
  float* staging = nullptr;  // device staging for host-pointer calls
  size_t staging_floats = 0;
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
};

// Launchers (return a hipError_t of the launch).
hipError_t launch_append(const KvGeom& g, const KvStore& s, int layer, int pos0, int n,
                         const float* k, const float* v, hipStream_t st);
// Returns hipErrorNotSupported for shapes without a kernel instance.
hipError_t launch_attention(const KvGeom& g, const KvStore& s, Workspace& ws,
                            const AttnCall& c, hipStream_t st);
// Number of partial floats one call needs (for workspace sizing).
size_t attention_workspace_need(const KvGeom& g, const AttnCall& c);
bool attention_supported(const KvGeom& g, int n_heads);

// Prefix pack/unpack between [L][len][nkv][hd] and the head-major store.
hipError_t launch_prefix_pack(const KvGeom& g, const float* src_store, float* dst, int len,
                              hipStream_t st);
hipError_t launch_prefix_unpack(const KvGeom& g, const float* src, float* dst_store, int len,
                                hipStream_t st);

}  // namespace dbi
