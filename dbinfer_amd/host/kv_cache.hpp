// C++ host mirror of the reference engine's KV-cache interface, backed by
// libdbi_kv.so (include/dbi_kv.h). Same names, argument meanings and layouts
// as dbinfer::model::KVCache (src/model/model.hpp:78-214), so the engine's
// call sites (decode_layer, decode_layer_chunk, speculative decoding, prefix
// cache) drive the MI355X cache unchanged.
//
// Differences the device imposes, all additive:
//  - storage lives in HBM, so the raw-pointer accessors (key(), key_i8(), ...)
//    become export_*() copies in the reference layout;
//  - truncate(n) names the rollback the reference performs implicitly
//    (speculative.cpp:82); reset()/mark_position() are kept;
//  - a device error is sticky (ok() / error()), so a caller can fall back to
//    its CPU path the way the reference does on a backend error
//    (model.cpp:887-907); the reference's KVCache aborts only on OOM.
#ifndef DBINFER_AMD_HOST_KV_CACHE_HPP
#define DBINFER_AMD_HOST_KV_CACHE_HPP

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "dbi_kv.h"

namespace dbinfer_amd::model {

enum class KvDtype { F32, Int8 };                 // model.hpp:78
inline constexpr std::size_t kKvBlock = 32;       // model.hpp:81
inline constexpr std::size_t kKvKGroup = 32;      // model.hpp:87

struct KvPolicy {                                 // model.hpp:96-100
  std::size_t n_sink = 0;
  std::size_t window = 0;
  KvDtype dtype = KvDtype::F32;
};

class KVCache {
 public:
  struct Resident {                               // model.hpp:111-114
    std::size_t slot;
    std::int32_t rope_pos;
  };

  // model.hpp:119-120. rope_theta is what the ring path ropes with
  // (Config::rope_theta, used by attend_ring model.cpp:671, 696).
  KVCache(std::size_t n_layers, std::size_t max_seq, std::size_t n_kv_heads,
          std::size_t head_dim, KvPolicy policy = {}, float rope_theta = 10000.0f);
  ~KVCache();
  KVCache(const KVCache&) = delete;
  KVCache& operator=(const KVCache&) = delete;
  KVCache(KVCache&& o) noexcept;
  KVCache& operator=(KVCache&& o) noexcept;

  // model.hpp:122: one position of every kv head of a layer, host [nkv*hd].
  void append(std::size_t layer, std::size_t pos, const float* k, const float* v);
  // n positions at pos0.. in one transfer ([n][nkv*hd]); same final state as
  // n append() calls (the append loop of decode_layer_chunk, model.cpp:935-954).
  void append_n(std::size_t layer, std::size_t pos0, std::size_t n, const float* k,
                const float* v);

  std::size_t slot_for(std::size_t pos) const;          // model.hpp:171
  std::size_t residents(Resident* out) const;           // model.hpp:175

  std::size_t n_blocks() const { return (head_dim_ + kKvBlock - 1) / kKvBlock; }
  std::size_t n_sink_fp32() const { return int8() && !ring() ? policy_.n_sink : 0; }
  bool k_per_channel() const { return int8() && !ring(); }
  bool int8() const { return policy_.dtype == KvDtype::Int8; }
  bool ring() const { return policy_.window > 0; }
  bool dense_f32() const { return !int8() && !ring(); }
  std::size_t n_layers() const { return n_layers_; }
  std::size_t prefix_elems(std::size_t prefix_len) const {
    return n_layers_ * prefix_len * pos_stride();
  }
  std::size_t capacity() const;
  std::size_t n_seen() const;
  const KvPolicy& policy() const { return policy_; }
  void reset() { truncate(0); }                              // model.hpp:164
  void mark_position(std::size_t pos) { truncate(pos + 1); }  // model.hpp:182-184
  void truncate(std::size_t n_seen);
  std::size_t n_kv_heads() const { return n_kv_heads_; }
  std::size_t head_dim() const { return head_dim_; }
  std::size_t pos_stride() const { return n_kv_heads_ * head_dim_; }
  float rope_theta() const { return rope_theta_; }

  // Reference-layout copies of one layer (model.cpp:420-455 accessors):
  // keys/values [capacity][nkv][hd]; scales as the reference stores them.
  std::vector<float> export_f32(std::uint32_t what, std::size_t layer) const;
  std::vector<std::int8_t> export_i8(std::uint32_t what, std::size_t layer) const;

  bool ok() const { return error_.empty(); }
  const std::string& error() const { return error_; }
  dbi_kv* handle() const { return h_; }
  // records a failed C-ABI call (sticky); returns false when st != DBI_OK
  bool check(dbi_status st) const;

 private:
  dbi_kv* h_ = nullptr;
  KvPolicy policy_;
  std::size_t n_layers_ = 0, n_kv_heads_ = 0, head_dim_ = 0;
  float rope_theta_ = 10000.0f;
  mutable std::string error_;
};

}  // namespace dbinfer_amd::model

#endif  // DBINFER_AMD_HOST_KV_CACHE_HPP
