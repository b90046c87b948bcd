// KVCache over the C-ABI (see kv_cache.hpp).
#include "kv_cache.hpp"

#include <utility>

namespace dbinfer_amd::model {

KVCache::KVCache(std::size_t n_layers, std::size_t max_seq, std::size_t n_kv_heads,
                 std::size_t head_dim, KvPolicy policy, float rope_theta)
    : policy_(policy),
      n_layers_(n_layers),
      n_kv_heads_(n_kv_heads),
      head_dim_(head_dim),
      rope_theta_(rope_theta) {
  dbi_kv_config cfg{};
  cfg.n_layers = static_cast<std::uint32_t>(n_layers);
  cfg.max_seq = static_cast<std::uint32_t>(max_seq);
  cfg.n_kv_heads = static_cast<std::uint32_t>(n_kv_heads);
  cfg.head_dim = static_cast<std::uint32_t>(head_dim);
  cfg.n_sink = static_cast<std::uint32_t>(policy.n_sink);
  cfg.window = static_cast<std::uint32_t>(policy.window);
  cfg.dtype = policy.dtype == KvDtype::Int8 ? DBI_KV_INT8 : DBI_KV_F32;
  cfg.rope_theta = rope_theta;
  check(dbi_kv_create(&cfg, &h_));
}

KVCache::~KVCache() { dbi_kv_destroy(h_); }

KVCache::KVCache(KVCache&& o) noexcept
    : h_(std::exchange(o.h_, nullptr)),
      policy_(o.policy_),
      n_layers_(o.n_layers_),
      n_kv_heads_(o.n_kv_heads_),
      head_dim_(o.head_dim_),
      rope_theta_(o.rope_theta_),
      error_(std::move(o.error_)) {}

KVCache& KVCache::operator=(KVCache&& o) noexcept {
  if (this != &o) {
    dbi_kv_destroy(h_);
    h_ = std::exchange(o.h_, nullptr);
    policy_ = o.policy_;
    n_layers_ = o.n_layers_;
    n_kv_heads_ = o.n_kv_heads_;
    head_dim_ = o.head_dim_;
    rope_theta_ = o.rope_theta_;
    error_ = std::move(o.error_);
  }
  return *this;
}

bool KVCache::check(dbi_status st) const {
  if (st == DBI_OK) return true;
  if (error_.empty()) error_ = dbi_last_error();
  return false;
}

void KVCache::append(std::size_t layer, std::size_t pos, const float* k, const float* v) {
  check(dbi_kv_append(h_, static_cast<std::uint32_t>(layer), static_cast<std::uint32_t>(pos), k,
                      v));
}

void KVCache::append_n(std::size_t layer, std::size_t pos0, std::size_t n, const float* k,
                       const float* v) {
  check(dbi_kv_append_n(h_, static_cast<std::uint32_t>(layer), static_cast<std::uint32_t>(pos0),
                        static_cast<std::uint32_t>(n), k, v));
}

std::size_t KVCache::slot_for(std::size_t pos) const {
  std::uint32_t slot = 0;
  check(dbi_kv_slot_for(h_, static_cast<std::uint32_t>(pos), &slot));
  return slot;
}

std::size_t KVCache::residents(Resident* out) const {
  const std::size_t cap = capacity();
  std::vector<std::uint32_t> slot(cap);
  std::vector<std::int32_t> rp(cap);
  std::uint32_t count = 0;
  if (!check(dbi_kv_residents(h_, slot.data(), rp.data(), static_cast<std::uint32_t>(cap),
                              &count)))
    return 0;
  for (std::uint32_t i = 0; i < count; ++i) out[i] = {slot[i], rp[i]};
  return count;
}

std::size_t KVCache::capacity() const { return dbi_kv_capacity(h_); }
std::size_t KVCache::n_seen() const { return dbi_kv_n_seen(h_); }

void KVCache::truncate(std::size_t n_seen) {
  check(dbi_kv_truncate(h_, static_cast<std::uint32_t>(n_seen)));
}

std::vector<float> KVCache::export_f32(std::uint32_t what, std::size_t layer) const {
  const std::size_t bytes = dbi_kv_export_bytes(h_, what);
  std::vector<float> out(bytes / sizeof(float));
  if (bytes == 0 || !check(dbi_kv_export(h_, what, static_cast<std::uint32_t>(layer), out.data(),
                                         bytes)))
    out.clear();
  return out;
}

std::vector<std::int8_t> KVCache::export_i8(std::uint32_t what, std::size_t layer) const {
  const std::size_t bytes = dbi_kv_export_bytes(h_, what);
  std::vector<std::int8_t> out(bytes);
  if (bytes == 0 || !check(dbi_kv_export(h_, what, static_cast<std::uint32_t>(layer), out.data(),
                                         bytes)))
    out.clear();
  return out;
}

}  // namespace dbinfer_amd::model
