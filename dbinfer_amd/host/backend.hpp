// C++ host mirror of the reference engine's offload seam, the decode half of
// backend::Backend (src/backend/backend.hpp:12-157): the same WeightType,
// QWeight and LayerQ, and setup_offload / decode_token / decode_token_full
// with the reference's argument meanings, backed by libdbi_kv.so's host-row
// offload calls (dbi_offload_setup_host, dbi_decode_token,
// dbi_decode_token_full). Model::forward's offload branch (model.cpp:887-907)
// drives it unchanged.
//
// Differences the device imposes, all additive:
//  - the bound KV is the device cache of the KVCache this backend is built
//    on, so setup_offload's k_base / v_base / capacity / pos_stride (the
//    reference wraps its host arrays no-copy) are checked against it and not
//    wrapped; the cache may be dense fp32 (the reference's only offload
//    layout, main.cpp:241-244), dense int8 or a ring;
//  - fp32 weights are served as well (WeightType::F32, not in the
//    reference's enum);
//  - Backend's Metal-kernel methods (mul_mat_f16, the batched matmuls, the
//    per-op kernels) are not mirrored: their work is inside decode_token.
#ifndef DBINFER_AMD_HOST_BACKEND_HPP
#define DBINFER_AMD_HOST_BACKEND_HPP

#include <cstddef>
#include <cstdint>
#include <span>
#include <string>
#include <vector>

#include "kv_cache.hpp"
#include "layer.hpp"

namespace dbinfer_amd::backend {

// backend.hpp:17 (F32 added: the device serves it)
enum class WeightType : std::uint8_t { F16, Q8_0, Q4_0, F32 };

// backend.hpp:19-24: non-owning view of one packed weight matrix (host
// memory, e.g. the model mmap) and its dtype
struct QWeight {
  const std::byte* data = nullptr;
  WeightType type = WeightType::F16;
};

// backend.hpp:26-47: one block's weights and hyperparameters (host memory)
struct LayerQ {
  const float* attn_norm = nullptr;
  const float* ffn_norm = nullptr;
  QWeight wq{};
  QWeight wk{};
  QWeight wv{};
  QWeight wo{};
  QWeight wgate{};
  QWeight wup{};
  QWeight wdown{};
  const float* bq = nullptr;
  const float* bk = nullptr;
  const float* bv = nullptr;
  std::size_t dim = 0;
  std::size_t ff = 0;
  std::size_t n_heads = 0;
  std::size_t n_kv_heads = 0;
  std::size_t head_dim = 0;
  float rms_eps = 0.0f;
  float rope_theta = 0.0f;
};

using model::Error;
using model::Result;
using model::Unit;

class HipBackend {
 public:
  // kv: the device cache decode_token reads and appends to (the bound KV)
  explicit HipBackend(model::KVCache& kv) : kv_(kv) {}

  // backend.hpp:133-143: copies each offloaded block's weights to the device
  // once (layers cover the first layers.size() blocks); output_norm and
  // lm_head feed decode_token_full (lm_head.data null: no tail). Must be
  // called before decode_token and again if the model or cache changes.
  Result<Unit> setup_offload(std::span<const LayerQ> layers, float* k_base, float* v_base,
                             std::size_t capacity, std::size_t pos_stride,
                             const float* output_norm, QWeight lm_head,
                             std::size_t vocab_size);

  // backend.hpp:145-149: every prepared block of one token; x is the
  // residual stream [dim], updated in place; writes the bound KV at pos.
  Result<Unit> decode_token(float* x, std::int32_t pos);

  // backend.hpp:151-157: every prepared block, the final rmsnorm and the
  // lm_head; x is the input row [dim]; the returned pointer views the logits
  // [vocab_size], valid until the next call.
  Result<const float*> decode_token_full(const float* x, std::int32_t pos);

 private:
  model::KVCache& kv_;
  std::vector<float> logits_;
};

}  // namespace dbinfer_amd::backend

#endif  // DBINFER_AMD_HOST_BACKEND_HPP
