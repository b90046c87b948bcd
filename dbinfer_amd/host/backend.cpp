#include "backend.hpp"

#include <cmath>

#include "dbi_kv.h"

namespace dbinfer_amd::backend {

namespace {

Error err(std::string msg) { return Error{std::move(msg), "", 0}; }

Error last_error(const char* what) {
  const char* m = dbi_last_error();
  return err(std::string(what) + ": " + (m ? m : "device error"));
}

std::uint32_t dbi_type(WeightType t) {
  switch (t) {
    case WeightType::F16: return DBI_W_F16;
    case WeightType::Q8_0: return DBI_W_Q8_0;
    case WeightType::Q4_0: return DBI_W_Q4_0;
    case WeightType::F32: return DBI_W_F32;
  }
  return 0xFFFFFFFFu;  // rejected by the setup as unsupported
}

dbi_weight weight(const QWeight& q) { return dbi_weight{q.data, dbi_type(q.type)}; }

}  // namespace

Result<Unit> HipBackend::setup_offload(std::span<const LayerQ> layers, float* k_base,
                                       float* v_base, std::size_t capacity,
                                       std::size_t pos_stride, const float* output_norm,
                                       QWeight lm_head, std::size_t vocab_size) {
  (void)k_base;
  (void)v_base;  // the device cache is the bound KV
  if (layers.empty()) return err("setup_offload: no layers");
  if (layers.size() > kv_.n_layers()) return err("setup_offload: more layers than the cache");
  if (pos_stride != 0 && pos_stride != kv_.pos_stride())
    return err("setup_offload: pos_stride does not match the cache");
  if (capacity != 0 && capacity > kv_.capacity())
    return err("setup_offload: capacity exceeds the cache's");
  const LayerQ& L0 = layers.front();
  std::vector<dbi_layer_weights> lw(layers.size());
  for (std::size_t l = 0; l < layers.size(); ++l) {
    const LayerQ& L = layers[l];
    // one shape for the whole model (the C-ABI binds one config)
    if (L.dim != L0.dim || L.ff != L0.ff || L.n_heads != L0.n_heads ||
        L.n_kv_heads != L0.n_kv_heads || L.head_dim != L0.head_dim ||
        L.rms_eps != L0.rms_eps || L.rope_theta != L0.rope_theta)
      return err("setup_offload: block " + std::to_string(l) + " differs in shape");
    lw[l] = dbi_layer_weights{L.attn_norm, L.ffn_norm, weight(L.wq), weight(L.wk),
                              weight(L.wv), weight(L.wo), weight(L.wgate), weight(L.wup),
                              weight(L.wdown), L.bq, L.bk, L.bv};
  }
  if (L0.n_kv_heads != kv_.n_kv_heads() || L0.head_dim != kv_.head_dim())
    return err("setup_offload: kv heads / head_dim do not match the cache");
  if (!kv_.ring() && L0.rope_theta != kv_.rope_theta())
    return err("setup_offload: rope_theta does not match the cache's");
  const dbi_offload_config cfg{static_cast<std::uint32_t>(L0.dim),
                               static_cast<std::uint32_t>(L0.ff),
                               static_cast<std::uint32_t>(L0.n_heads),
                               L0.rms_eps,
                               lm_head.data ? output_norm : nullptr,
                               weight(lm_head),
                               static_cast<std::uint32_t>(lm_head.data ? vocab_size : 0)};
  if (dbi_offload_setup_host(kv_.handle(), &cfg, lw.data(),
                             static_cast<std::uint32_t>(lw.size())) != DBI_OK)
    return last_error("setup_offload");
  logits_.assign(lm_head.data ? vocab_size : 0, 0.0f);
  return Unit{};
}

Result<Unit> HipBackend::decode_token(float* x, std::int32_t pos) {
  if (pos < 0) return err("decode_token: negative position");
  if (dbi_decode_token(kv_.handle(), x, static_cast<std::uint32_t>(pos)) != DBI_OK)
    return last_error("decode_token");
  return Unit{};
}

Result<const float*> HipBackend::decode_token_full(const float* x, std::int32_t pos) {
  if (pos < 0) return err("decode_token_full: negative position");
  if (logits_.empty()) return err("decode_token_full: no lm_head was set up");
  if (dbi_decode_token_full(kv_.handle(), x, static_cast<std::uint32_t>(pos),
                            logits_.data()) != DBI_OK)
    return last_error("decode_token_full");
  return static_cast<const float*>(logits_.data());
}

}  // namespace dbinfer_amd::backend
