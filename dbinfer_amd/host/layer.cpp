// Reference call sites over the device KV cache (see layer.hpp).
#include "layer.hpp"

#include <cmath>

namespace dbinfer_amd::model {

void rope(float* x, const std::int32_t* positions, float theta, std::size_t n_heads,
          std::size_t seq, std::size_t head_dim) {
  const std::size_t half = head_dim / 2;
  for (std::size_t h = 0; h < n_heads; ++h) {
    for (std::size_t s = 0; s < seq; ++s) {
      float* row = x + (h * seq + s) * head_dim;
      const double p = static_cast<double>(positions[s]);
      for (std::size_t j = 0; j < half; ++j) {
        const double freq = std::pow(static_cast<double>(theta),
                                     -2.0 * static_cast<double>(j) / static_cast<double>(head_dim));
        const double angle = p * freq;
        const double c = std::cos(angle), sn = std::sin(angle);
        const float a = row[j], b = row[j + half];
        row[j] = static_cast<float>(a * c - b * sn);
        row[j + half] = static_cast<float>(b * c + a * sn);
      }
    }
  }
}

namespace {

float attn_scale(const Config& cfg) {
  return 1.0f / std::sqrt(static_cast<float>(cfg.head_dim));  // model.cpp:757
}

}  // namespace

bool decode_attention(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos,
                      float* q, float* k, const float* v, float* attn_out) {
  const auto l = static_cast<std::uint32_t>(layer);
  const auto p = static_cast<std::uint32_t>(pos);
  if (!kv.ring()) {
    rope(q, &pos, cfg.rope_theta, cfg.n_heads, 1, cfg.head_dim);
    rope(k, &pos, cfg.rope_theta, cfg.n_kv_heads, 1, cfg.head_dim);
  }
  if (!kv.ok()) return false;
  // kv.append + attend in one launch (dbi_kv_decode)
  return kv.check(dbi_kv_decode(kv.handle(), l, p, k, v, static_cast<std::uint32_t>(cfg.n_heads),
                                attn_scale(cfg), q, attn_out));
}

bool chunk_attention(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos0,
                     std::size_t n, float* q, float* k, const float* v, float* attn_out) {
  const std::size_t qrow = cfg.n_heads * cfg.head_dim, krow = cfg.n_kv_heads * cfg.head_dim;
  for (std::size_t c = 0; c < n; ++c) {
    const std::int32_t p = pos0 + static_cast<std::int32_t>(c);
    rope(q + c * qrow, &p, cfg.rope_theta, cfg.n_heads, 1, cfg.head_dim);
    rope(k + c * krow, &p, cfg.rope_theta, cfg.n_kv_heads, 1, cfg.head_dim);
  }
  kv.append_n(layer, static_cast<std::size_t>(pos0), n, k, v);
  if (!kv.ok()) return false;
  return kv.check(dbi_attn_chunk(kv.handle(), static_cast<std::uint32_t>(layer),
                                 static_cast<std::uint32_t>(pos0), static_cast<std::uint32_t>(n),
                                 static_cast<std::uint32_t>(cfg.n_heads), attn_scale(cfg), q,
                                 attn_out));
}

bool decode_attention_qkv(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos,
                          const float* q, const float* k, const float* v, const AttnBias& bias,
                          float* attn_out) {
  if (!kv.ok()) return false;
  return kv.check(dbi_kv_decode_qkv(kv.handle(), static_cast<std::uint32_t>(layer),
                                    static_cast<std::uint32_t>(pos),
                                    static_cast<std::uint32_t>(cfg.n_heads), attn_scale(cfg), q,
                                    k, v, bias.attn_q_bias, bias.attn_k_bias, bias.attn_v_bias,
                                    attn_out));
}

bool chunk_attention_qkv(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos0,
                         std::size_t n, const float* q, const float* k, const float* v,
                         const AttnBias& bias, float* attn_out) {
  if (!kv.ok()) return false;
  return kv.check(dbi_kv_chunk_qkv(kv.handle(), static_cast<std::uint32_t>(layer),
                                   static_cast<std::uint32_t>(pos0), static_cast<std::uint32_t>(n),
                                   static_cast<std::uint32_t>(cfg.n_heads), attn_scale(cfg), q, k,
                                   v, bias.attn_q_bias, bias.attn_k_bias, bias.attn_v_bias,
                                   attn_out));
}

Result<Unit> save_kv_prefix(const KVCache& kv, const std::string& path,
                            std::span<const std::int32_t> prefix_tokens) {
  const dbi_status st = dbi_kv_prefix_save(kv.handle(), path.c_str(), prefix_tokens.data(),
                                           static_cast<std::uint32_t>(prefix_tokens.size()));
  if (st != DBI_OK) return Error{dbi_last_error(), path, 0};
  return Unit{};
}

Result<std::size_t> load_kv_prefix(KVCache& kv, const std::string& path,
                                   std::span<const std::int32_t> prefix_tokens) {
  std::uint32_t len = 0;
  const dbi_status st = dbi_kv_prefix_load(kv.handle(), path.c_str(), prefix_tokens.data(),
                                           static_cast<std::uint32_t>(prefix_tokens.size()), &len);
  if (st != DBI_OK) return Error{dbi_last_error(), path, 0};
  return static_cast<std::size_t>(len);
}

std::size_t speculative_merge(std::span<const std::int32_t> draft,
                              std::span<const std::int32_t> target,
                              std::vector<std::int32_t>& out) {
  std::size_t j = 0;
  while (j < draft.size() && draft[j] == target[j]) out.push_back(draft[j++]);
  out.push_back(target[j]);  // correction at the first mismatch, or the bonus token
  return j;
}

std::int32_t speculative_commit(KVCache& kv, std::int32_t pos, std::size_t accepted) {
  const std::int32_t next = pos + static_cast<std::int32_t>(accepted) + 1;
  kv.truncate(static_cast<std::size_t>(next));
  return next;
}

bool output_projection(KVCache& kv, std::uint32_t wtype, const void* w_dev,
                       const float* attn_dev, float* x_dev, std::size_t dim, std::size_t in) {
  return kv.check(dbi_oproj_residual_async(kv.handle(), wtype, w_dev, attn_dev, x_dev,
                                           static_cast<std::uint32_t>(dim),
                                           static_cast<std::uint32_t>(in)));
}

Result<std::size_t> speculative_verify(KVCache& kv, std::int32_t pos, std::size_t vocab,
                                       const float* logits_dev,
                                       std::span<const std::int32_t> draft,
                                       std::vector<std::int32_t>& merged) {
  merged.assign(draft.size() + 1, 0);
  std::uint32_t accepted = 0;
  const dbi_status st = dbi_kv_verify_commit(
      kv.handle(), static_cast<std::uint32_t>(pos), static_cast<std::uint32_t>(draft.size()),
      static_cast<std::uint32_t>(vocab), logits_dev, draft.data(), merged.data(), &accepted);
  if (st != DBI_OK) {
    merged.clear();
    return Error{dbi_last_error(), "", 0};
  }
  merged.resize(accepted + 1);
  return static_cast<std::size_t>(accepted);
}

}  // namespace dbinfer_amd::model
