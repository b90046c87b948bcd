// Forward-pass call sites of the reference model, restricted to the KV-cache
// hot path: the attention half of Model::decode_layer (model.cpp:757-771) and
// of Model::decode_layer_chunk (model.cpp:933-981), the prefix cache
// (model.cpp:1023-1156) and speculative decoding's merge + rollback
// (speculative.cpp:10-23, 82). Weight projections, norms and the FFN are the
// engine's and stay outside (q/k/v come in already projected).
#ifndef DBINFER_AMD_HOST_LAYER_HPP
#define DBINFER_AMD_HOST_LAYER_HPP

#include <cstddef>
#include <cstdint>
#include <span>
#include <string>
#include <variant>
#include <vector>

#include "kv_cache.hpp"

namespace dbinfer_amd::model {

// The attention-shape slice of Config (model.hpp:21-34).
struct Config {
  std::size_t n_heads = 0;
  std::size_t n_kv_heads = 0;
  std::size_t head_dim = 0;
  float rope_theta = 0.0f;
};

// gguf::Error (gguf.hpp:69-73): message plus file and byte offset.
struct Error {
  std::string message;
  std::string file;
  std::size_t offset = 0;
};

// std::expected<T, Error> stand-in (<expected> is not in this toolchain).
template <typename T>
class Result {
 public:
  Result(T v) : v_(std::move(v)) {}  // NOLINT(google-explicit-constructor)
  Result(Error e) : v_(std::move(e)) {}  // NOLINT(google-explicit-constructor)
  explicit operator bool() const { return v_.index() == 0; }
  const T& operator*() const { return std::get<0>(v_); }
  const Error& error() const { return std::get<1>(v_); }

 private:
  std::variant<T, Error> v_;
};
struct Unit {};

// tensor::rope (ops.cpp:19-38): NeoX pairs (j, j + hd/2), angle pos *
// theta^(-2j/hd) in fp64, in place over [n_heads][seq][head_dim].
void rope(float* x, const std::int32_t* positions, float theta, std::size_t n_heads,
          std::size_t seq, std::size_t head_dim);

// The attention half of decode_layer (model.cpp:757-771): dense caches rope q
// and k at pos, append, then attend; a ring appends un-roped k and the device
// ropes q and every resident key (attend_ring, model.cpp:662-700). The append
// and the attention run as one fused launch (dbi_kv_decode). q and k are
// modified in place for dense caches like the reference's q_/k_. attn_out is
// [n_heads*head_dim]. Returns false on a device error.
bool decode_attention(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos,
                      float* q, float* k, const float* v, float* attn_out);

// The attention half of decode_layer_chunk (model.cpp:933-981): rope every
// row at pos0 + c, append all n rows, then causal attention of row c over
// [0, pos0 + c]. q [n][nh*hd], k, v [n][nkv*hd], attn_out [n][nh*hd].
bool chunk_attention(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos0,
                     std::size_t n, float* q, float* k, const float* v, float* attn_out);

// The optional q/k/v projection biases of LayerWeights (model.hpp:41-43).
struct AttnBias {
  const float* attn_q_bias = nullptr;
  const float* attn_k_bias = nullptr;
  const float* attn_v_bias = nullptr;
};

// decode_attention from the raw projections, with the bias adds and the rope
// on the device (dbi_kv_decode_qkv; model.cpp:747-771): q, k, v are not
// modified. Same cache state and output as adding the biases on the host
// and calling decode_attention.
bool decode_attention_qkv(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos,
                          const float* q, const float* k, const float* v, const AttnBias& bias,
                          float* attn_out);

// chunk_attention from the raw projections (dbi_kv_chunk_qkv;
// model.cpp:933-981): bias and rope every row on the device, append, attend.
bool chunk_attention_qkv(KVCache& kv, const Config& cfg, std::size_t layer, std::int32_t pos0,
                         std::size_t n, const float* q, const float* k, const float* v,
                         const AttnBias& bias, float* attn_out);

// The step after attention in decode_layer (model.cpp:773-774): x += W_o ·
// attn on the device (dbi_oproj_residual_async, on the cache handle's
// stream). w_dev is W_o [dim][in] in device memory as fp32, f16 or Q8_0
// blocks (wtype DBI_W_F32 / DBI_W_F16 / DBI_W_Q8_0); attn_dev [in] and x_dev
// [dim] are device memory, x_dev updated in place. Returns false on an
// argument or device error (kv.error() has the message).
bool output_projection(KVCache& kv, std::uint32_t wtype, const void* w_dev,
                       const float* attn_dev, float* x_dev, std::size_t dim, std::size_t in);

// Model::save_kv_prefix / load_kv_prefix (model.hpp:292-299).
Result<Unit> save_kv_prefix(const KVCache& kv, const std::string& path,
                            std::span<const std::int32_t> prefix_tokens);
Result<std::size_t> load_kv_prefix(KVCache& kv, const std::string& path,
                                   std::span<const std::int32_t> prefix_tokens);

// speculative.cpp:10-23: accept the longest matching draft prefix plus one
// target token; returns the accepted count.
std::size_t speculative_merge(std::span<const std::int32_t> draft,
                              std::span<const std::int32_t> target,
                              std::vector<std::int32_t>& out);

// One verify round's cache side (speculative.cpp:64-82): the k+1 rows at pos
// were appended and attended by chunk_attention; after the merge the cache
// keeps pos + accepted + 1 positions. Returns the new pos.
std::int32_t speculative_commit(KVCache& kv, std::int32_t pos, std::size_t accepted);

// A verify round's token side plus its commit, with the argmax of the
// target's k+1 logit rows and the merge on the device (dbi_kv_verify_commit;
// speculative.cpp:69-82 with sample::argmax): logits_dev is device memory
// [draft.size()+1][vocab] and never leaves it. merged is cleared, then
// receives what speculative_merge emits (the accepted draft prefix, then the
// correction or the bonus token); the cache keeps pos + accepted + 1
// positions. Returns the accepted count.
Result<std::size_t> speculative_verify(KVCache& kv, std::int32_t pos, std::size_t vocab,
                                       const float* logits_dev,
                                       std::span<const std::int32_t> draft,
                                       std::vector<std::int32_t>& merged);

}  // namespace dbinfer_amd::model

#endif  // DBINFER_AMD_HOST_LAYER_HPP
