/*
 * dbi_kv.h -- C-ABI of the MI355X KV-cache + attention hot path.
 *
 * This is the drop-in boundary for the reference engine's KV cache
 * (src/model/model.hpp:102-214, src/model/model.cpp:258-474), its three
 * single-query attention kernels and the causal chunk attention
 * (model.cpp:567-728, 956-981), its prefix cache I/O
 * (model.cpp:1023-1156), the token side of a speculative verify round
 * (speculative.cpp:64-82), and the output projection + residual add that
 * follows attention (model.cpp:773-774). Plain C types only; no exceptions
 * cross it.
 *
 * Conventions
 *  - Every entry point returns a dbi_status. On failure the handle's state is
 *    unchanged and dbi_last_error() (thread-local) holds a message, so the
 *    caller can fall back to its CPU path (the reference's own pattern on a
 *    backend error, model.cpp:887-907).
 *  - Plain entry points take HOST pointers, block until the results are in the
 *    caller's buffers, and are what a CPU call site swaps in. The *_async
 *    variants take DEVICE pointers and enqueue on the handle's HIP stream.
 *  - Element layouts are the reference's: k, v per position [n_kv_heads][head_dim]
 *    (model.hpp:117-122), q and out [n_heads][head_dim] (model.cpp:574-600).
 *  - One handle per host thread; calls on a handle are ordered on its stream
 *    (the reference KVCache is not thread-safe either).
 */
#ifndef DBI_KV_H
#define DBI_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DBI_KV_ABI_VERSION 1

typedef struct dbi_kv dbi_kv;
typedef int32_t dbi_status;

enum {
  DBI_OK = 0,
  DBI_ERR_INVALID = 1,     /* bad argument: null pointer, layer/pos out of range */
  DBI_ERR_UNSUPPORTED = 2, /* layout or shape this entry point does not serve */
  DBI_ERR_NOMEM = 3,       /* device or host allocation failed */
  DBI_ERR_DEVICE = 4,      /* HIP runtime error */
  DBI_ERR_IO = 5,          /* prefix file open/read/write failed */
  DBI_ERR_FORMAT = 6       /* prefix file failed validation */
};

/* KvDtype (model.hpp:78) */
enum { DBI_KV_F32 = 0, DBI_KV_INT8 = 1 };

/* KvPolicy (model.hpp:96-100) plus the cache geometry the KVCache constructor
 * takes (model.hpp:119-120) and the rope base the ring path needs
 * (Config::rope_theta, model.hpp:30). */
typedef struct dbi_kv_config {
  uint32_t n_layers;
  uint32_t max_seq;    /* dense capacity; ignored when window > 0 */
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t n_sink;     /* ring: pinned sinks; dense int8: fp32 sink tokens */
  uint32_t window;     /* 0 = dense full-context cache, > 0 = ring of n_sink + window */
  uint32_t dtype;      /* DBI_KV_F32 or DBI_KV_INT8 */
  float rope_theta;    /* rope base: a ring's cache-relative re-rope, and the
                          q/k/v producer's rope (dbi_kv_decode_qkv) */
} dbi_kv_config;

/* Message of the last failed call on this thread ("" if none). */
const char* dbi_last_error(void);

/* KVCache::KVCache (model.hpp:119-120, model.cpp:258-297) and
 * Model::configure_kv (model.hpp:284). Allocates and zero-fills all device
 * storage on the current HIP device. One kv head's K (or V) array, capacity
 * rounded up to 64 x head_dim x element size, must stay below 2 GiB (e.g.
 * up to ~4M positions at head_dim 128 fp32). */
dbi_status dbi_kv_create(const dbi_kv_config* cfg, dbi_kv** out);
void dbi_kv_destroy(dbi_kv* kv);
dbi_status dbi_kv_get_config(const dbi_kv* kv, dbi_kv_config* out);

/* Use this HIP stream (a hipStream_t) for every later call; NULL = the
 * handle's own stream. */
dbi_status dbi_kv_set_stream(dbi_kv* kv, void* hip_stream);
/* Block until all work enqueued on the handle's stream has finished. */
dbi_status dbi_kv_sync(dbi_kv* kv);

/* KVCache::append (model.hpp:122, model.cpp:357-404): one position of every
 * kv head of one layer; k, v are host [n_kv_heads*head_dim]. Int8 layouts
 * quantize on append (dense: per-channel K over 32-token groups + per-block V
 * + fp32 sinks; ring: per-block K and V). Sets n_seen = pos + 1. */
dbi_status dbi_kv_append(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k,
                         const float* v);
/* n sequential appends at pos0..pos0+n-1 (the append loop of
 * decode_layer_chunk, model.cpp:935-954); k, v host [n][n_kv_heads*head_dim].
 * The final state equals n calls of dbi_kv_append. */
dbi_status dbi_kv_append_n(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                           const float* k, const float* v);
/* As dbi_kv_append_n with device pointers, enqueued on the handle's stream. */
dbi_status dbi_kv_append_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                               const float* k_dev, const float* v_dev);

/* Sets n_seen. reset() (model.hpp:164) is truncate(0), mark_position(p)
 * (model.hpp:182-184) is truncate(p+1), and a speculative rollback
 * (speculative.cpp:82) is truncate(pos + accepted + 1). Slots past n_seen are
 * not scrubbed: the next append overwrites them, exactly as in the reference. */
dbi_status dbi_kv_truncate(dbi_kv* kv, uint32_t n_seen);
uint32_t dbi_kv_n_seen(const dbi_kv* kv);   /* KVCache::n_seen (model.hpp:161) */
uint32_t dbi_kv_capacity(const dbi_kv* kv); /* KVCache::capacity (model.hpp:160) */

/* KVCache::slot_for (model.hpp:171, model.cpp:321-324); ring only. */
dbi_status dbi_kv_slot_for(const dbi_kv* kv, uint32_t pos, uint32_t* slot);
/* KVCache::residents (model.hpp:175, model.cpp:406-418); ring only. Writes up
 * to cap entries (sinks first, then the window oldest to newest) and the
 * count. */
dbi_status dbi_kv_residents(const dbi_kv* kv, uint32_t* slot, int32_t* rope_pos, uint32_t cap,
                            uint32_t* count);

/* Single-query GQA attention of one layer at position pos, for the cache's
 * layout: Model::attend_dense_f32 (model.cpp:567-603), attend_dense_int8
 * (model.cpp:605-660) or attend_ring (model.cpp:662-728), and the dense-only
 * Backend::attention seam (backend.hpp:126-131). q, out host [n_heads*head_dim];
 * scale is the caller's 1/sqrt(head_dim) (model.cpp:757). Dense layouts read
 * positions [0, pos] with q already roped (model.cpp:759-763). A ring reads
 * the residents of n_seen = pos + 1 (append pos first, as model.cpp:668 does),
 * and q is un-roped: it is roped at n_res - 1 and every resident key at its
 * cache-relative position (model.cpp:669-700). */
dbi_status dbi_attn_decode(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                           float scale, const float* q, float* out);
dbi_status dbi_attn_decode_async(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                                 float scale, const float* q_dev, float* out_dev);

/* Key splits of an attention call: how many partial records per query row
 * and kv head a decode (rows = 1, at pos0) or chunk call (rows rows from
 * pos0) over the current kernels writes and merges; 1 means the call writes
 * its output directly. A query for tests and tuning, with no counterpart in
 * the reference (its attention is one loop per head, model.cpp:575-600). */
dbi_status dbi_attn_splits(const dbi_kv* kv, uint32_t pos0, uint32_t rows, uint32_t n_heads,
                           uint32_t* n_split);

/* One decode step of a layer, fused: KVCache::append of position pos then
 * the single-query attention at pos, exactly as dbi_kv_append followed by
 * dbi_attn_decode (the attention half of Model::decode_layer,
 * model.cpp:759-771). k, v host [n_kv_heads*head_dim] (for dense layouts
 * already roped, as the reference's k_), q, out host [n_heads*head_dim]. One
 * kernel launch writes the row and attends; sets n_seen = pos + 1. */
dbi_status dbi_kv_decode(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k,
                         const float* v, uint32_t n_heads, float scale, const float* q,
                         float* out);
dbi_status dbi_kv_decode_async(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k_dev,
                               const float* v_dev, uint32_t n_heads, float scale,
                               const float* q_dev, float* out_dev);

/* dbi_kv_decode_async for callers that cannot allocate: no counterpart in
 * the reference, for code under HIP graph capture, tight serving loops and
 * harnesses that forbid hipMalloc. Same arguments, kernels and results; it
 * calls no allocating routine, ever. Its split records and arrival counters
 * live in a static per-GPU scratch array (2 MiB of records, 64 KiB of
 * counters), set up when the first handle on that GPU is created. Every
 * decode plan fits (at most 256 split records of at most 8 heads x 130
 * floats); a call whose plan needed more would fail with DBI_ERR_UNSUPPORTED
 * before any launch. Every call on one GPU shares that array: calls that
 * overlap on one GPU (other handles, other streams) race. */
dbi_status dbi_kv_decode_noalloc_async(dbi_kv* kv, uint32_t layer, uint32_t pos,
                                       const float* k_dev, const float* v_dev, uint32_t n_heads,
                                       float scale, const float* q_dev, float* out_dev);

/* Causal chunk attention of decode_layer_chunk (model.cpp:956-981): row c of
 * q [n][n_heads][head_dim] attends [0, pos0 + c] and writes row c of out.
 * Every row must have been appended first (model.cpp:933-954). Dense fp32
 * and dense int8 (rows attend with the int8 rule of model.cpp:605-660 over
 * the cache as it stands after all n appends); rings are not served. */
dbi_status dbi_attn_chunk(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                          uint32_t n_heads, float scale, const float* q, float* out);
dbi_status dbi_attn_chunk_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                                uint32_t n_heads, float scale, const float* q_dev,
                                float* out_dev);

/* The attention half of Model::decode_layer from the q/k/v projections
 * (model.cpp:747-771), on the device. Adds the biases (each may be null, as
 * the reference's optional attn_*_bias; model.cpp:747-755), ropes q and k at
 * pos on dense layouts (tensor::rope's NeoX pairs in fp64, ops.cpp:19-38;
 * a ring appends k un-roped and ropes inside attention, model.cpp:662-700),
 * then appends k/v at pos and attends, as dbi_kv_decode does. q, out
 * [n_heads*head_dim], k, v [n_kv_heads*head_dim], biases the same sizes; the
 * inputs are not modified. Appended rows are bit-identical to what the
 * reference appends after its host-side bias and rope. Needs
 * rope_theta > 0 for dense layouts; the first such call on a handle builds
 * its (cos, sin) table and must not be under graph capture. */
dbi_status dbi_kv_decode_qkv(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                             float scale, const float* q, const float* k, const float* v,
                             const float* q_bias, const float* k_bias, const float* v_bias,
                             float* out);
dbi_status dbi_kv_decode_qkv_async(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                                   float scale, const float* q_dev, const float* k_dev,
                                   const float* v_dev, const float* q_bias_dev,
                                   const float* k_bias_dev, const float* v_bias_dev,
                                   float* out_dev);

/* The attention half of Model::decode_layer_chunk from the projections
 * (model.cpp:933-981), on the device: bias and rope every row c at
 * pos0 + c (model.cpp:935-952), append all n rows (:953), then the causal
 * chunk attention of dbi_attn_chunk. q, out [n][n_heads*head_dim], k, v
 * [n][n_kv_heads*head_dim]; each bias (or null) is one row's worth and is
 * added to every row. Dense layouts only. */
dbi_status dbi_kv_chunk_qkv(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                            uint32_t n_heads, float scale, const float* q, const float* k,
                            const float* v, const float* q_bias, const float* k_bias,
                            const float* v_bias, float* out);
dbi_status dbi_kv_chunk_qkv_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                                  uint32_t n_heads, float scale, const float* q_dev,
                                  const float* k_dev, const float* v_dev,
                                  const float* q_bias_dev, const float* k_bias_dev,
                                  const float* v_bias_dev, float* out_dev);

/* Token side of one speculative verify round, on the device. Replaces the
 * host loop of speculative_generate (speculative.cpp:69-76): sample::argmax
 * of each of the k+1 chunk rows (sample.cpp:11-28), then speculative_merge of
 * the k draft proposals against them (speculative.cpp:10-23).
 * logits_dev: device [k+1][vocab] fp32, the target model's rows for the chunk
 * [last, draft...]; draft_dev: device [k] int32.
 * Writes verified_dev[0..k], the argmax of every row (the first maximum wins;
 * NaNs never win, and a NaN in slot 0 gives 0, as the reference's strict >
 * scan does), and *accepted_dev = j, the length of the accepted draft prefix.
 * The merged tokens are verified_dev[0..j] (the draft prefix equals them).
 * 1 <= k <= 64, 1 <= vocab <= 2^30. Ordered on the handle's stream; the
 * handle's small verify workspace is allocated on its first verify call, so
 * make one call before capturing a graph. Verify calls on one handle must not
 * overlap (they share an arrival counter). */
dbi_status dbi_spec_verify_async(dbi_kv* kv, uint32_t k, uint32_t vocab, const float* logits_dev,
                                 const int32_t* draft_dev, int32_t* verified_dev,
                                 int32_t* accepted_dev);

/* A verify round with the cache commit, blocking: dbi_spec_verify_async on a
 * device copy of the host draft[k], then the argmaxes and the count copied
 * back (4(k+2) bytes; the logits stay in HBM), then the cache truncated to
 * pos + accepted + 1. The round appended its k+1 rows at pos..pos+k (the
 * chunk of speculative.cpp:69); speculative.cpp:82 moves pos past the accepted
 * tokens and the correction, and the next round's rows overwrite the rest.
 * merged receives accepted + 1 tokens (room for k+1). Needs
 * pos + k + 1 <= n_seen. */
dbi_status dbi_kv_verify_commit(dbi_kv* kv, uint32_t pos, uint32_t k, uint32_t vocab,
                                const float* logits_dev, const int32_t* draft, int32_t* merged,
                                uint32_t* accepted);

/* Weight types of the matvecs (dbi_oproj_residual_async, the layer offload),
 * numbered as GgmlType. */
enum { DBI_W_F32 = 0, DBI_W_F16 = 1, DBI_W_Q4_0 = 2, DBI_W_Q8_0 = 8 };

/* The step after attention in Model::decode_layer (model.cpp:773-774):
 * matvec_quant(attn_output, attn, proj, dim, nh*hd) then x[i] += proj[i],
 * for fp32 weights (tensor::matvec, matmul.cpp:36-43), f16 weights
 * (tensor::matvec_f16, matmul.cpp:45-54), Q8_0 blocks (matvec_q8_0_scalar,
 * matmul.cpp:56-75) and Q4_0 blocks (matvec_q4_0_scalar, :77-99), the
 * quantized types after quantize_row_q8_0 of attn (dequant.cpp:80-97).
 * w_dev: device [dim][in] row-major (Q8_0: [dim][in/32] blocks of an f16
 * scale and 32 int8 codes, 34 bytes; Q4_0: of an f16 scale and 16 bytes of
 * nibbles, 18 bytes); attn_dev: device [in] (the attention row, in =
 * n_heads*head_dim); x_dev: device [dim], the residual stream, updated in
 * place. in must be a multiple of 8, at most 2^24 (Q8_0, Q4_0: a multiple of
 * 32, at most 32768); w_dev 16-byte aligned (Q8_0, Q4_0: 4), attn_dev
 * 16-byte aligned. Each row's terms
 * are summed in a tree, so proj agrees with the reference's sequential sum
 * to the rounding of a dot product, not bit for bit (the Q8_0 codes and
 * per-block integer sums are exact). Other GGUF block types return
 * DBI_ERR_UNSUPPORTED. Ordered on the handle's stream; allocates nothing. */
dbi_status dbi_oproj_residual_async(dbi_kv* kv, uint32_t wtype, const void* w_dev,
                                    const float* attn_dev, float* x_dev, uint32_t dim,
                                    uint32_t in);

/* ---- Full-layer offload: the whole of Model::decode_layer on the device
 * (replaces backend::Backend::setup_offload / decode_token /
 * decode_token_full, backend.hpp:133-157, and the offload branch of
 * Model::forward, model.cpp:896-917). */

/* one matmul weight: device data and its type (DBI_W_*) */
typedef struct dbi_weight {
  const void* data;
  uint32_t type;
} dbi_weight;

/* one transformer block (backend::LayerQ, backend.hpp:29-48): device
 * pointers; attn_norm, ffn_norm [dim]; wq [n_heads*hd][dim], wk and wv
 * [n_kv*hd][dim], wo [dim][n_heads*hd], wgate and wup [ff][dim], wdown
 * [dim][ff]; biases [n_heads*hd] / [n_kv*hd] or NULL. Alignment as
 * dbi_oproj_residual_async's w_dev. */
typedef struct dbi_layer_weights {
  const float* attn_norm;
  const float* ffn_norm;
  dbi_weight wq, wk, wv, wo, wgate, wup, wdown;
  const float* bq;
  const float* bk;
  const float* bv;
} dbi_layer_weights;

/* the shape shared by every block (LayerQ's dim, ff, n_heads, rms_eps; the
 * kv heads, head_dim and rope_theta are the cache's), and the tail of
 * decode_token_full: output_norm [dim] and lm_head [vocab][dim] (device), or
 * lm_head.data == NULL for no tail. */
typedef struct dbi_offload_config {
  uint32_t dim, ff, n_heads;
  float rms_eps;
  const float* output_norm;
  dbi_weight lm_head;
  uint32_t vocab;
} dbi_offload_config;

/* Backend::setup_offload (backend.hpp:133-143): binds n_layers blocks (the
 * first n_layers of the cache's layers) and the tail; the weights are the
 * caller's device memory, used in place until the next setup or destroy.
 * Allocates the layer's scratch rows, the dense cache's rope table and the
 * attention split workspace of the largest decode plan at any position;
 * not under graph capture. The cache may
 * be any layout (the reference offloads dense fp32 only, main.cpp:241-244):
 * dense fp32 and int8 attend after rope + append at pos, a ring through its
 * own attention (model.cpp:757-771). dim, ff and n_heads*head_dim must be
 * multiples of 32 for Q8_0 / Q4_0 weights (of 8 otherwise). */
dbi_status dbi_offload_setup(dbi_kv* kv, const dbi_offload_config* cfg,
                             const dbi_layer_weights* layers, uint32_t n_layers);

/* Backend::decode_token (backend.hpp:145-149): every bound block of one
 * token at position pos, on the handle's stream, per block exactly
 * decode_layer's sequence: rmsnorm, q/k/v matvecs, biases, rope, append,
 * attention (the fused decode step), o_proj + residual, rmsnorm, gate/up,
 * silu(gate) * up, down + residual. x_dev: device [dim] (16-byte aligned),
 * the residual stream, updated in place. Allocates nothing and never syncs:
 * dbi_offload_setup builds the rope table and sizes the split workspace for
 * the largest decode plan at any position, so a call is capturable into a
 * HIP graph right after setup.
 * Each matvec sums in a tree and rmsnorm's sum of squares too, so results
 * agree with the reference to the rounding of those sums; with Q8_0 / Q4_0
 * weights a rounding difference can move an activation code across a
 * quantization boundary (the reference's own result depends on its
 * compiler's contraction of rmsnorm's sum in the same way). */
dbi_status dbi_decode_token_async(dbi_kv* kv, float* x_dev, uint32_t pos);

/* Backend::decode_token_full (backend.hpp:151-157): dbi_decode_token_async,
 * then the final rmsnorm with output_norm and the lm_head matvec into
 * logits_dev [vocab] (Model::forward, model.cpp:914-915). Needs a tail. */
dbi_status dbi_decode_token_full_async(dbi_kv* kv, float* x_dev, uint32_t pos,
                                       float* logits_dev);

/* The same three calls on host memory, the reference Backend's own contract
 * (backend.hpp:133-157: setup_offload "copies each offloaded block's weights
 * to the device once"; decode_token and decode_token_full take host rows).
 *
 * dbi_offload_setup_host: dbi_offload_setup with every pointer of cfg and
 * layers in host memory; the library copies the norms, weights, biases,
 * output_norm and lm_head into one device allocation of its own (released
 * by the next setup or by destroy) and binds the copies. Synchronous; not
 * under graph capture. */
dbi_status dbi_offload_setup_host(dbi_kv* kv, const dbi_offload_config* cfg,
                                  const dbi_layer_weights* layers, uint32_t n_layers);

/* Backend::decode_token (backend.hpp:145-149) on a host residual row x [dim],
 * updated in place: upload, every bound block, read back. Synchronous. */
dbi_status dbi_decode_token(dbi_kv* kv, float* x, uint32_t pos);

/* Backend::decode_token_full (backend.hpp:151-157) on a host input row x
 * [dim] (not modified) into host logits [vocab]. Synchronous. */
dbi_status dbi_decode_token_full(dbi_kv* kv, const float* x, uint32_t pos, float* logits);

/* Model::save_kv_prefix (model.hpp:292-293, model.cpp:1072-1107): writes the
 * DBKVCACH v1 file of positions [0, len) with the token ids from a dense
 * fp32 cache. A dense int8 cache writes version 2, which has no counterpart
 * in the reference (its v1 is dense-fp32-only, model.cpp:1074-1075):
 *   header  "DBKVCACH", u32 2, n_layers, n_kv_heads, head_dim, len,
 *           u32 dtype (1 = int8), u32 n_sink, i32 tokens[len];
 *   payload K codes, V codes   int8 [L][len][n_kv_heads][head_dim] (signed);
 *           V block scales     f32 [L][len][n_kv_heads][head_dim/32];
 *           K channel scales   f32 [L][ceil(len/32)][n_kv_heads][head_dim];
 *           raw K rows of a partial last group f32 [L][len % 32][n_kv_heads][head_dim];
 *           K sinks, V sinks   f32 [L][min(n_sink, len)][n_kv_heads][head_dim].
 * An int8 prefix must end on a 32-token group boundary or at n_seen (a group
 * that later appends extended was requantized with their rows). Rings have
 * no prefix files. */
dbi_status dbi_kv_prefix_save(dbi_kv* kv, const char* path, const int32_t* tokens,
                              uint32_t len);
/* Model::load_kv_prefix (model.hpp:298-299, model.cpp:1109-1156): validates
 * magic, version, hyperparameters, length, token ids and exact size in the
 * reference's order, then restores K/V and sets n_seen = prefix length
 * (written to *out_len). Leaves the cache untouched on any error. A v1 file
 * loads into a dense fp32 cache, or into a dense int8 cache as the
 * quantize-on-append of its rows; a v2 file into a dense int8 cache with the
 * same n_sink, restoring its codes, scales, raw rows and sinks exactly. */
dbi_status dbi_kv_prefix_load(dbi_kv* kv, const char* path, const int32_t* tokens,
                              uint32_t n_tokens, uint32_t* out_len);

/* Read back one layer of a storage array in the reference's layout, for
 * bit-exact comparison with the CPU path. Mirrors the accessors of
 * model.cpp:420-455. Shapes (per layer):
 *   DBI_EXPORT_K, _V            fp32 [capacity][n_kv][head_dim]    (fp32 layouts)
 *   DBI_EXPORT_K8, _V8          int8 [capacity][n_kv][head_dim]    (int8 layouts)
 *   DBI_EXPORT_V_SCALE          fp32 [capacity][n_kv][n_blocks]    (int8)
 *   DBI_EXPORT_K_SCALE          ring int8: fp32 [capacity][n_kv][n_blocks];
 *                               dense int8: fp32 [n_groups][n_kv][head_dim]
 *   DBI_EXPORT_K_SINK, _V_SINK  fp32 [n_sink][n_kv][head_dim]      (dense int8)
 *   DBI_EXPORT_K_RAW            fp32 [32][n_kv][head_dim]          (dense int8)
 * bytes must equal the array's size (dbi_kv_export_bytes). */
enum {
  DBI_EXPORT_K = 0,
  DBI_EXPORT_V = 1,
  DBI_EXPORT_K8 = 2,
  DBI_EXPORT_V8 = 3,
  DBI_EXPORT_K_SCALE = 4,
  DBI_EXPORT_V_SCALE = 5,
  DBI_EXPORT_K_SINK = 6,
  DBI_EXPORT_V_SINK = 7,
  DBI_EXPORT_K_RAW = 8
};
size_t dbi_kv_export_bytes(const dbi_kv* kv, uint32_t what);
dbi_status dbi_kv_export(dbi_kv* kv, uint32_t what, uint32_t layer, void* dst, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* DBI_KV_H */
