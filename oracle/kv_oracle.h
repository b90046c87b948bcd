/*
 * kv_oracle.h -- CPU restatement of dbinfer's KV-cache + attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * implementation in dbinfer_amd/. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product path (libdbi_kv.so and
 * the C++ host above it) never links or calls it.
 *
 * Every function restates the reference algorithm in plain C and cites the
 * reference file:line it follows (paths relative to the reference checkout).
 * Compiled with -O2 -ffp-contract=off and no fast-math so the fp32 evaluation
 * order written here is the one executed.
 *
 * Layout and strides are the reference's (model.hpp:108-214):
 *   dense/ring fp32  k, v        [layer][slot][kv_head][head_dim]
 *   int8             k8, v8      [layer][slot][kv_head][head_dim]
 *                    v_scale     [layer][slot][kv_head][n_blocks]
 *   ring int8        k_scale     [layer][slot][kv_head][n_blocks]
 *   dense int8       k_scale     [layer][group][kv_head][head_dim]
 *                    k_raw       [layer][32][kv_head][head_dim]
 *                    k_sink/v_sink [layer][n_sink][kv_head][head_dim]
 *
 * Pinning status of each function (how it is checked, see tests/):
 *   ok_rope            golden rope_q/k vectors + reference ops.cpp (oracle/_ref)
 *   ok_softmax         golden softmax vectors + reference ops.cpp (oracle/_ref)
 *   okv_slot_for / okv_residents   kv_ring_test case matrix + brute-force deque
 *   okv_append (int8)  closed-form quant properties, tie/zero/outlier cases,
 *                      brute-force re-derivation from the append history
 *   attention (3 layouts + chunk)  fp64 textbook attention on tiny shapes,
 *                      ring == dense-on-explicitly-roped-keys reduction,
 *                      chunk == per-row decode, int8 vs fp32 rel-L2 bound
 *   prefix save/load   byte-level format check, round trip, every error path
 *   ok_spec_merge      speculative_test merge vectors
 *   ok_argmax          sample_test argmax vectors, plus NaN / signed-zero /
 *                      infinity cases whose answer the strict-greater scan fixes
 *   ok_f16_to_f32      all 65536 half values against numpy's float16 -> float32
 *   ok_f32_to_f16      numpy's float32 -> float16 (round to nearest even) on
 *                      random, tie, subnormal, overflow and special values
 *   ok_quantize_row_q8_0  closed-form properties: |code| <= 127, the block max
 *                      maps to +-127, codes reconstruct x within d/2
 *   ok_oproj_residual  exact on small-integer data (every partial sum is an
 *                      integer below 2^24, so any order is exact); fp64 dot
 *                      product within the sequential-sum rounding bound
 *   ok_matvec          the same checks per type; Q4_0 and Q8_0 against an
 *                      integer (numpy int64) restatement of each block's sum
 *                      and the reference's term expression
 *   ok_rmsnorm, ok_silu  bit for bit against the reference's ops.cpp (oracle/_ref)
 *   okv_decode_layer   composed of the pinned functions above; checked
 *                      against a numpy restatement of model.cpp:730-787 built
 *                      from them, and with identity weights against its parts
 */
#ifndef DBI_KV_ORACLE_H
#define DBI_KV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OKV_F32 = 0, OKV_INT8 = 1 };
enum { OKV_BLOCK = 32, OKV_KGROUP = 32 }; /* kKvBlock, kKvKGroup model.hpp:81,87 */

typedef struct okv {
  /* policy (model.hpp:96-100) */
  size_t n_sink_policy;
  size_t window;
  int dtype;
  /* geometry (model.cpp:258-268) */
  size_t n_layers, capacity, layer_stride, pos_stride, n_kv_heads, head_dim;
  size_t n_blocks, scale_stride;
  size_t k_group, n_kgroups, k_scale_stride, n_sink; /* dense int8 only */
  size_t n_seen;
  float *k, *v;
  int8_t *k8, *v8;
  float *k_scale, *v_scale, *k_raw, *k_sink, *v_sink;
} okv;

/* model.cpp:258-297. Returns NULL on allocation failure. */
okv* okv_create(size_t n_layers, size_t max_seq, size_t n_kv_heads, size_t head_dim,
                size_t n_sink, size_t window, int dtype);
void okv_destroy(okv* kv);

int okv_is_ring(const okv* kv);
int okv_is_int8(const okv* kv);
int okv_is_dense_f32(const okv* kv);

/* model.cpp:303-317 */
void ok_quant_head(const float* src, size_t n, int8_t* dst, float* scales);
/* model.cpp:321-324 */
size_t okv_slot_for(const okv* kv, size_t pos);
/* model.cpp:357-404 (requantize_kgroup :329-355 inside) */
void okv_append(okv* kv, size_t layer, size_t pos, const float* k, const float* v);
/* n sequential okv_append calls at pos0..pos0+n-1 (the append loop of
 * decode_layer_chunk, model.cpp:935-954); k, v are [n][pos_stride]. */
void okv_append_n(okv* kv, size_t layer, size_t pos0, size_t n, const float* k, const float* v);
/* model.cpp:406-418; writes up to capacity entries, returns the count */
size_t okv_residents(const okv* kv, size_t* slot, int32_t* rope_pos);
/* reset() model.hpp:164 is truncate(0); mark_position(p) model.hpp:182 is truncate(p+1) */
void okv_truncate(okv* kv, size_t n_seen);

/* accessors, model.cpp:420-455 */
const float* okv_key(const okv* kv, size_t layer, size_t slot, size_t kh);
const float* okv_value(const okv* kv, size_t layer, size_t slot, size_t kh);
const int8_t* okv_key_i8(const okv* kv, size_t layer, size_t slot, size_t kh);
const int8_t* okv_value_i8(const okv* kv, size_t layer, size_t slot, size_t kh);
const float* okv_key_scales(const okv* kv, size_t layer, size_t slot, size_t kh);
const float* okv_value_scales(const okv* kv, size_t layer, size_t slot, size_t kh);
const float* okv_key_sink(const okv* kv, size_t layer, size_t slot, size_t kh);
const float* okv_value_sink(const okv* kv, size_t layer, size_t slot, size_t kh);

/* model.cpp:457-474 */
void okv_copy_prefix_out(const okv* kv, size_t prefix_len, float* k_out, float* v_out);
void okv_copy_prefix_in(okv* kv, size_t prefix_len, const float* k_in, const float* v_in);

/* ops.cpp:19-38, in place, layout [n_heads][seq][head_dim] */
void ok_rope(float* x, const int32_t* positions, float theta, size_t n_heads, size_t seq,
             size_t head_dim);
/* ops.cpp:40-52 */
void ok_softmax(const float* in, float* out, size_t n);

/* model.cpp:567-603. q [nh][hd], out [nh][hd]. n_threads >= 1 splits query heads
 * with the reference pool's contiguous split (thread_pool.cpp:32-40). */
void okv_attend_dense_f32(const okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                          const float* q, float* out, int n_threads);
/* model.cpp:605-660 */
void okv_attend_dense_int8(const okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                           const float* q, float* out, int n_threads);
/* model.cpp:662-728: appends (k, v) at pos, ropes a copy of q at n_res-1 and
 * every resident key at its rope position, attends. Rope uses a cos/sin table
 * evaluated with exactly ops.cpp's expressions (bitwise equal to calling
 * ok_rope per key) and is applied once per kv head instead of per query head
 * (same values). */
void okv_attend_ring(okv* kv, size_t layer, size_t pos, size_t n_heads, float scale, float theta,
                     const float* q, const float* k, const float* v, float* out, int n_threads);
/* literal form of the above (rope via ok_rope per query head per resident),
 * only for pinning okv_attend_ring on small shapes */
void okv_attend_ring_literal(okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                             float theta, const float* q, const float* k, const float* v,
                             float* out);
/* causal chunk attention, model.cpp:956-981: rows c in [0,n) attend [0, pos0+c].
 * q [n][nh][hd], out [n][nh][hd]. Dense fp32 follows the reference exactly;
 * dense int8 runs attend_dense_int8 per row (the reference has no int8 chunk
 * path; this is the fixed definition used for verify rounds). Keys must have
 * been appended for every row first. */
void okv_attend_chunk(const okv* kv, size_t layer, size_t pos0, size_t n, size_t n_heads,
                      float scale, const float* q, float* out, int n_threads);

/* model.cpp:1072-1107 and :1109-1156. Return 0 on success, nonzero on error
 * with the reference's message in err. load leaves the cache untouched on error. */
int okv_prefix_save(const okv* kv, const char* path, const int32_t* tokens, size_t len, char* err,
                    size_t err_len);
int okv_prefix_load(okv* kv, const char* path, const int32_t* tokens, size_t n_tokens,
                    size_t* out_len, char* err, size_t err_len);

/* speculative.cpp:10-23. out must hold k+1 entries. returns accepted count. */
size_t ok_spec_merge(const int32_t* draft, size_t k, const int32_t* target, int32_t* out,
                     size_t* n_out);

/* sample.cpp:11-28: greedy argmax, first maximum wins (strict >), n >= 1. */
int32_t ok_argmax(const float* logits, size_t n);

/* dequant.cpp:14: IEEE half to float (exact). */
float ok_f16_to_f32(uint16_t h);
/* dequant.cpp:36: float to IEEE half, round to nearest even. */
uint16_t ok_f32_to_f16(float f);
/* dequant.cpp:80-97: one row of n floats (n % 32 == 0) to Q8_0 blocks of
 * 34 bytes (f16 scale, 32 int8 codes). */
void ok_quantize_row_q8_0(const float* x, size_t n, uint8_t* out);
/* model.cpp:773-774 with matvec_quant's weight types (wtype numbered as
 * GgmlType): 0 fp32 (tensor::matvec, matmul.cpp:36-43), 1 f16
 * (tensor::matvec_f16, :45-54), 8 Q8_0 (attn quantized by
 * ok_quantize_row_q8_0, then matvec_q8_0_scalar, :56-75): proj[o] is a
 * sequential sum over the row, then x[o] += proj[o]. */
void ok_oproj_residual(const void* w, int wtype, const float* attn, float* x, size_t dim,
                       size_t in);
/* tensor::matvec_quant (matmul.cpp:225-281): y[o] = row o . x, a sequential
 * fp32 sum; wtype 0 fp32, 1 f16, 2 Q4_0 (matvec_q4_0_scalar, :77-99: 18-byte
 * blocks of an f16 scale and 16 bytes of nibbles, element j the low nibble
 * of byte j, element j + 16 its high nibble, value nibble - 8), 8 Q8_0; the
 * quantized types quantize x with ok_quantize_row_q8_0 first. */
void ok_matvec(const void* w, int wtype, const float* x, float* y, size_t out, size_t in);
/* ops.cpp:7-17 (one row) and :54-56 */
void ok_rmsnorm(const float* x, const float* weight, float eps, float* out, size_t dim);
void ok_silu(const float* in, float* out, size_t n);

/* one transformer block's weights for okv_decode_layer: w / wtype in the
 * order q, k, v, o, gate, up, down; biases may be NULL */
typedef struct {
  const float* attn_norm;
  const float* ffn_norm;
  const void* w[7];
  int wtype[7];
  const float* bq;
  const float* bk;
  const float* bv;
} ok_layer;
/* Model::decode_layer (model.cpp:730-787): rmsnorm, q/k/v matvecs, biases,
 * rope + append + attention of the cache's layout (dense: rope at pos then
 * append, attend_dense_f32/int8; ring: attend_ring), o_proj + residual,
 * rmsnorm, gate/up, silu(gate) * up, down + residual. x [dim] in place. */
void okv_decode_layer(okv* kv, size_t layer, float* x, int32_t pos, const ok_layer* L,
                      size_t dim, size_t ff, size_t n_heads, float eps, float theta,
                      int n_threads);
/* Model::forward's tail (model.cpp:914-915): rmsnorm with output_norm, then
 * the lm_head matvec into logits [vocab] */
void ok_logits(const float* x, const float* output_norm, const void* lm_head, int wtype,
               float eps, float* logits, size_t dim, size_t vocab);

#ifdef __cplusplus
}
#endif

#endif /* DBI_KV_ORACLE_H */
