/*
 * kv_oracle.c -- CPU restatement of dbinfer's KV cache + attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for dbinfer_amd's HIP path and
 * the CPU baseline timed by bench.py. Never linked into the product library.
 * Each function cites the reference file:line it restates; the comments in
 * kv_oracle.h list how each one is pinned by tests/.
 */
#define _POSIX_C_SOURCE 200809L
#include "kv_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* construction (model.cpp:258-297)                                    */
/* ------------------------------------------------------------------ */

static void* zalloc(size_t n, size_t sz) {
  if (n == 0) return NULL;
  return calloc(n, sz);
}

okv* okv_create(size_t n_layers, size_t max_seq, size_t n_kv_heads, size_t head_dim,
                size_t n_sink, size_t window, int dtype) {
  okv* kv = (okv*)calloc(1, sizeof(okv));
  if (!kv) return NULL;
  kv->n_sink_policy = n_sink;
  kv->window = window;
  kv->dtype = dtype;
  kv->n_layers = n_layers;
  kv->capacity = window > 0 ? n_sink + window : max_seq;
  kv->layer_stride = kv->capacity * n_kv_heads * head_dim;
  kv->pos_stride = n_kv_heads * head_dim;
  kv->n_kv_heads = n_kv_heads;
  kv->head_dim = head_dim;
  kv->n_blocks = (head_dim + OKV_BLOCK - 1) / OKV_BLOCK;
  kv->scale_stride = kv->capacity * n_kv_heads * kv->n_blocks;
  const size_t cells = n_layers * kv->layer_stride;
  int ok = 1;
  if (dtype != OKV_INT8) {
    kv->k = (float*)zalloc(cells, sizeof(float));
    kv->v = (float*)zalloc(cells, sizeof(float));
    ok = cells == 0 || (kv->k && kv->v);
  } else {
    kv->k8 = (int8_t*)zalloc(cells, 1);
    kv->v8 = (int8_t*)zalloc(cells, 1);
    kv->v_scale = (float*)zalloc(n_layers * kv->scale_stride, sizeof(float));
    ok = cells == 0 || (kv->k8 && kv->v8 && kv->v_scale);
    if (window > 0) {
      /* ring int8 keeps keys per-block (model.cpp:279-285) */
      kv->k_scale = (float*)zalloc(n_layers * kv->scale_stride, sizeof(float));
      ok = ok && (cells == 0 || kv->k_scale);
    } else {
      /* dense int8: per-channel K groups + fp32 sinks (model.cpp:287-296) */
      kv->k_group = OKV_KGROUP;
      kv->n_kgroups = (kv->capacity + kv->k_group - 1) / kv->k_group;
      kv->k_scale_stride = kv->n_kgroups * n_kv_heads * head_dim;
      kv->n_sink = n_sink;
      kv->k_scale = (float*)zalloc(n_layers * kv->k_scale_stride, sizeof(float));
      kv->k_raw = (float*)zalloc(n_layers * kv->k_group * kv->pos_stride, sizeof(float));
      ok = ok && (cells == 0 || (kv->k_scale && kv->k_raw));
      if (n_sink > 0) {
        kv->k_sink = (float*)zalloc(n_layers * n_sink * kv->pos_stride, sizeof(float));
        kv->v_sink = (float*)zalloc(n_layers * n_sink * kv->pos_stride, sizeof(float));
        ok = ok && (kv->pos_stride == 0 || n_layers == 0 || (kv->k_sink && kv->v_sink));
      }
    }
  }
  if (!ok) {
    okv_destroy(kv);
    return NULL;
  }
  return kv;
}

void okv_destroy(okv* kv) {
  if (!kv) return;
  free(kv->k);
  free(kv->v);
  free(kv->k8);
  free(kv->v8);
  free(kv->k_scale);
  free(kv->v_scale);
  free(kv->k_raw);
  free(kv->k_sink);
  free(kv->v_sink);
  free(kv);
}

int okv_is_ring(const okv* kv) { return kv->window > 0; }
int okv_is_int8(const okv* kv) { return kv->dtype == OKV_INT8; }
int okv_is_dense_f32(const okv* kv) { return !okv_is_int8(kv) && !okv_is_ring(kv); }

/* ------------------------------------------------------------------ */
/* quantization (model.cpp:303-355)                                    */
/* ------------------------------------------------------------------ */

static float max_f(float a, float b) { return (a < b) ? b : a; } /* std::max */

static int8_t clamp_code(long q) {
  if (q < -127) q = -127;
  if (q > 127) q = 127;
  return (int8_t)q;
}

/* model.cpp:303-317: symmetric per-32 block quant, zero block -> zero scale */
void ok_quant_head(const float* src, size_t n, int8_t* dst, float* scales) {
  size_t b = 0;
  for (size_t start = 0; start < n; start += OKV_BLOCK, ++b) {
    const size_t end = start + OKV_BLOCK < n ? start + OKV_BLOCK : n;
    float max_abs = 0.0f;
    for (size_t i = start; i < end; ++i) max_abs = max_f(max_abs, fabsf(src[i]));
    const float scale = max_abs / 127.0f;
    scales[b] = scale;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (size_t i = start; i < end; ++i) dst[i] = clamp_code(lroundf(src[i] * inv));
  }
}

size_t okv_slot_for(const okv* kv, size_t pos) {
  if (pos < kv->n_sink_policy) return pos;
  return kv->n_sink_policy + (pos - kv->n_sink_policy) % kv->window;
}

/* model.cpp:329-355: per-channel requant of group g over rows [0, within],
 * skipping sink slots; rows come from the [32][P] raw staging buffer */
static void requantize_kgroup(okv* kv, size_t layer, size_t g, size_t within) {
  const size_t hd = kv->head_dim, P = kv->pos_stride;
  const size_t first = g * kv->k_group;
  float* sc_base = kv->k_scale + layer * kv->k_scale_stride + g * kv->n_kv_heads * hd;
  const float* raw_base = kv->k_raw + layer * kv->k_group * P;
  for (size_t kh = 0; kh < kv->n_kv_heads; ++kh) {
    float* sc = sc_base + kh * hd;
    for (size_t c = 0; c < hd; ++c) sc[c] = 0.0f;
    for (size_t w = 0; w <= within; ++w) {
      if (first + w < kv->n_sink) continue;
      const float* raw = raw_base + w * P + kh * hd;
      for (size_t c = 0; c < hd; ++c) sc[c] = max_f(sc[c], fabsf(raw[c]));
    }
    for (size_t c = 0; c < hd; ++c) sc[c] /= 127.0f;
    for (size_t w = 0; w <= within; ++w) {
      if (first + w < kv->n_sink) continue;
      const float* raw = raw_base + w * P + kh * hd;
      int8_t* dst = kv->k8 + layer * kv->layer_stride + (first + w) * P + kh * hd;
      for (size_t c = 0; c < hd; ++c) {
        const float inv = sc[c] > 0.0f ? 1.0f / sc[c] : 0.0f;
        dst[c] = clamp_code(lroundf(raw[c] * inv));
      }
    }
  }
}

/* model.cpp:357-404 */
void okv_append(okv* kv, size_t layer, size_t pos, const float* k, const float* v) {
  const size_t P = kv->pos_stride, hd = kv->head_dim;
  if (kv->k_group > 0) {
    const size_t within = pos % kv->k_group;
    const size_t g = pos / kv->k_group;
    float* raw = kv->k_raw + layer * kv->k_group * P + within * P;
    for (size_t i = 0; i < P; ++i) raw[i] = k[i];
    if (pos < kv->n_sink) {
      float* ks = kv->k_sink + layer * kv->n_sink * P + pos * P;
      float* vs = kv->v_sink + layer * kv->n_sink * P + pos * P;
      for (size_t i = 0; i < P; ++i) {
        ks[i] = k[i];
        vs[i] = v[i];
      }
    } else {
      const size_t base = layer * kv->layer_stride + pos * P;
      const size_t sbase = layer * kv->scale_stride + pos * kv->n_kv_heads * kv->n_blocks;
      for (size_t kh = 0; kh < kv->n_kv_heads; ++kh) {
        const size_t off = kh * hd;
        ok_quant_head(v + off, hd, kv->v8 + base + off, kv->v_scale + sbase + kh * kv->n_blocks);
      }
    }
    requantize_kgroup(kv, layer, g, within);
    kv->n_seen = pos + 1;
    return;
  }
  const size_t slot = okv_is_ring(kv) ? okv_slot_for(kv, pos) : pos;
  const size_t base = layer * kv->layer_stride + slot * P;
  if (kv->dtype == OKV_INT8) {
    const size_t sbase = layer * kv->scale_stride + slot * kv->n_kv_heads * kv->n_blocks;
    for (size_t kh = 0; kh < kv->n_kv_heads; ++kh) {
      const size_t off = kh * hd;
      const size_t soff = sbase + kh * kv->n_blocks;
      ok_quant_head(k + off, hd, kv->k8 + base + off, kv->k_scale + soff);
      ok_quant_head(v + off, hd, kv->v8 + base + off, kv->v_scale + soff);
    }
  } else {
    for (size_t i = 0; i < P; ++i) {
      kv->k[base + i] = k[i];
      kv->v[base + i] = v[i];
    }
  }
  kv->n_seen = pos + 1;
}

void okv_append_n(okv* kv, size_t layer, size_t pos0, size_t n, const float* k, const float* v) {
  for (size_t r = 0; r < n; ++r)
    okv_append(kv, layer, pos0 + r, k + r * kv->pos_stride, v + r * kv->pos_stride);
}

/* model.cpp:406-418 */
size_t okv_residents(const okv* kv, size_t* slot, int32_t* rope_pos) {
  const size_t n_sink = kv->n_sink_policy, window = kv->window, n_seen = kv->n_seen;
  const size_t sinks = n_seen < n_sink ? n_seen : n_sink;
  size_t count = 0;
  for (size_t t = 0; t < sinks; ++t) {
    slot[count] = t;
    rope_pos[count] = (int32_t)t;
    ++count;
  }
  size_t window_start = n_sink;
  if (n_seen > n_sink && n_seen - n_sink > window) window_start = n_seen - window;
  for (size_t t = window_start; t < n_seen; ++t) {
    slot[count] = okv_slot_for(kv, t);
    rope_pos[count] = (int32_t)(n_sink + (t - window_start));
    ++count;
  }
  return count;
}

void okv_truncate(okv* kv, size_t n_seen) { kv->n_seen = n_seen; }

/* model.cpp:420-455 */
const float* okv_key(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->k + layer * kv->layer_stride + slot * kv->pos_stride + kh * kv->head_dim;
}
const float* okv_value(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->v + layer * kv->layer_stride + slot * kv->pos_stride + kh * kv->head_dim;
}
const int8_t* okv_key_i8(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->k8 + layer * kv->layer_stride + slot * kv->pos_stride + kh * kv->head_dim;
}
const int8_t* okv_value_i8(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->v8 + layer * kv->layer_stride + slot * kv->pos_stride + kh * kv->head_dim;
}
const float* okv_key_scales(const okv* kv, size_t layer, size_t slot, size_t kh) {
  if (kv->k_group > 0) {
    const size_t g = slot / kv->k_group;
    return kv->k_scale + layer * kv->k_scale_stride + (g * kv->n_kv_heads + kh) * kv->head_dim;
  }
  return kv->k_scale + layer * kv->scale_stride + (slot * kv->n_kv_heads + kh) * kv->n_blocks;
}
const float* okv_value_scales(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->v_scale + layer * kv->scale_stride + (slot * kv->n_kv_heads + kh) * kv->n_blocks;
}
const float* okv_key_sink(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->k_sink + layer * kv->n_sink * kv->pos_stride + slot * kv->pos_stride +
         kh * kv->head_dim;
}
const float* okv_value_sink(const okv* kv, size_t layer, size_t slot, size_t kh) {
  return kv->v_sink + layer * kv->n_sink * kv->pos_stride + slot * kv->pos_stride +
         kh * kv->head_dim;
}

/* model.cpp:457-474 */
void okv_copy_prefix_out(const okv* kv, size_t prefix_len, float* k_out, float* v_out) {
  const size_t span = prefix_len * kv->pos_stride;
  for (size_t l = 0; l < kv->n_layers; ++l) {
    memcpy(k_out + l * span, kv->k + l * kv->layer_stride, span * sizeof(float));
    memcpy(v_out + l * span, kv->v + l * kv->layer_stride, span * sizeof(float));
  }
}

void okv_copy_prefix_in(okv* kv, size_t prefix_len, const float* k_in, const float* v_in) {
  const size_t span = prefix_len * kv->pos_stride;
  for (size_t l = 0; l < kv->n_layers; ++l) {
    memcpy(kv->k + l * kv->layer_stride, k_in + l * span, span * sizeof(float));
    memcpy(kv->v + l * kv->layer_stride, v_in + l * span, span * sizeof(float));
  }
  kv->n_seen = prefix_len;
}

/* ------------------------------------------------------------------ */
/* rope / softmax (ops.cpp:19-52)                                      */
/* ------------------------------------------------------------------ */

static double rope_inv(float theta, size_t j, size_t head_dim) {
  return pow((double)theta, -2.0 * (double)j / (double)head_dim);
}

void ok_rope(float* x, const int32_t* positions, float theta, size_t n_heads, size_t seq,
             size_t head_dim) {
  const size_t half = head_dim / 2;
  for (size_t h = 0; h < n_heads; ++h) {
    for (size_t s = 0; s < seq; ++s) {
      float* v = x + (h * seq + s) * head_dim;
      const double p = (double)positions[s];
      for (size_t j = 0; j < half; ++j) {
        const double inv = rope_inv(theta, j, head_dim);
        const double c = cos(p * inv);
        const double sn = sin(p * inv);
        const float a = v[j];
        const float b = v[j + half];
        v[j] = (float)(a * c - b * sn);
        v[j + half] = (float)(b * c + a * sn);
      }
    }
  }
}

void ok_softmax(const float* in, float* out, size_t n) {
  float m = in[0];
  for (size_t i = 1; i < n; ++i)
    if (in[i] > m) m = in[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float e = expf(in[i] - m);
    out[i] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) out[i] *= inv;
}

/* ------------------------------------------------------------------ */
/* head-parallel split (thread_pool.cpp:32-40)                         */
/* ------------------------------------------------------------------ */

static void split_range(size_t idx, size_t count, size_t n, size_t* b, size_t* e) {
  const size_t base = n / count, rem = n % count;
  const size_t b0 = idx * base + (idx < rem ? idx : rem);
  const size_t b1 = b0 + base + (idx < rem ? 1u : 0u);
  *b = b0 < n ? b0 : n;
  *e = b1 < n ? b1 : n;
}

#define HEAD_PARALLEL(nt, nh, hb, he, BODY)                                  \
  do {                                                                       \
    int nt_ = (nt) < 1 ? 1 : (nt);                                           \
    if ((size_t)nt_ > (nh)) nt_ = (int)(nh);                                 \
    if (nt_ <= 1) {                                                          \
      size_t hb = 0, he = (nh);                                              \
      BODY;                                                                  \
    } else {                                                                 \
      _Pragma("omp parallel num_threads(nt_)") {                             \
        size_t hb, he;                                                       \
        split_range((size_t)omp_get_thread_num(), (size_t)nt_, (nh), &hb, &he); \
        BODY;                                                                \
      }                                                                      \
    }                                                                        \
  } while (0)

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */

/* model.cpp:567-603, one query head */
static void head_dense_f32(const okv* kv, size_t layer, size_t last, size_t kh, float scale,
                           const float* qh, float* outh, float* sc) {
  const size_t hd = kv->head_dim;
  for (size_t pp = 0; pp <= last; ++pp) {
    const float* kp = okv_key(kv, layer, pp, kh);
    float dot = 0.0f;
    for (size_t i = 0; i < hd; ++i) dot += qh[i] * kp[i];
    sc[pp] = dot * scale;
  }
  ok_softmax(sc, sc, last + 1);
  for (size_t i = 0; i < hd; ++i) outh[i] = 0.0f;
  for (size_t pp = 0; pp <= last; ++pp) {
    const float* vp = okv_value(kv, layer, pp, kh);
    const float w = sc[pp];
    for (size_t i = 0; i < hd; ++i) outh[i] += w * vp[i];
  }
}

void okv_attend_dense_f32(const okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                          const float* q, float* out, int n_threads) {
  const size_t hd = kv->head_dim, gqa = n_heads / kv->n_kv_heads;
  HEAD_PARALLEL(n_threads, n_heads, hb, he, {
    float* sc = (float*)malloc((pos + 1) * sizeof(float));
    for (size_t h = hb; h < he; ++h)
      head_dense_f32(kv, layer, pos, h / gqa, scale, q + h * hd, out + h * hd, sc);
    free(sc);
  });
}

/* model.cpp:605-660, one query head */
static void head_dense_int8(const okv* kv, size_t layer, size_t last, size_t kh, float scale,
                            const float* qh, float* outh, float* sc) {
  const size_t hd = kv->head_dim, nb = kv->n_blocks, n_sink = kv->n_sink;
  for (size_t pp = 0; pp <= last; ++pp) {
    float dot = 0.0f;
    if (pp < n_sink) {
      const float* kp = okv_key_sink(kv, layer, pp, kh);
      for (size_t i = 0; i < hd; ++i) dot += qh[i] * kp[i];
    } else {
      const int8_t* kp = okv_key_i8(kv, layer, pp, kh);
      const float* ks = okv_key_scales(kv, layer, pp, kh);
      for (size_t i = 0; i < hd; ++i) dot += qh[i] * ks[i] * (float)kp[i];
    }
    sc[pp] = dot * scale;
  }
  ok_softmax(sc, sc, last + 1);
  for (size_t i = 0; i < hd; ++i) outh[i] = 0.0f;
  for (size_t pp = 0; pp <= last; ++pp) {
    const float w = sc[pp];
    if (pp < n_sink) {
      const float* vp = okv_value_sink(kv, layer, pp, kh);
      for (size_t i = 0; i < hd; ++i) outh[i] += w * vp[i];
      continue;
    }
    const int8_t* vp = okv_value_i8(kv, layer, pp, kh);
    const float* vs = okv_value_scales(kv, layer, pp, kh);
    for (size_t b = 0; b < nb; ++b) {
      const size_t start = b * OKV_BLOCK;
      const size_t end = start + OKV_BLOCK < hd ? start + OKV_BLOCK : hd;
      const float wv = w * vs[b];
      for (size_t i = start; i < end; ++i) outh[i] += wv * (float)vp[i];
    }
  }
}

void okv_attend_dense_int8(const okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                           const float* q, float* out, int n_threads) {
  const size_t hd = kv->head_dim, gqa = n_heads / kv->n_kv_heads;
  HEAD_PARALLEL(n_threads, n_heads, hb, he, {
    float* sc = (float*)malloc((pos + 1) * sizeof(float));
    for (size_t h = hb; h < he; ++h)
      head_dense_int8(kv, layer, pos, h / gqa, scale, q + h * hd, out + h * hd, sc);
    free(sc);
  });
}

/* ring: dequantize (int8: ks[i/32]*k8, model.cpp:686-690) or copy the key of
 * one slot into kbuf */
static void ring_key(const okv* kv, size_t layer, size_t slot, size_t kh, float* kbuf) {
  const size_t hd = kv->head_dim;
  if (okv_is_int8(kv)) {
    const int8_t* kp = okv_key_i8(kv, layer, slot, kh);
    const float* ks = okv_key_scales(kv, layer, slot, kh);
    for (size_t i = 0; i < hd; ++i) kbuf[i] = ks[i / OKV_BLOCK] * (float)kp[i];
  } else {
    const float* kp = okv_key(kv, layer, slot, kh);
    for (size_t i = 0; i < hd; ++i) kbuf[i] = kp[i];
  }
}

/* ring PV accumulation of one resident, model.cpp:704-721 */
static void ring_pv(const okv* kv, size_t layer, size_t slot, size_t kh, float w, float* outh) {
  const size_t hd = kv->head_dim, nb = kv->n_blocks;
  if (okv_is_int8(kv)) {
    const int8_t* vp = okv_value_i8(kv, layer, slot, kh);
    const float* vs = okv_value_scales(kv, layer, slot, kh);
    for (size_t b = 0; b < nb; ++b) {
      const size_t start = b * OKV_BLOCK;
      const size_t end = start + OKV_BLOCK < hd ? start + OKV_BLOCK : hd;
      const float wv = w * vs[b];
      for (size_t i = start; i < end; ++i) outh[i] += wv * (float)vp[i];
    }
  } else {
    const float* vp = okv_value(kv, layer, slot, kh);
    for (size_t i = 0; i < hd; ++i) outh[i] += w * vp[i];
  }
}

/* model.cpp:662-728. The key rope is the expression of ops.cpp:27-34 with c and
 * s taken from a table holding the very same cos(p*inv)/sin(p*inv) doubles, and
 * each resident key is roped once per kv head; both changes leave every bit of
 * the result unchanged (pinned against okv_attend_ring_literal). */
void okv_attend_ring(okv* kv, size_t layer, size_t pos, size_t n_heads, float scale, float theta,
                     const float* q, const float* k, const float* v, float* out, int n_threads) {
  const size_t hd = kv->head_dim, half = hd / 2, nkv = kv->n_kv_heads;
  const size_t gqa = n_heads / nkv;
  okv_append(kv, layer, pos, k, v);
  size_t* slot = (size_t*)malloc(kv->capacity * sizeof(size_t));
  int32_t* rp = (int32_t*)malloc(kv->capacity * sizeof(int32_t));
  const size_t n_res = okv_residents(kv, slot, rp);
  const int32_t q_pos = rp[n_res - 1];
  float* qr = (float*)malloc(n_heads * hd * sizeof(float));
  memcpy(qr, q, n_heads * hd * sizeof(float));
  ok_rope(qr, &q_pos, theta, n_heads, 1, hd);

  /* cos/sin of every resident rope position (rope positions are 0..n_res-1) */
  double* cs = (double*)malloc(n_res * half * 2 * sizeof(double));
  for (size_t r = 0; r < n_res; ++r) {
    const double p = (double)rp[r];
    for (size_t j = 0; j < half; ++j) {
      const double inv = rope_inv(theta, j, hd);
      cs[(r * half + j) * 2 + 0] = cos(p * inv);
      cs[(r * half + j) * 2 + 1] = sin(p * inv);
    }
  }
  /* roped keys per kv head: [nkv][n_res][hd] */
  float* kr = (float*)malloc(nkv * n_res * hd * sizeof(float));
  for (size_t kh = 0; kh < nkv; ++kh) {
    for (size_t r = 0; r < n_res; ++r) {
      float* kb = kr + (kh * n_res + r) * hd;
      ring_key(kv, layer, slot[r], kh, kb);
      for (size_t j = 0; j < half; ++j) {
        const double c = cs[(r * half + j) * 2 + 0];
        const double sn = cs[(r * half + j) * 2 + 1];
        const float a = kb[j];
        const float b = kb[j + half];
        kb[j] = (float)(a * c - b * sn);
        kb[j + half] = (float)(b * c + a * sn);
      }
    }
  }
  HEAD_PARALLEL(n_threads, n_heads, hb, he, {
    float* sc = (float*)malloc(n_res * sizeof(float));
    for (size_t h = hb; h < he; ++h) {
      const size_t kh = h / gqa;
      const float* qh = qr + h * hd;
      for (size_t r = 0; r < n_res; ++r) {
        const float* kb = kr + (kh * n_res + r) * hd;
        float dot = 0.0f;
        for (size_t i = 0; i < hd; ++i) dot += qh[i] * kb[i];
        sc[r] = dot * scale;
      }
      ok_softmax(sc, sc, n_res);
      float* outh = out + h * hd;
      for (size_t i = 0; i < hd; ++i) outh[i] = 0.0f;
      for (size_t r = 0; r < n_res; ++r) ring_pv(kv, layer, slot[r], kh, sc[r], outh);
    }
    free(sc);
  });
  free(kr);
  free(cs);
  free(qr);
  free(rp);
  free(slot);
}

/* model.cpp:662-728 literally: rope via ops.cpp per query head per resident */
void okv_attend_ring_literal(okv* kv, size_t layer, size_t pos, size_t n_heads, float scale,
                             float theta, const float* q, const float* k, const float* v,
                             float* out) {
  const size_t hd = kv->head_dim, gqa = n_heads / kv->n_kv_heads;
  okv_append(kv, layer, pos, k, v);
  size_t* slot = (size_t*)malloc(kv->capacity * sizeof(size_t));
  int32_t* rp = (int32_t*)malloc(kv->capacity * sizeof(int32_t));
  const size_t n_res = okv_residents(kv, slot, rp);
  const int32_t q_pos = rp[n_res - 1];
  float* qr = (float*)malloc(n_heads * hd * sizeof(float));
  memcpy(qr, q, n_heads * hd * sizeof(float));
  ok_rope(qr, &q_pos, theta, n_heads, 1, hd);
  float* sc = (float*)malloc(n_res * sizeof(float));
  float* kbuf = (float*)malloc(hd * sizeof(float));
  for (size_t h = 0; h < n_heads; ++h) {
    const size_t kh = h / gqa;
    const float* qh = qr + h * hd;
    for (size_t r = 0; r < n_res; ++r) {
      ring_key(kv, layer, slot[r], kh, kbuf);
      ok_rope(kbuf, &rp[r], theta, 1, 1, hd);
      float dot = 0.0f;
      for (size_t i = 0; i < hd; ++i) dot += qh[i] * kbuf[i];
      sc[r] = dot * scale;
    }
    ok_softmax(sc, sc, n_res);
    float* outh = out + h * hd;
    for (size_t i = 0; i < hd; ++i) outh[i] = 0.0f;
    for (size_t r = 0; r < n_res; ++r) ring_pv(kv, layer, slot[r], kh, sc[r], outh);
  }
  free(kbuf);
  free(sc);
  free(qr);
  free(rp);
  free(slot);
}

/* model.cpp:956-981 (dense fp32); dense int8 runs model.cpp:605-660 per row */
void okv_attend_chunk(const okv* kv, size_t layer, size_t pos0, size_t n, size_t n_heads,
                      float scale, const float* q, float* out, int n_threads) {
  const size_t hd = kv->head_dim, gqa = n_heads / kv->n_kv_heads;
  const size_t last = pos0 + n - 1;
  const int i8 = okv_is_int8(kv);
  HEAD_PARALLEL(n_threads, n_heads, hb, he, {
    float* sc = (float*)malloc((last + 1) * sizeof(float));
    for (size_t h = hb; h < he; ++h) {
      for (size_t c = 0; c < n; ++c) {
        const float* qh = q + c * n_heads * hd + h * hd;
        float* outh = out + c * n_heads * hd + h * hd;
        if (i8)
          head_dense_int8(kv, layer, pos0 + c, h / gqa, scale, qh, outh, sc);
        else
          head_dense_f32(kv, layer, pos0 + c, h / gqa, scale, qh, outh, sc);
      }
    }
    free(sc);
  });
}

/* ------------------------------------------------------------------ */
/* prefix cache (model.cpp:1023-1156)                                  */
/* ------------------------------------------------------------------ */

static const unsigned char kMagic[8] = {'D', 'B', 'K', 'V', 'C', 'A', 'C', 'H'};
enum { kVersion = 1 };

static int fail(char* err, size_t n, const char* msg) {
  if (err && n) snprintf(err, n, "%s", msg);
  return 1;
}

int okv_prefix_save(const okv* kv, const char* path, const int32_t* tokens, size_t len, char* err,
                    size_t err_len) {
  char msg[512];
  if (!okv_is_dense_f32(kv))
    return fail(err, err_len, "kv prefix cache supports only the dense fp32 cache");
  if (len == 0) return fail(err, err_len, "kv prefix is empty");
  if (kv->n_seen < len) return fail(err, err_len, "cache holds fewer positions than the prefix");
  const size_t elems = kv->n_layers * len * kv->pos_stride;
  const size_t hdr = 8 + 5 * 4 + len * 4;
  const size_t total = hdr + 2 * elems * sizeof(float);
  unsigned char* buf = (unsigned char*)malloc(total);
  if (!buf) return fail(err, err_len, "out of memory");
  memcpy(buf, kMagic, 8);
  const uint32_t h[5] = {kVersion, (uint32_t)kv->n_layers, (uint32_t)kv->n_kv_heads,
                         (uint32_t)kv->head_dim, (uint32_t)len};
  memcpy(buf + 8, h, sizeof h);
  memcpy(buf + 28, tokens, len * 4);
  okv_copy_prefix_out(kv, len, (float*)(buf + hdr), (float*)(buf + hdr + elems * sizeof(float)));
  FILE* f = fopen(path, "wb");
  if (!f) {
    free(buf);
    snprintf(msg, sizeof msg, "cannot open kv prefix cache for writing %s", path);
    return fail(err, err_len, msg);
  }
  const size_t wrote = fwrite(buf, 1, total, f);
  const int ok = wrote == total && ferror(f) == 0;
  fclose(f);
  free(buf);
  if (!ok) {
    snprintf(msg, sizeof msg, "write error on kv prefix cache %s", path);
    return fail(err, err_len, msg);
  }
  return 0;
}

int okv_prefix_load(okv* kv, const char* path, const int32_t* tokens, size_t n_tokens,
                    size_t* out_len, char* err, size_t err_len) {
  char msg[512];
  if (!okv_is_dense_f32(kv))
    return fail(err, err_len, "kv prefix cache supports only the dense fp32 cache");
  FILE* f = fopen(path, "rb");
  if (!f) {
    snprintf(msg, sizeof msg, "cannot open kv prefix cache %s", path);
    return fail(err, err_len, msg);
  }
  size_t cap = 1 << 16, size = 0;
  unsigned char* data = (unsigned char*)malloc(cap);
  for (;;) {
    if (size == cap) {
      cap *= 2;
      data = (unsigned char*)realloc(data, cap);
    }
    const size_t got = fread(data + size, 1, cap - size, f);
    if (got == 0) break;
    size += got;
  }
  const int rd_ok = ferror(f) == 0;
  fclose(f);
  if (!rd_ok) {
    free(data);
    snprintf(msg, sizeof msg, "read error on kv prefix cache %s", path);
    return fail(err, err_len, msg);
  }
  size_t p = 0;
#define NEED(n)                                                \
  do {                                                         \
    if (p + (n) > size) {                                      \
      free(data);                                              \
      return fail(err, err_len, "kv prefix cache truncated");  \
    }                                                          \
  } while (0)
  for (int i = 0; i < 8; ++i) {
    NEED(1);
    if (data[p] != kMagic[i]) {
      free(data);
      return fail(err, err_len, "kv prefix cache bad magic");
    }
    ++p;
  }
  uint32_t u[5];
  NEED(4);
  memcpy(&u[0], data + p, 4);
  p += 4;
  if (u[0] != kVersion) {
    free(data);
    snprintf(msg, sizeof msg, "kv prefix cache version %u unsupported", u[0]);
    return fail(err, err_len, msg);
  }
  for (int i = 1; i < 5; ++i) {
    NEED(4);
    memcpy(&u[i], data + p, 4);
    p += 4;
  }
  const uint32_t n_layers = u[1], n_kv = u[2], hd = u[3], prefix_len = u[4];
  if (n_layers != kv->n_layers || n_kv != kv->n_kv_heads || hd != kv->head_dim) {
    free(data);
    return fail(err, err_len, "kv prefix cache hyperparams do not match this model");
  }
  if (prefix_len == 0) {
    free(data);
    return fail(err, err_len, "kv prefix cache has a zero-length prefix");
  }
  if (prefix_len > n_tokens) {
    free(data);
    return fail(err, err_len, "kv prefix is longer than the prompt");
  }
  if (prefix_len > kv->capacity) {
    free(data);
    return fail(err, err_len, "kv prefix exceeds cache capacity");
  }
  for (uint32_t i = 0; i < prefix_len; ++i) {
    int32_t saved;
    NEED(4);
    memcpy(&saved, data + p, 4);
    p += 4;
    if (saved != tokens[i]) {
      free(data);
      snprintf(msg, sizeof msg, "prompt prefix differs from saved cache at token %u", i);
      return fail(err, err_len, msg);
    }
  }
#undef NEED
  const size_t elems = kv->n_layers * (size_t)prefix_len * kv->pos_stride;
  if (p + 2 * elems * sizeof(float) != size) {
    free(data);
    return fail(err, err_len, "kv prefix cache payload size mismatch");
  }
  okv_copy_prefix_in(kv, prefix_len, (const float*)(data + p),
                     (const float*)(data + p + elems * sizeof(float)));
  free(data);
  if (out_len) *out_len = prefix_len;
  return 0;
}

/* ------------------------------------------------------------------ */
/* speculative merge (speculative.cpp:10-23)                           */
/* ------------------------------------------------------------------ */

size_t ok_spec_merge(const int32_t* draft, size_t k, const int32_t* target, int32_t* out,
                     size_t* n_out) {
  size_t j = 0, n = 0;
  while (j < k && draft[j] == target[j]) {
    out[n++] = draft[j];
    ++j;
  }
  out[n++] = target[j];
  if (n_out) *n_out = n;
  return j;
}

/* ------------------------------------------------------------------ */
/* greedy argmax (sample.cpp:11-28)                                    */
/* ------------------------------------------------------------------ */

/* A scan that replaces the best only on a strictly greater value: ties keep
 * the earlier index, a NaN never replaces (every comparison with it is
 * false), and a NaN in slot 0 is never replaced either, so the answer is 0. */
int32_t ok_argmax(const float* logits, size_t n) {
  int32_t best = 0;
  float bestv = logits[0];
  for (size_t i = 1; i < n; ++i) {
    if (logits[i] > bestv) {
      bestv = logits[i];
      best = (int32_t)i;
    }
  }
  return best;
}

/* ------------------------------------------------------------------ */
/* output projection + residual (model.cpp:773-774)                    */
/* ------------------------------------------------------------------ */

/* sign, 5-bit exponent, 10-bit mantissa; subnormals are man * 2^-24 */
float ok_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float v = ldexpf((float)m, -24);
    memcpy(&bits, &v, 4);
    bits |= sign;
  } else if (e == 31) {
    /* infinity keeps its sign; every NaN becomes the canonical quiet NaN,
     * std::numeric_limits<float>::quiet_NaN() (dequant.cpp:27-29) */
    bits = m == 0 ? (sign | 0x7f800000u) : 0x7fc00000u;
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* sign, exponent rebiased 127 -> 15; mantissa rounded to 10 bits, to
 * nearest with ties to even; below the normal range the implicit one is
 * shifted into a subnormal, above it the result is infinity */
uint16_t ok_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t eb = (x >> 23) & 0xffu;
  uint32_t m = x & 0x7fffffu;
  if (eb == 0xffu) return (uint16_t)(sign | (m != 0 ? 0x7e00u : 0x7c00u));
  const int32_t e = (int32_t)eb - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return sign;
    m |= 0x800000u;
    const int32_t sh = 14 - e;
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;  /* a carry may reach inf */
  return (uint16_t)(sign | q);
}

void ok_quantize_row_q8_0(const float* x, size_t n, uint8_t* out) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float* xb = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
      const float a = fabsf(xb[i]);
      if (amax < a) amax = a;  /* std::max(amax, a): a NaN never replaces */
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t db = ok_f32_to_f16(d);
    uint8_t* blk = out + b * 34;
    memcpy(blk, &db, 2);
    for (int i = 0; i < 32; ++i) {
      long q = lround(xb[i] * id);
      if (q < -127) q = -127;
      if (q > 127) q = 127;
      blk[2 + i] = (uint8_t)(int8_t)q;
    }
  }
}

/* tensor::matvec_quant (matmul.cpp:275-281, matvec_rows :225-272): Q8_0
 * and Q4_0 weights quantize the activation once (quantize_activation,
 * :27-32) and take the scalar kernels; every row is a sequential fp32 sum. */
void ok_matvec(const void* w, int wtype, const float* x, float* y, size_t out, size_t in) {
  uint8_t* xq = NULL;
  if (wtype == 8 || wtype == 2) {
    xq = (uint8_t*)malloc(in / 32 * 34);
    ok_quantize_row_q8_0(x, in, xq);
  }
  for (size_t o = 0; o < out; ++o) {
    float acc = 0.0f;
    if (wtype == 1) { /* matvec_f16, matmul.cpp:45-54: explicit fma */
      const uint16_t* row = (const uint16_t*)w + o * in;
      for (size_t i = 0; i < in; ++i) acc = fmaf(ok_f16_to_f32(row[i]), x[i], acc);
    } else if (wtype == 8) { /* matvec_q8_0_scalar, matmul.cpp:56-75 */
      const uint8_t* row = (const uint8_t*)w + o * (in / 32) * 34;
      for (size_t b = 0; b < in / 32; ++b) {
        const uint8_t* wb = row + b * 34;
        const uint8_t* ab = xq + b * 34;
        uint16_t dw, dx;
        memcpy(&dw, wb, 2);
        memcpy(&dx, ab, 2);
        int32_t sumi = 0;
        for (int i = 0; i < 32; ++i) sumi += (int32_t)(int8_t)wb[2 + i] * (int32_t)(int8_t)ab[2 + i];
        acc += ok_f16_to_f32(dw) * ok_f16_to_f32(dx) * (float)sumi;
      }
    } else if (wtype == 2) { /* matvec_q4_0_scalar, matmul.cpp:77-99: 18-byte blocks */
      const uint8_t* row = (const uint8_t*)w + o * (in / 32) * 18;
      for (size_t b = 0; b < in / 32; ++b) {
        const uint8_t* wb = row + b * 18;
        const uint8_t* ab = xq + b * 34;
        uint16_t dw, dx;
        memcpy(&dw, wb, 2);
        memcpy(&dx, ab, 2);
        int32_t sumi = 0;
        for (int j = 0; j < 16; ++j) {
          const uint8_t q = wb[2 + j];
          sumi += ((int32_t)(q & 0x0Fu) - 8) * (int32_t)(int8_t)ab[2 + j];
          sumi += ((int32_t)(q >> 4) - 8) * (int32_t)(int8_t)ab[2 + j + 16];
        }
        acc += ok_f16_to_f32(dw) * ok_f16_to_f32(dx) * (float)sumi;
      }
    } else { /* tensor::matvec, matmul.cpp:36-43 */
      const float* row = (const float*)w + o * in;
      for (size_t i = 0; i < in; ++i) acc += row[i] * x[i];
    }
    y[o] = acc;
  }
  free(xq);
}

void ok_oproj_residual(const void* w, int wtype, const float* attn, float* x, size_t dim,
                       size_t in) {
  float* proj = (float*)malloc(dim * sizeof(float));
  ok_matvec(w, wtype, attn, proj, dim, in);
  for (size_t o = 0; o < dim; ++o) x[o] += proj[o];
  free(proj);
}

/* ------------------------------------------------------------------ */
/* the whole decode layer (model.cpp:730-787)                          */
/* ------------------------------------------------------------------ */

/* ops.cpp:7-17, one row */
void ok_rmsnorm(const float* x, const float* weight, float eps, float* out, size_t dim) {
  float sumsq = 0.0f;
  for (size_t i = 0; i < dim; ++i) sumsq += x[i] * x[i];
  const float scale = 1.0f / sqrtf(sumsq / (float)dim + eps);
  for (size_t i = 0; i < dim; ++i) out[i] = x[i] * scale * weight[i];
}

/* ops.cpp:54-56 */
void ok_silu(const float* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = in[i] / (1.0f + expf(-in[i]));
}

void okv_decode_layer(okv* kv, size_t layer, float* x, int32_t pos, const ok_layer* L,
                      size_t dim, size_t ff, size_t n_heads, float eps, float theta,
                      int n_threads) {
  const size_t hd = kv->head_dim, nkv = kv->n_kv_heads;
  float* normed = (float*)malloc(dim * sizeof(float));
  float* q = (float*)malloc(n_heads * hd * sizeof(float));
  float* k = (float*)malloc(nkv * hd * sizeof(float));
  float* v = (float*)malloc(nkv * hd * sizeof(float));
  float* attn = (float*)malloc(n_heads * hd * sizeof(float));
  float* proj = (float*)malloc(dim * sizeof(float));
  float* gate = (float*)malloc(ff * sizeof(float));
  float* up = (float*)malloc(ff * sizeof(float));

  ok_rmsnorm(x, L->attn_norm, eps, normed, dim);
  ok_matvec(L->w[0], L->wtype[0], normed, q, n_heads * hd, dim);
  ok_matvec(L->w[1], L->wtype[1], normed, k, nkv * hd, dim);
  ok_matvec(L->w[2], L->wtype[2], normed, v, nkv * hd, dim);
  if (L->bq)
    for (size_t i = 0; i < n_heads * hd; ++i) q[i] += L->bq[i];
  if (L->bk)
    for (size_t i = 0; i < nkv * hd; ++i) k[i] += L->bk[i];
  if (L->bv)
    for (size_t i = 0; i < nkv * hd; ++i) v[i] += L->bv[i];
  const float scale = 1.0f / sqrtf((float)hd);
  if (!okv_is_ring(kv)) {
    const int32_t p = pos;
    ok_rope(q, &p, theta, n_heads, 1, hd);
    ok_rope(k, &p, theta, nkv, 1, hd);
    okv_append(kv, layer, (size_t)pos, k, v);
    if (okv_is_int8(kv))
      okv_attend_dense_int8(kv, layer, (size_t)pos, n_heads, scale, q, attn, n_threads);
    else
      okv_attend_dense_f32(kv, layer, (size_t)pos, n_heads, scale, q, attn, n_threads);
  } else {
    okv_attend_ring(kv, layer, (size_t)pos, n_heads, scale, theta, q, k, v, attn, n_threads);
  }
  ok_matvec(L->w[3], L->wtype[3], attn, proj, dim, n_heads * hd);
  for (size_t i = 0; i < dim; ++i) x[i] += proj[i];

  ok_rmsnorm(x, L->ffn_norm, eps, normed, dim);
  ok_matvec(L->w[4], L->wtype[4], normed, gate, ff, dim);
  ok_matvec(L->w[5], L->wtype[5], normed, up, ff, dim);
  ok_silu(gate, gate, ff);
  for (size_t i = 0; i < ff; ++i) gate[i] *= up[i];
  ok_matvec(L->w[6], L->wtype[6], gate, proj, dim, ff);
  for (size_t i = 0; i < dim; ++i) x[i] += proj[i];

  free(normed); free(q); free(k); free(v); free(attn); free(proj); free(gate); free(up);
}

void ok_logits(const float* x, const float* output_norm, const void* lm_head, int wtype,
               float eps, float* logits, size_t dim, size_t vocab) {
  float* normed = (float*)malloc(dim * sizeof(float));
  ok_rmsnorm(x, output_norm, eps, normed, dim);
  ok_matvec(lm_head, wtype, normed, logits, vocab, dim);
  free(normed);
}
