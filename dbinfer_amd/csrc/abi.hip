// C-ABI of libdbi_kv.so: handle state, argument validation, host<->device
// staging, prefix-cache file I/O and readback. Kernels live in append.hip and
// attention.hip.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "kv_internal.hpp"

// The full-layer offload's bound blocks and scratch rows (dbi_offload_setup).
struct OffloadState {
  dbi_offload_config cfg{};
  std::vector<dbi_layer_weights> layers;
  float* buf = nullptr;  // one allocation: the rows below
  float *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
  float *gate = nullptr, *up = nullptr;
  float *xrow = nullptr, *logits = nullptr;  // the host-row calls' device rows
  void* owned = nullptr;  // device copies of host weights (dbi_offload_setup_host)
};

struct dbi_kv {
  dbi_kv_config cfg{};
  dbi::KvGeom geom{};
  dbi::KvStore store{};
  dbi::Workspace ws{};
  OffloadState off;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  uint32_t n_seen = 0;
  int device = 0;
};

namespace {

thread_local std::string g_error;

dbi_status fail(dbi_status st, const std::string& msg) {
  g_error = msg;
  return st;
}

dbi_status hip_fail(hipError_t e, const char* what) {
  return fail(DBI_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// Prefix files move through one pinned host chunk per handle (allocated on
// first use, kept): PCIe copies run at DMA speed and no pageable bounce or
// whole-file host buffer is needed.
constexpr size_t kPinChunk = size_t(32) << 20;

#define HIP_TRY(expr, what)                  \
  do {                                       \
    hipError_t e_ = (expr);                  \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

template <typename T>
hipError_t dalloc(T** p, size_t n, int fill = 0) {
  *p = nullptr;
  if (n == 0) return hipSuccess;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T));
  if (e != hipSuccess) return e;
  return hipMemset(*p, fill, n * sizeof(T));
}

void free_store(dbi::KvStore& s) {
  void* ptrs[] = {s.k, s.v, s.k8, s.v8, s.k_scale, s.v_scale, s.k_raw, s.k_sink, s.v_sink,
                  s.rope_cs, s.rope_dd};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  s = dbi::KvStore{};
}

void free_ws(dbi::Workspace& w) {
  if (w.part) (void)hipFree(w.part);
  if (w.pinned) (void)hipHostFree(w.pinned);
  if (w.counters) (void)hipFree(w.counters);
  if (w.staging) (void)hipFree(w.staging);
  if (w.prod) (void)hipFree(w.prod);
  if (w.verify) (void)hipFree(w.verify);
  w = dbi::Workspace{};
}

// device staging buffer for host-pointer calls (grown on demand)
dbi_status need_staging(dbi_kv* kv, size_t floats) {
  if (kv->ws.staging_floats >= floats) return DBI_OK;
  if (kv->ws.staging) (void)hipFree(kv->ws.staging);
  kv->ws.staging = nullptr;
  kv->ws.staging_floats = 0;
  if (hipMalloc(reinterpret_cast<void**>(&kv->ws.staging), floats * sizeof(float)) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "device staging allocation failed");
  kv->ws.staging_floats = floats;
  return DBI_OK;
}

dbi_status check_layer(const dbi_kv* kv, uint32_t layer) {
  if (layer >= kv->cfg.n_layers)
    return fail(DBI_ERR_INVALID, "layer " + std::to_string(layer) + " out of range");
  return DBI_OK;
}

// dense caches hold positions [0, capacity); a ring wraps any position
dbi_status check_rows(const dbi_kv* kv, uint64_t pos0, uint64_t n) {
  if (!kv->geom.ring && pos0 + n > static_cast<uint64_t>(kv->geom.cap))
    return fail(DBI_ERR_INVALID, "position " + std::to_string(pos0 + n - 1) +
                                     " exceeds cache capacity " + std::to_string(kv->geom.cap));
  if (pos0 + n > 0x7fffffffull) return fail(DBI_ERR_INVALID, "position out of range");
  return DBI_OK;
}

dbi::RingView ring_view(const dbi_kv* kv, uint32_t n_seen) {
  dbi::RingView r{};
  const uint32_t s = kv->cfg.n_sink, W = kv->cfg.window;
  r.s = static_cast<int>(s);
  r.W = static_cast<int>(W);
  const bool full = n_seen > s && n_seen - s > W;
  r.n_res = full ? static_cast<int>(s + W) : static_cast<int>(n_seen);
  r.base = full ? static_cast<int>((n_seen - s) % W) : 0;
  return r;
}

dbi_status need_pinned(dbi_kv* kv) {
  if (kv->ws.pinned) return DBI_OK;
  if (hipHostMalloc(reinterpret_cast<void**>(&kv->ws.pinned), kPinChunk, 0) != hipSuccess) {
    kv->ws.pinned = nullptr;
    return fail(DBI_ERR_NOMEM, "out of pinned host memory for prefix-file transfers");
  }
  return DBI_OK;
}

// Workspace growth syncs, frees and allocates, none of which a graph
// capture may record: under capture a call that needs more than the handle
// holds fails, and the caller makes that call once before capturing.
dbi_status refuse_capture(dbi_kv* kv, const char* what) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(kv->stream, &cap), "capture status");
  if (cap != hipStreamCaptureStatusNone)
    return fail(DBI_ERR_INVALID, std::string(what) +
                                     " would grow under graph capture; make the same call once "
                                     "before capturing");
  return DBI_OK;
}

dbi_status ensure_part(dbi_kv* kv, size_t part) {
  if (part > kv->ws.part_floats) {
    if (dbi_status st = refuse_capture(kv, "the attention workspace")) return st;
    HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
    if (kv->ws.part) (void)hipFree(kv->ws.part);
    kv->ws.part = nullptr;
    kv->ws.part_floats = 0;
    if (hipMalloc(reinterpret_cast<void**>(&kv->ws.part), part * sizeof(float)) != hipSuccess)
      return fail(DBI_ERR_NOMEM, "attention workspace allocation failed");
    kv->ws.part_floats = part;
  }
  return DBI_OK;
}

// records of `part` floats and `cnt` split counters, grown only
dbi_status ensure_ws_sizes(dbi_kv* kv, size_t part, size_t cnt) {
  if (dbi_status st = ensure_part(kv, part)) return st;
  // the kernels leave the counters at zero; a fresh array starts there
  if (cnt > kv->ws.counters_n) {
    if (dbi_status st = refuse_capture(kv, "the split counters")) return st;
    HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
    if (kv->ws.counters) (void)hipFree(kv->ws.counters);
    kv->ws.counters = nullptr;
    kv->ws.counters_n = 0;
    if (hipMalloc(reinterpret_cast<void**>(&kv->ws.counters), cnt * sizeof(unsigned)) !=
        hipSuccess)
      return fail(DBI_ERR_NOMEM, "attention counter allocation failed");
    HIP_TRY(hipMemsetAsync(kv->ws.counters, 0, cnt * sizeof(unsigned), kv->stream),
            "counter clear");
    HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
    kv->ws.counters_n = cnt;
  }
  return DBI_OK;
}

dbi_status ensure_workspace(dbi_kv* kv, const dbi::AttnCall& c) {
  return ensure_ws_sizes(kv, dbi::attention_workspace_need(kv->geom, c),
                         dbi::attention_counters_need(kv->geom, c));
}

dbi_status check_attend(const dbi_kv* kv, uint32_t layer, uint32_t n_heads, const void* q,
                        const void* out) {
  if (dbi_status st = check_layer(kv, layer)) return st;
  if (q == nullptr || out == nullptr) return fail(DBI_ERR_INVALID, "null q or out");
  if (n_heads == 0 || n_heads % kv->cfg.n_kv_heads != 0)
    return fail(DBI_ERR_INVALID, "n_heads must be a positive multiple of n_kv_heads");
  if (!dbi::attention_supported(kv->geom, static_cast<int>(n_heads)))
    return fail(DBI_ERR_UNSUPPORTED,
                "no attention kernel for head_dim " + std::to_string(kv->cfg.head_dim) +
                    " and gqa " + std::to_string(n_heads / kv->cfg.n_kv_heads) +
                    " (served: head_dim 64/128, gqa 1-8)");
  return DBI_OK;
}

dbi_status append_impl(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, const float* k_dev,
                       const float* v_dev);

// The attention call of one decode step at pos; with k_dev/v_dev set, the
// fused step that appends that row first.
dbi::AttnCall decode_call(const dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                          float scale, const float* q_dev, float* out_dev, const float* k_dev,
                          const float* v_dev) {
  dbi::AttnCall c{};
  if (k_dev != nullptr) {
    const dbi::KvGeom& g = kv->geom;
    c.app_k = k_dev;
    c.app_v = v_dev;
    c.app_pos = static_cast<int>(pos);
    c.app_slot = g.ring ? (static_cast<int>(pos) < g.n_sink
                               ? static_cast<int>(pos)
                               : g.n_sink + static_cast<int>((pos - g.n_sink) % g.window))
                        : static_cast<int>(pos);
  }
  c.layer = static_cast<int>(layer);
  c.rows = 1;
  c.pos0 = static_cast<int>(pos);
  c.n_heads = static_cast<int>(n_heads);
  c.scale = scale;
  c.q = q_dev;
  c.out = out_dev;
  if (kv->geom.ring) c.ring = ring_view(kv, pos + 1);
  return c;
}

dbi_status decode_impl(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads, float scale,
                       const float* q_dev, float* out_dev, const float* k_dev = nullptr,
                       const float* v_dev = nullptr) {
  if (dbi_status st = check_rows(kv, pos, 1)) return st;
  // the fused kernel reads the new rows 16 bytes per lane; rows that are not
  // 16-byte aligned go through the append kernel first
  if (k_dev != nullptr &&
      ((reinterpret_cast<uintptr_t>(k_dev) | reinterpret_cast<uintptr_t>(v_dev)) & 15) != 0) {
    if (dbi_status st = append_impl(kv, layer, pos, 1, k_dev, v_dev)) return st;
    k_dev = v_dev = nullptr;
  }
  const dbi::AttnCall c = decode_call(kv, layer, pos, n_heads, scale, q_dev, out_dev, k_dev, v_dev);
  if (dbi_status st = ensure_workspace(kv, c)) return st;
  HIP_TRY(dbi::launch_attention(kv->geom, kv->store, kv->ws, c, kv->stream), "attention launch");
  if (k_dev != nullptr) kv->n_seen = pos + 1;
  return DBI_OK;
}

dbi::AttnCall chunk_call(uint32_t layer, uint32_t pos0, uint32_t n, uint32_t n_heads,
                         float scale, const float* q_dev, float* out_dev) {
  dbi::AttnCall c{};
  c.layer = static_cast<int>(layer);
  c.rows = static_cast<int>(n);
  c.pos0 = static_cast<int>(pos0);
  c.n_heads = static_cast<int>(n_heads);
  c.scale = scale;
  c.q = q_dev;
  c.out = out_dev;
  return c;
}

dbi_status check_chunk(const dbi_kv* kv, uint32_t pos0, uint32_t n) {
  if (kv->geom.ring)
    return fail(DBI_ERR_UNSUPPORTED, "chunk attention serves the dense layouts only");
  if (n == 0) return DBI_OK;
  if (dbi_status st = check_rows(kv, pos0, n)) return st;
  if (n > 65535) return fail(DBI_ERR_INVALID, "chunk longer than 65535 rows");
  return DBI_OK;
}

// workspace of a chunk call (no launch)
dbi_status chunk_prepare(dbi_kv* kv, const dbi::AttnCall& c, bool* prefill) {
  *prefill = dbi::prefill_supported(kv->geom, c.n_heads, c.rows);
  if (*prefill) return ensure_part(kv, dbi::prefill_workspace_need(kv->geom, c));
  return ensure_workspace(kv, c);
}

dbi_status chunk_launch(dbi_kv* kv, const dbi::AttnCall& c, bool prefill) {
  if (prefill) {
    HIP_TRY(dbi::launch_prefill(kv->geom, kv->store, kv->ws, c, kv->stream), "prefill launch");
  } else {
    HIP_TRY(dbi::launch_attention(kv->geom, kv->store, kv->ws, c, kv->stream),
            "attention launch");
  }
  return DBI_OK;
}

dbi_status chunk_impl(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, uint32_t n_heads,
                      float scale, const float* q_dev, float* out_dev) {
  if (dbi_status st = check_chunk(kv, pos0, n)) return st;
  if (n == 0) return DBI_OK;
  const dbi::AttnCall c = chunk_call(layer, pos0, n, n_heads, scale, q_dev, out_dev);
  bool prefill = false;
  if (dbi_status st = chunk_prepare(kv, c, &prefill)) return st;
  return chunk_launch(kv, c, prefill);
}

dbi_status append_impl(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, const float* k_dev,
                       const float* v_dev) {
  HIP_TRY(dbi::launch_append(kv->geom, kv->store, static_cast<int>(layer),
                             static_cast<int>(pos0), static_cast<int>(n), k_dev, v_dev,
                             kv->stream),
          "append launch");
  kv->n_seen = pos0 + n;
  return DBI_OK;
}

dbi_status append_check(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, const void* k,
                        const void* v) {
  if (dbi_status st = check_layer(kv, layer)) return st;
  if (n > 0 && (k == nullptr || v == nullptr)) return fail(DBI_ERR_INVALID, "null k or v");
  return check_rows(kv, pos0, n);
}

// ---------------------------------------------------------------------------
// q/k/v producer: raw projections in, roped rows into the workspace, then
// the append and attention launches of the plain entry points.

struct RawQkv {
  const float* q;
  const float* k;
  const float* v;
  const float* qb;
  const float* kb;
  const float* vb;
};

// The producer's fp64 (cos, sin) table of a dense cache, built on its first
// producer call with the host's libm and uploaded once. A ring needs none:
// its keys are stored un-roped.
dbi_status ensure_rope_table(dbi_kv* kv) {
  const dbi::KvGeom& g = kv->geom;
  if (g.ring || kv->store.rope_dd != nullptr) return DBI_OK;
  if (!(kv->cfg.rope_theta > 0.0f))
    return fail(DBI_ERR_INVALID, "the q/k/v producer needs rope_theta > 0");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(kv->stream, &cap), "capture status");
  if (cap != hipStreamCaptureStatusNone)
    return fail(DBI_ERR_INVALID,
                "the first q/k/v producer call of a handle builds its rope table and cannot be "
                "captured; make one call before capturing");
  std::vector<double2> tab(size_t(g.cap) * (g.hd / 2));
  if (!dbi::rope_table_host(g, kv->cfg.rope_theta, tab.data()))
    return fail(DBI_ERR_UNSUPPORTED, "the q/k/v producer needs an even head_dim");
  double2* d = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&d), tab.size() * sizeof(double2)) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "rope table allocation failed");
  const hipError_t e = hipMemcpy(d, tab.data(), tab.size() * sizeof(double2),
                                 hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return hip_fail(e, "rope table upload");
  }
  kv->store.rope_dd = d;
  return DBI_OK;
}

dbi_status ensure_prod(dbi_kv* kv, size_t floats) {
  if (floats <= kv->ws.prod_floats) return DBI_OK;
  if (dbi_status st = refuse_capture(kv, "the producer workspace")) return st;
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  if (kv->ws.prod) (void)hipFree(kv->ws.prod);
  kv->ws.prod = nullptr;
  kv->ws.prod_floats = 0;
  if (hipMalloc(reinterpret_cast<void**>(&kv->ws.prod), floats * sizeof(float)) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "producer workspace allocation failed");
  kv->ws.prod_floats = floats;
  return DBI_OK;
}

dbi_status check_qkv(const dbi_kv* kv, uint32_t layer, uint32_t n_heads, const RawQkv& r,
                     const void* out) {
  if (dbi_status st = check_attend(kv, layer, n_heads, r.q, out)) return st;
  if (r.k == nullptr || r.v == nullptr) return fail(DBI_ERR_INVALID, "null k or v");
  return DBI_OK;
}

// decode_layer (model.cpp:747-771) from the projections: produce, then the
// fused append + attention launch. Every check and allocation comes first,
// so a failure leaves the cache as it was.
dbi_status decode_qkv_impl(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                           float scale, const RawQkv& r, float* out_dev) {
  if (dbi_status st = check_rows(kv, pos, 1)) return st;
  if (dbi_status st = ensure_rope_table(kv)) return st;
  const double2* rope_row =
      kv->geom.ring ? nullptr : kv->store.rope_dd + size_t(pos) * (kv->geom.hd / 2);
  // one launch: the attention kernel produces q, k and v itself (its row and
  // bias loads are 16 bytes per lane)
  const uintptr_t addr_bits = reinterpret_cast<uintptr_t>(r.q) | reinterpret_cast<uintptr_t>(r.k) |
                              reinterpret_cast<uintptr_t>(r.v) | reinterpret_cast<uintptr_t>(r.qb) |
                              reinterpret_cast<uintptr_t>(r.kb) | reinterpret_cast<uintptr_t>(r.vb);
  if ((addr_bits & 15) == 0) {
    dbi::AttnCall c = decode_call(kv, layer, pos, n_heads, scale, r.q, out_dev, r.k, r.v);
    c.q_bias = r.qb;
    c.k_bias = r.kb;
    c.v_bias = r.vb;
    c.rope_row = rope_row;
    if (dbi_status st = ensure_workspace(kv, c)) return st;
    HIP_TRY(dbi::launch_attention(kv->geom, kv->store, kv->ws, c, kv->stream),
            "attention launch");
    kv->n_seen = pos + 1;
    return DBI_OK;
  }
  // otherwise the producer kernel writes aligned rows for the fused step
  const size_t qn = size_t(n_heads) * kv->geom.hd, P = size_t(kv->geom.nkv) * kv->geom.hd;
  if (dbi_status st = ensure_prod(kv, qn + 2 * P)) return st;
  float* qo = kv->ws.prod;  // 16-byte aligned rows (hd is a multiple of 4)
  float* ko = qo + qn;
  float* vo = ko + P;
  const dbi::AttnCall c = decode_call(kv, layer, pos, n_heads, scale, qo, out_dev, ko, vo);
  if (dbi_status st = ensure_workspace(kv, c)) return st;
  const dbi::ProduceCall pc{1, static_cast<int>(pos), static_cast<int>(n_heads), r.q, r.k, r.v,
                            r.qb, r.kb, r.vb, qo, ko, vo};
  HIP_TRY(dbi::launch_produce(kv->geom, kv->store.rope_dd, pc, kv->stream), "producer launch");
  HIP_TRY(dbi::launch_attention(kv->geom, kv->store, kv->ws, c, kv->stream), "attention launch");
  kv->n_seen = pos + 1;
  return DBI_OK;
}

// matvec arguments of dbi_oproj_residual_async and the offload: weight type,
// alignment (fp32/f16 16 bytes, Q8_0/Q4_0 4), in a multiple of 8 (32 for the
// quantized types, whose activation row sits in LDS: in <= 32768), the
// activation 16-byte aligned (x == nullptr: the handle's own rows)
dbi_status check_matvec(uint32_t wtype, const void* w, const void* x, uint32_t out, uint32_t in,
                        const char* what) {
  if (w == nullptr) return fail(DBI_ERR_INVALID, std::string(what) + ": null weight");
  if (wtype != DBI_W_F32 && wtype != DBI_W_F16 && wtype != DBI_W_Q8_0 && wtype != DBI_W_Q4_0)
    return fail(DBI_ERR_UNSUPPORTED,
                std::string(what) + ": the matvecs serve fp32, f16, Q8_0 and Q4_0 weights only");
  const bool quant = wtype == DBI_W_Q8_0 || wtype == DBI_W_Q4_0;
  const uint32_t mult = quant ? 32 : 8;
  const uint32_t max_in = quant ? (uint32_t(1) << 15) : (uint32_t(1) << 24);
  if (out == 0 || in == 0 || in % mult != 0 || out > (uint32_t(1) << 30) || in > max_in)
    return fail(DBI_ERR_INVALID, std::string(what) +
                                     ": needs dim in [1, 2^30] and in a positive multiple of " +
                                     std::to_string(mult) + " (at most " +
                                     std::to_string(max_in) + ")");
  const uintptr_t walign = quant ? 3 : 15;
  if ((reinterpret_cast<uintptr_t>(w) & walign) != 0 ||
      (x != nullptr && (reinterpret_cast<uintptr_t>(x) & 15) != 0))
    return fail(DBI_ERR_INVALID, std::string(what) +
                                     ": needs aligned weights (16 bytes; Q8_0, Q4_0: 4) and a "
                                     "16-byte aligned activation row");
  return DBI_OK;
}

bool quant_weight(uint32_t type) { return type == DBI_W_Q8_0 || type == DBI_W_Q4_0; }

// the fused quantized matvec kernels take rows of an even block count
bool fused_matvec(uint32_t type, uint32_t in) { return quant_weight(type) && in % 64 == 0; }

// y = W x, or y += W x with accumulate. With norm_w the activation is
// rmsnorm(x, norm_w) (eps of the offload): quantized weights normalize inside
// the matvec launch; float weights read the handle's normalized row, written
// once per activation (*normed tracks that).
hipError_t run_matvec(dbi_kv* kv, const dbi_weight& w, const float* x, float* y, uint32_t out,
                      uint32_t in, bool accumulate, const float* norm_w = nullptr,
                      bool* normed = nullptr) {
  if (fused_matvec(w.type, in)) {
    dbi::MatvecCall c{};
    c.x = x;
    c.norm_w = norm_w;
    c.eps = kv->off.cfg.rms_eps;
    c.in = static_cast<int>(in);
    c.q4 = w.type == DBI_W_Q4_0;
    c.nseg = 1;
    c.w[0] = w.data;
    c.y[0] = y;
    c.rows[0] = static_cast<int>(out);
    c.acc = accumulate;
    return dbi::launch_matvec_q(c, kv->stream);
  }
  if (norm_w != nullptr) {
    if (!*normed) {
      hipError_t e = dbi::launch_rmsnorm(x, norm_w, kv->off.cfg.rms_eps, kv->off.normed,
                                         static_cast<int>(in), kv->stream);
      if (e != hipSuccess) return e;
      *normed = true;
    }
    x = kv->off.normed;
  }
  dbi::OprojCall c{};
  c.w = w.data;
  c.attn = x;
  c.x = y;
  c.dim = static_cast<int>(out);
  c.in = static_cast<int>(in);
  c.f16 = w.type == DBI_W_F16;
  c.q8 = w.type == DBI_W_Q8_0;
  c.q4 = w.type == DBI_W_Q4_0;
  c.overwrite = !accumulate;
  return dbi::launch_oproj(c, kv->stream);
}

// Model::decode_layer (model.cpp:730-787) for every bound block at pos, on
// the handle's stream. All checks come first; the q/k/v step is the
// producer's fused decode (decode_qkv_impl). With quantized weights of one
// type and dim, ff multiples of 64 a block is five launches: rmsnorm + q/k/v
// matvecs, the fused decode, o_proj + residual, rmsnorm + gate/up + silu *
// up, down + residual.
dbi_status decode_token_impl(dbi_kv* kv, float* x, uint32_t pos) {
  const OffloadState& o = kv->off;
  if (o.layers.empty()) return fail(DBI_ERR_INVALID, "decode_token needs dbi_offload_setup first");
  if (x == nullptr || (reinterpret_cast<uintptr_t>(x) & 15) != 0)
    return fail(DBI_ERR_INVALID, "decode_token needs a 16-byte aligned residual row");
  if (dbi_status st = check_rows(kv, pos, 1)) return st;
  const uint32_t hd = kv->cfg.head_dim, nkv = kv->cfg.n_kv_heads, nh = o.cfg.n_heads;
  const uint32_t dim = o.cfg.dim, ff = o.cfg.ff, qn = nh * hd, kvn = nkv * hd;
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  const uint32_t nr = static_cast<uint32_t>(dbi::matvec_rows_per_task());
  hipStream_t st = kv->stream;
  for (uint32_t l = 0; l < o.layers.size(); ++l) {
    const dbi_layer_weights& L = o.layers[l];
    bool normed = false;
    if (fused_matvec(L.wq.type, dim) && L.wk.type == L.wq.type && L.wv.type == L.wq.type &&
        qn % nr == 0 && kvn % nr == 0) {
      dbi::MatvecCall c{};
      c.x = x;
      c.norm_w = L.attn_norm;
      c.eps = o.cfg.rms_eps;
      c.in = static_cast<int>(dim);
      c.q4 = L.wq.type == DBI_W_Q4_0;
      c.nseg = 3;
      c.w[0] = L.wq.data;
      c.w[1] = L.wk.data;
      c.w[2] = L.wv.data;
      c.y[0] = o.q;
      c.y[1] = o.k;
      c.y[2] = o.v;
      c.rows[0] = static_cast<int>(qn);
      c.rows[1] = c.rows[2] = static_cast<int>(kvn);
      HIP_TRY(dbi::launch_matvec_q(c, st), "q/k/v matvec launch");
    } else {
      HIP_TRY(run_matvec(kv, L.wq, x, o.q, qn, dim, false, L.attn_norm, &normed),
              "q matvec launch");
      HIP_TRY(run_matvec(kv, L.wk, x, o.k, kvn, dim, false, L.attn_norm, &normed),
              "k matvec launch");
      HIP_TRY(run_matvec(kv, L.wv, x, o.v, kvn, dim, false, L.attn_norm, &normed),
              "v matvec launch");
    }
    const RawQkv r{o.q, o.k, o.v, L.bq, L.bk, L.bv};
    if (dbi_status s2 = decode_qkv_impl(kv, l, pos, nh, scale, r, o.attn)) return s2;
    HIP_TRY(run_matvec(kv, L.wo, o.attn, x, dim, qn, true), "o_proj launch");
    normed = false;
    if (fused_matvec(L.wgate.type, dim) && L.wup.type == L.wgate.type) {
      dbi::MatvecCall c{};
      c.x = x;
      c.norm_w = L.ffn_norm;
      c.eps = o.cfg.rms_eps;
      c.in = static_cast<int>(dim);
      c.q4 = L.wgate.type == DBI_W_Q4_0;
      c.nseg = 2;
      c.w[0] = L.wgate.data;
      c.w[1] = L.wup.data;
      c.y[0] = c.y[1] = o.gate;
      c.rows[0] = c.rows[1] = static_cast<int>(ff);
      c.pair = true;
      HIP_TRY(dbi::launch_matvec_q(c, st), "gate/up matvec launch");
    } else {
      HIP_TRY(run_matvec(kv, L.wgate, x, o.gate, ff, dim, false, L.ffn_norm, &normed),
              "gate matvec launch");
      HIP_TRY(run_matvec(kv, L.wup, x, o.up, ff, dim, false, L.ffn_norm, &normed),
              "up matvec launch");
      HIP_TRY(dbi::launch_silu_mul(o.gate, o.up, int(ff), st), "silu launch");
    }
    HIP_TRY(run_matvec(kv, L.wdown, o.gate, x, dim, ff, true), "down matvec launch");
  }
  return DBI_OK;
}

// decode_layer_chunk (model.cpp:933-981) from the projections: produce all n
// rows, append them, then the causal chunk attention.
dbi_status chunk_qkv_impl(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                          uint32_t n_heads, float scale, const RawQkv& r, float* out_dev) {
  if (dbi_status st = check_chunk(kv, pos0, n)) return st;
  if (n == 0) return DBI_OK;
  if (dbi_status st = ensure_rope_table(kv)) return st;
  const size_t qn = size_t(n) * n_heads * kv->geom.hd;
  const size_t kn = size_t(n) * kv->geom.nkv * kv->geom.hd;
  if (dbi_status st = ensure_prod(kv, qn + 2 * kn)) return st;
  float* qo = kv->ws.prod;
  float* ko = qo + qn;
  float* vo = ko + kn;
  const dbi::AttnCall c = chunk_call(layer, pos0, n, n_heads, scale, qo, out_dev);
  bool prefill = false;
  if (dbi_status st = chunk_prepare(kv, c, &prefill)) return st;
  const dbi::ProduceCall pc{static_cast<int>(n), static_cast<int>(pos0),
                            static_cast<int>(n_heads), r.q, r.k, r.v, r.qb, r.kb, r.vb,
                            qo, ko, vo};
  HIP_TRY(dbi::launch_produce(kv->geom, kv->store.rope_dd, pc, kv->stream), "producer launch");
  if (dbi_status st = append_impl(kv, layer, pos0, n, ko, vo)) return st;
  return chunk_launch(kv, c, prefill);
}

// Host-pointer form of the producer calls: q, k, v rows, the biases that are
// given, and the output share one staging buffer.
dbi_status qkv_host(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, uint32_t n_heads,
                    float scale, const RawQkv& h, float* out, bool chunk) {
  if (dbi_status st = check_qkv(kv, layer, n_heads, h, out)) return st;
  if (n == 0) return chunk ? check_chunk(kv, pos0, n) : DBI_OK;
  const size_t hq = size_t(n_heads) * kv->geom.hd, hk = size_t(kv->geom.nkv) * kv->geom.hd;
  const size_t qn = n * hq, kn = n * hk;
  const size_t need = 2 * qn + 2 * kn + (h.qb ? hq : 0) + (h.kb ? hk : 0) + (h.vb ? hk : 0);
  if (dbi_status st = need_staging(kv, need)) return st;
  float* at = kv->ws.staging;
  auto up = [&](const float* src, size_t elems, const float** dst) -> hipError_t {
    *dst = nullptr;
    if (src == nullptr) return hipSuccess;
    *dst = at;
    at += elems;
    return hipMemcpyAsync(const_cast<float*>(*dst), src, elems * sizeof(float),
                          hipMemcpyHostToDevice, kv->stream);
  };
  RawQkv d{};
  HIP_TRY(up(h.q, qn, &d.q), "q upload");
  HIP_TRY(up(h.k, kn, &d.k), "k upload");
  HIP_TRY(up(h.v, kn, &d.v), "v upload");
  HIP_TRY(up(h.qb, hq, &d.qb), "q bias upload");
  HIP_TRY(up(h.kb, hk, &d.kb), "k bias upload");
  HIP_TRY(up(h.vb, hk, &d.vb), "v bias upload");
  float* od = at;
  const dbi_status st = chunk ? chunk_qkv_impl(kv, layer, pos0, n, n_heads, scale, d, od)
                              : decode_qkv_impl(kv, layer, pos0, n_heads, scale, d, od);
  if (st != DBI_OK) {
    (void)hipStreamSynchronize(kv->stream);  // the uploads read the caller's buffers
    return st;
  }
  HIP_TRY(hipMemcpyAsync(out, od, qn * sizeof(float), hipMemcpyDeviceToHost, kv->stream),
          "out readback");
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  return DBI_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free decode step (dbi_kv_decode_noalloc_async): its split records
// and arrival counters live in one file-scope device array. Each GPU holds
// its own copy until the process ends; host code reaches it only through
// the address hipGetSymbolAddress returns on that device, taken once per
// device when the first handle on it is created (the array's name is a host
// stand-in, not a device address). Every call on a GPU shares the array:
// calls that overlap on one GPU race.
constexpr size_t kScratchRecordBytes = size_t(2) << 20;    // split records
constexpr size_t kScratchCounterBytes = size_t(64) << 10;  // arrival counters
constexpr size_t kScratchBytes = kScratchRecordBytes + kScratchCounterBytes;
constexpr int kScratchDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kScratchDevices] = {};
std::string g_scratch_error[kScratchDevices];

// With `device` current: the array's device address, and its counters
// cleared (each launch leaves them at zero again). Synchronous; called from
// dbi_kv_create, never under graph capture.
void scratch_setup(int device) {
  if (device < 0 || device >= kScratchDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] != nullptr) return;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e == hipSuccess && p == nullptr) e = hipErrorInvalidSymbol;
  if (e == hipSuccess)
    e = hipMemset(static_cast<unsigned char*>(p) + kScratchRecordBytes, 0, kScratchCounterBytes);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) {
    g_scratch_error[device] = std::string("scratch set-up failed: ") + hipGetErrorString(e);
    return;
  }
  g_scratch_ptr[device] = static_cast<unsigned char*>(p);
}

unsigned char* scratch_ptr(int device, std::string* why) {
  if (device < 0 || device >= kScratchDevices) {
    *why = "device index beyond the scratch table";
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr)
    *why = g_scratch_error[device].empty() ? "scratch not set up on this device"
                                           : g_scratch_error[device];
  return g_scratch_ptr[device];
}

}  // namespace

extern "C" {

const char* dbi_last_error(void) { return g_error.c_str(); }

dbi_status dbi_kv_create(const dbi_kv_config* cfg, dbi_kv** out) {
  if (cfg == nullptr || out == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  *out = nullptr;
  if (cfg->n_layers == 0 || cfg->n_kv_heads == 0 || cfg->head_dim == 0)
    return fail(DBI_ERR_INVALID, "n_layers, n_kv_heads and head_dim must be positive");
  if (cfg->dtype != DBI_KV_F32 && cfg->dtype != DBI_KV_INT8)
    return fail(DBI_ERR_INVALID, "unknown dtype");
  const uint64_t cap = cfg->window > 0 ? uint64_t(cfg->n_sink) + cfg->window : cfg->max_seq;
  if (cap == 0 || cap > 0x7fffffffull) return fail(DBI_ERR_INVALID, "capacity out of range");
  // kernels address one kv head's K or V array with 32-bit byte offsets
  const uint64_t capg = (cap + dbi::kCapAlign - 1) / dbi::kCapAlign * dbi::kCapAlign;
  if (capg * cfg->head_dim * (cfg->dtype == DBI_KV_INT8 ? 1 : 4) > 0x7fffffffull)
    return fail(DBI_ERR_INVALID,
                "capacity too large: one kv head's K or V array must stay below 2 GiB");
  if (cfg->window > 0 && !(cfg->rope_theta > 0.0f))
    return fail(DBI_ERR_INVALID, "ring cache needs rope_theta > 0");

  dbi_kv* kv = new (std::nothrow) dbi_kv();
  if (kv == nullptr) return fail(DBI_ERR_NOMEM, "out of host memory");
  kv->cfg = *cfg;
  dbi::KvGeom& g = kv->geom;
  g.n_layers = static_cast<int>(cfg->n_layers);
  g.cap = static_cast<int>(cap);
  g.nkv = static_cast<int>(cfg->n_kv_heads);
  g.hd = static_cast<int>(cfg->head_dim);
  g.nb = (g.hd + dbi::kBlock - 1) / dbi::kBlock;
  g.ring = cfg->window > 0;
  g.int8 = cfg->dtype == DBI_KV_INT8;
  g.window = static_cast<int>(cfg->window);
  g.n_sink = static_cast<int>(cfg->n_sink);
  g.ngroups = (g.cap + dbi::kKGroup - 1) / dbi::kKGroup;
  g.capg = (g.cap + dbi::kCapAlign - 1) / dbi::kCapAlign * dbi::kCapAlign;
  g.tiled = g.hd == 64 || g.hd == 128;
  (void)hipGetDevice(&kv->device);

  const size_t cells = size_t(g.n_layers) * g.nkv * dbi::head_elems(g);
  const size_t scales = size_t(g.n_layers) * g.nkv * g.capg * g.nb;
  dbi::KvStore& s = kv->store;
  hipError_t e = hipSuccess;
  auto A = [&](auto** p, size_t n, int fill = 0) {
    if (e == hipSuccess) e = dalloc(p, n, fill);
  };
  if (!g.int8) {
    A(&s.k, cells);
    A(&s.v, cells);
  } else {
    A(&s.k8, cells);  // code 0, like the reference's zeroed storage
    A(&s.v8, cells);
    A(&s.v_scale, scales);
    if (g.ring) {
      A(&s.k_scale, scales);
    } else {
      A(&s.k_scale, size_t(g.n_layers) * g.nkv * g.ngroups * g.hd);
      A(&s.k_raw, size_t(g.n_layers) * dbi::kKGroup * g.nkv * g.hd);
      if (g.n_sink > 0) {
        A(&s.k_sink, size_t(g.n_layers) * g.nkv * g.n_sink * g.hd);
        A(&s.v_sink, size_t(g.n_layers) * g.nkv * g.n_sink * g.hd);
      }
    }
  }
  if (e == hipSuccess && g.ring && g.hd >= 2) {
    // cos/sin of every cache-relative rope position, evaluated in fp64 with the
    // expressions of ops.cpp:27-30 and rounded to fp32
    const int half = g.hd / 2;
    std::vector<float2> tab(size_t(g.cap) * half);
    for (int p = 0; p < g.cap; ++p)
      for (int j = 0; j < half; ++j) {
        const double inv = std::pow(static_cast<double>(cfg->rope_theta),
                                    -2.0 * static_cast<double>(j) / static_cast<double>(g.hd));
        const double ang = static_cast<double>(p) * inv;
        tab[size_t(p) * half + j] = make_float2(static_cast<float>(std::cos(ang)),
                                                static_cast<float>(std::sin(ang)));
      }
    A(&s.rope_cs, tab.size());
    if (e == hipSuccess)
      e = hipMemcpy(s.rope_cs, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
  }
  if (e == hipSuccess) scratch_setup(kv->device);
  // the fills above run on the null stream, which a non-blocking stream does
  // not wait for: finish them before any work can reach the arrays
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&kv->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    free_store(s);
    delete kv;
    return fail(e == hipErrorOutOfMemory ? DBI_ERR_NOMEM : DBI_ERR_DEVICE,
                std::string("kv cache allocation failed: ") + hipGetErrorString(e));
  }
  kv->stream = kv->own_stream;
  *out = kv;
  return DBI_OK;
}

void dbi_kv_destroy(dbi_kv* kv) {
  if (kv == nullptr) return;
  (void)hipStreamSynchronize(kv->stream);
  free_store(kv->store);
  free_ws(kv->ws);
  if (kv->off.buf) (void)hipFree(kv->off.buf);
  if (kv->off.owned) (void)hipFree(kv->off.owned);
  if (kv->own_stream) (void)hipStreamDestroy(kv->own_stream);
  delete kv;
}

dbi_status dbi_kv_get_config(const dbi_kv* kv, dbi_kv_config* out) {
  if (kv == nullptr || out == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  *out = kv->cfg;
  return DBI_OK;
}

dbi_status dbi_kv_set_stream(dbi_kv* kv, void* hip_stream) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  kv->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : kv->own_stream;
  return DBI_OK;
}

dbi_status dbi_kv_sync(dbi_kv* kv) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  return DBI_OK;
}

dbi_status dbi_kv_append(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k,
                         const float* v) {
  return dbi_kv_append_n(kv, layer, pos, 1, k, v);
}

dbi_status dbi_kv_append_n(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n, const float* k,
                           const float* v) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = append_check(kv, layer, pos0, n, k, v)) return st;
  if (n == 0) return DBI_OK;
  const size_t elems = size_t(n) * kv->cfg.n_kv_heads * kv->cfg.head_dim;
  if (dbi_status st = need_staging(kv, 2 * elems)) return st;
  float* kd = kv->ws.staging;
  float* vd = kv->ws.staging + elems;
  HIP_TRY(hipMemcpyAsync(kd, k, elems * sizeof(float), hipMemcpyHostToDevice, kv->stream),
          "copy k");
  HIP_TRY(hipMemcpyAsync(vd, v, elems * sizeof(float), hipMemcpyHostToDevice, kv->stream),
          "copy v");
  if (dbi_status st = append_impl(kv, layer, pos0, n, kd, vd)) return st;
  HIP_TRY(hipStreamSynchronize(kv->stream), "append sync");
  return DBI_OK;
}

dbi_status dbi_kv_append_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                               const float* k_dev, const float* v_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = append_check(kv, layer, pos0, n, k_dev, v_dev)) return st;
  if (n == 0) return DBI_OK;
  return append_impl(kv, layer, pos0, n, k_dev, v_dev);
}

dbi_status dbi_kv_truncate(dbi_kv* kv, uint32_t n_seen) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (!kv->geom.ring && n_seen > static_cast<uint32_t>(kv->geom.cap))
    return fail(DBI_ERR_INVALID, "n_seen exceeds cache capacity");
  kv->n_seen = n_seen;
  return DBI_OK;
}

uint32_t dbi_kv_n_seen(const dbi_kv* kv) { return kv ? kv->n_seen : 0; }
uint32_t dbi_kv_capacity(const dbi_kv* kv) { return kv ? static_cast<uint32_t>(kv->geom.cap) : 0; }

dbi_status dbi_kv_slot_for(const dbi_kv* kv, uint32_t pos, uint32_t* slot) {
  if (kv == nullptr || slot == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  if (!kv->geom.ring) return fail(DBI_ERR_UNSUPPORTED, "slot_for is defined for a ring only");
  const uint32_t s = kv->cfg.n_sink, W = kv->cfg.window;
  *slot = pos < s ? pos : s + (pos - s) % W;
  return DBI_OK;
}

dbi_status dbi_kv_residents(const dbi_kv* kv, uint32_t* slot, int32_t* rope_pos, uint32_t cap,
                            uint32_t* count) {
  if (kv == nullptr || count == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  if (!kv->geom.ring) return fail(DBI_ERR_UNSUPPORTED, "residents is defined for a ring only");
  const uint32_t s = kv->cfg.n_sink, W = kv->cfg.window, n_seen = kv->n_seen;
  const uint32_t sinks = n_seen < s ? n_seen : s;
  uint32_t ws = s;
  if (n_seen > s && n_seen - s > W) ws = n_seen - W;
  const uint32_t total = sinks + (n_seen > ws ? n_seen - ws : 0);
  if (total > cap || (total > 0 && (slot == nullptr || rope_pos == nullptr)))
    return fail(DBI_ERR_INVALID, "residents output too small");
  uint32_t c = 0;
  for (uint32_t t = 0; t < sinks; ++t) {
    slot[c] = t;
    rope_pos[c] = static_cast<int32_t>(t);
    ++c;
  }
  for (uint32_t t = ws; t < n_seen; ++t) {
    slot[c] = s + (t - s) % W;
    rope_pos[c] = static_cast<int32_t>(s + (t - ws));
    ++c;
  }
  *count = c;
  return DBI_OK;
}

dbi_status dbi_attn_decode(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                           float scale, const float* q, float* out) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = check_attend(kv, layer, n_heads, q, out)) return st;
  const size_t elems = size_t(n_heads) * kv->cfg.head_dim;
  if (dbi_status st = need_staging(kv, 2 * elems)) return st;
  float* qd = kv->ws.staging;
  float* od = kv->ws.staging + elems;
  HIP_TRY(hipMemcpyAsync(qd, q, elems * sizeof(float), hipMemcpyHostToDevice, kv->stream),
          "copy q");
  if (dbi_status st = decode_impl(kv, layer, pos, n_heads, scale, qd, od)) return st;
  HIP_TRY(hipMemcpyAsync(out, od, elems * sizeof(float), hipMemcpyDeviceToHost, kv->stream),
          "copy out");
  HIP_TRY(hipStreamSynchronize(kv->stream), "attention sync");
  return DBI_OK;
}

dbi_status dbi_attn_decode_async(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                                 float scale, const float* q_dev, float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = check_attend(kv, layer, n_heads, q_dev, out_dev)) return st;
  return decode_impl(kv, layer, pos, n_heads, scale, q_dev, out_dev);
}

dbi_status dbi_attn_splits(const dbi_kv* kv, uint32_t pos0, uint32_t rows, uint32_t n_heads,
                           uint32_t* n_split) {
  if (kv == nullptr || n_split == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  if (rows == 0 || (kv->geom.ring && rows != 1))
    return fail(DBI_ERR_INVALID, "rows must be 1 (decode) or, on a dense cache, a chunk's rows");
  if (n_heads == 0 || n_heads % kv->cfg.n_kv_heads != 0 ||
      !dbi::attention_supported(kv->geom, static_cast<int>(n_heads)))
    return fail(DBI_ERR_UNSUPPORTED, "no attention kernel for this shape");
  if (dbi_status st = check_rows(kv, pos0, rows)) return st;
  dbi::AttnCall c = chunk_call(0, pos0, rows, n_heads, 1.0f, nullptr, nullptr);
  if (kv->geom.ring) c.ring = ring_view(kv, pos0 + 1);
  const bool pre = dbi::prefill_supported(kv->geom, c.n_heads, c.rows);
  *n_split = static_cast<uint32_t>(pre ? dbi::prefill_split_count(kv->geom, c)
                                       : dbi::attention_split_count(kv->geom, c));
  return DBI_OK;
}

dbi_status dbi_kv_decode(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k,
                         const float* v, uint32_t n_heads, float scale, const float* q,
                         float* out) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = append_check(kv, layer, pos, 1, k, v)) return st;
  if (dbi_status st = check_attend(kv, layer, n_heads, q, out)) return st;
  const size_t P = size_t(kv->cfg.n_kv_heads) * kv->cfg.head_dim;
  const size_t qn = size_t(n_heads) * kv->cfg.head_dim;
  if (dbi_status st = need_staging(kv, 2 * P + 2 * qn)) return st;
  float* kd = kv->ws.staging;
  float* vd = kd + P;
  float* qd = vd + P;
  float* od = qd + qn;
  HIP_TRY(hipMemcpyAsync(kd, k, P * 4, hipMemcpyHostToDevice, kv->stream), "k upload");
  HIP_TRY(hipMemcpyAsync(vd, v, P * 4, hipMemcpyHostToDevice, kv->stream), "v upload");
  HIP_TRY(hipMemcpyAsync(qd, q, qn * 4, hipMemcpyHostToDevice, kv->stream), "q upload");
  if (dbi_status st = decode_impl(kv, layer, pos, n_heads, scale, qd, od, kd, vd)) return st;
  HIP_TRY(hipMemcpyAsync(out, od, qn * 4, hipMemcpyDeviceToHost, kv->stream), "out readback");
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  return DBI_OK;
}

dbi_status dbi_kv_decode_async(dbi_kv* kv, uint32_t layer, uint32_t pos, const float* k_dev,
                               const float* v_dev, uint32_t n_heads, float scale,
                               const float* q_dev, float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = append_check(kv, layer, pos, 1, k_dev, v_dev)) return st;
  if (dbi_status st = check_attend(kv, layer, n_heads, q_dev, out_dev)) return st;
  return decode_impl(kv, layer, pos, n_heads, scale, q_dev, out_dev, k_dev, v_dev);
}

dbi_status dbi_kv_decode_noalloc_async(dbi_kv* kv, uint32_t layer, uint32_t pos,
                                       const float* k_dev, const float* v_dev, uint32_t n_heads,
                                       float scale, const float* q_dev, float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = append_check(kv, layer, pos, 1, k_dev, v_dev)) return st;
  if (dbi_status st = check_attend(kv, layer, n_heads, q_dev, out_dev)) return st;
  if (dbi_status st = check_rows(kv, pos, 1)) return st;
  std::string why;
  unsigned char* base = scratch_ptr(kv->device, &why);
  if (base == nullptr) return fail(DBI_ERR_DEVICE, why);
  // size checks come before any launch, so a refusal leaves the cache as it was
  const dbi::AttnCall sized =
      decode_call(kv, layer, pos, n_heads, scale, q_dev, out_dev, nullptr, nullptr);
  const size_t rec = dbi::attention_workspace_need(kv->geom, sized) * sizeof(float);
  const size_t cnt = dbi::attention_counters_need(kv->geom, sized) * sizeof(unsigned);
  if (rec > kScratchRecordBytes || cnt > kScratchCounterBytes)
    return fail(DBI_ERR_UNSUPPORTED,
                "allocation-free decode: this call needs " + std::to_string(rec) +
                    " bytes of split records and " + std::to_string(cnt) +
                    " bytes of counters; the scratch holds " +
                    std::to_string(kScratchRecordBytes) + " and " +
                    std::to_string(kScratchCounterBytes));
  dbi::Workspace ws{};
  ws.part = reinterpret_cast<float*>(base);
  ws.part_floats = kScratchRecordBytes / sizeof(float);
  ws.counters = reinterpret_cast<unsigned*>(base + kScratchRecordBytes);
  ws.counters_n = kScratchCounterBytes / sizeof(unsigned);
  // rows that are not 16-byte aligned go through the append kernel first
  if (((reinterpret_cast<uintptr_t>(k_dev) | reinterpret_cast<uintptr_t>(v_dev)) & 15) != 0) {
    if (dbi_status st = append_impl(kv, layer, pos, 1, k_dev, v_dev)) return st;
    k_dev = v_dev = nullptr;
  }
  const dbi::AttnCall c = decode_call(kv, layer, pos, n_heads, scale, q_dev, out_dev, k_dev, v_dev);
  HIP_TRY(dbi::launch_attention(kv->geom, kv->store, ws, c, kv->stream), "attention launch");
  kv->n_seen = pos + 1;
  return DBI_OK;
}

dbi_status dbi_attn_chunk(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                          uint32_t n_heads, float scale, const float* q, float* out) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = check_attend(kv, layer, n_heads, q, out)) return st;
  if (n == 0) return DBI_OK;
  const size_t elems = size_t(n) * n_heads * kv->cfg.head_dim;
  if (dbi_status st = need_staging(kv, 2 * elems)) return st;
  float* qd = kv->ws.staging;
  float* od = kv->ws.staging + elems;
  HIP_TRY(hipMemcpyAsync(qd, q, elems * sizeof(float), hipMemcpyHostToDevice, kv->stream),
          "copy q");
  if (dbi_status st = chunk_impl(kv, layer, pos0, n, n_heads, scale, qd, od)) return st;
  HIP_TRY(hipMemcpyAsync(out, od, elems * sizeof(float), hipMemcpyDeviceToHost, kv->stream),
          "copy out");
  HIP_TRY(hipStreamSynchronize(kv->stream), "attention sync");
  return DBI_OK;
}

dbi_status dbi_attn_chunk_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                                uint32_t n_heads, float scale, const float* q_dev,
                                float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (dbi_status st = check_attend(kv, layer, n_heads, q_dev, out_dev)) return st;
  return chunk_impl(kv, layer, pos0, n, n_heads, scale, q_dev, out_dev);
}

dbi_status dbi_kv_decode_qkv(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                             float scale, const float* q, const float* k, const float* v,
                             const float* q_bias, const float* k_bias, const float* v_bias,
                             float* out) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  return qkv_host(kv, layer, pos, 1, n_heads, scale, RawQkv{q, k, v, q_bias, k_bias, v_bias},
                  out, false);
}

dbi_status dbi_kv_decode_qkv_async(dbi_kv* kv, uint32_t layer, uint32_t pos, uint32_t n_heads,
                                   float scale, const float* q_dev, const float* k_dev,
                                   const float* v_dev, const float* q_bias_dev,
                                   const float* k_bias_dev, const float* v_bias_dev,
                                   float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  const RawQkv r{q_dev, k_dev, v_dev, q_bias_dev, k_bias_dev, v_bias_dev};
  if (dbi_status st = check_qkv(kv, layer, n_heads, r, out_dev)) return st;
  return decode_qkv_impl(kv, layer, pos, n_heads, scale, r, out_dev);
}

dbi_status dbi_kv_chunk_qkv(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                            uint32_t n_heads, float scale, const float* q, const float* k,
                            const float* v, const float* q_bias, const float* k_bias,
                            const float* v_bias, float* out) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  return qkv_host(kv, layer, pos0, n, n_heads, scale, RawQkv{q, k, v, q_bias, k_bias, v_bias},
                  out, true);
}

dbi_status dbi_kv_chunk_qkv_async(dbi_kv* kv, uint32_t layer, uint32_t pos0, uint32_t n,
                                  uint32_t n_heads, float scale, const float* q_dev,
                                  const float* k_dev, const float* v_dev,
                                  const float* q_bias_dev, const float* k_bias_dev,
                                  const float* v_bias_dev, float* out_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  const RawQkv r{q_dev, k_dev, v_dev, q_bias_dev, k_bias_dev, v_bias_dev};
  if (dbi_status st = check_qkv(kv, layer, n_heads, r, out_dev)) return st;
  return chunk_qkv_impl(kv, layer, pos0, n, n_heads, scale, r, out_dev);
}

// ---------------------------------------------------------------------------
// prefix cache, DBKVCACH v1 (model.cpp:1023-1033): little-endian magic, u32
// version, u32 n_layers, n_kv_heads, head_dim, prefix_len, i32 tokens, fp32 K
// [L][len][nkv][hd], fp32 V in the same layout.

static const unsigned char kMagic[8] = {'D', 'B', 'K', 'V', 'C', 'A', 'C', 'H'};
static const uint32_t kVersion = 1;      // model.cpp:1033: dense fp32 K then V
static const uint32_t kVersionInt8 = 2;  // dense int8 (this library; v1 is fp32-only)

}  // extern "C"

namespace {

// v2 payload of a dense int8 cache's first len positions, in file order:
// K codes, V codes (int8 [L][len][nkv][hd], signed), V block scales
// [L][len][nkv][nb], K channel scales of the groups covering len
// [L][ceil(len/32)][nkv][hd], the raw K rows of a partial last group
// [L][len % 32][nkv][hd], K sinks then V sinks [L][min(n_sink, len)][nkv][hd]
// (all fp32 but the codes).
struct Int8Payload {
  size_t codes, vsc, ksc, raw, sinks;  // bytes per code array; floats per section
  int ngl, w, ns;
  size_t bytes() const { return 2 * codes + 4 * (vsc + ksc + raw + 2 * sinks); }
};

Int8Payload int8_payload(const dbi::KvGeom& g, uint32_t len) {
  Int8Payload p{};
  const size_t L = g.n_layers, P = size_t(g.nkv) * g.hd;
  p.ngl = static_cast<int>((len + dbi::kKGroup - 1) / dbi::kKGroup);
  p.w = static_cast<int>(len % dbi::kKGroup);
  p.ns = static_cast<int>(len < uint32_t(g.n_sink) ? len : uint32_t(g.n_sink));
  p.codes = L * len * P;
  p.vsc = L * len * g.nkv * g.nb;
  p.ksc = L * size_t(p.ngl) * P;
  p.raw = L * size_t(p.w) * P;
  p.sinks = L * size_t(p.ns) * P;
  return p;
}

// every v2 section between the store and a device buffer in file order
// (unpack: buffer -> store)
hipError_t int8_sections(dbi_kv* kv, unsigned char* dev, uint32_t len, bool unpack) {
  const dbi::KvGeom& g = kv->geom;
  dbi::KvStore& s = kv->store;
  const Int8Payload p = int8_payload(g, len);
  const int n = static_cast<int>(len), L = g.n_layers, P = g.nkv * g.hd;
  int8_t* kc = reinterpret_cast<int8_t*>(dev);
  int8_t* vc = kc + p.codes;
  float* f = reinterpret_cast<float*>(dev + 2 * p.codes);
  hipError_t e = dbi::launch_prefix_codes(g, s.k8, kc, n, true, unpack, kv->stream);
  if (e == hipSuccess) e = dbi::launch_prefix_codes(g, s.v8, vc, n, false, unpack, kv->stream);
  float* at = f;
  auto rows = [&](float* store, int nkv, int dev_rows, int r, int inner, size_t count) {
    if (e == hipSuccess)
      e = dbi::launch_rows_pack(store, at, L, nkv, dev_rows, r, inner, unpack, kv->stream);
    at += count;
  };
  rows(s.v_scale, g.nkv, g.capg, n, g.nb, p.vsc);
  rows(s.k_scale, g.nkv, g.ngroups, p.ngl, g.hd, p.ksc);
  rows(s.k_raw, 1, dbi::kKGroup, p.w, P, p.raw);
  rows(s.k_sink, g.nkv, g.n_sink, p.ns, g.hd, p.sinks);
  rows(s.v_sink, g.nkv, g.n_sink, p.ns, g.hd, p.sinks);
  return e;
}

}  // namespace

extern "C" {

dbi_status dbi_kv_prefix_save(dbi_kv* kv, const char* path, const int32_t* tokens,
                              uint32_t len) {
  if (kv == nullptr || path == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  // checks in the order of model.cpp:1074-1079; a dense int8 cache writes v2
  if (kv->geom.ring)
    return fail(DBI_ERR_UNSUPPORTED, "kv prefix cache supports only the dense fp32 cache");
  if (len == 0) return fail(DBI_ERR_INVALID, "kv prefix is empty");
  if (tokens == nullptr) return fail(DBI_ERR_INVALID, "null tokens");
  if (kv->n_seen < len) return fail(DBI_ERR_INVALID, "cache holds fewer positions than the prefix");
  const dbi::KvGeom& g = kv->geom;
  // an int8 group that later appends extended was requantized with their
  // rows: only a prefix ending on a group boundary, or at n_seen, is the
  // state those len appends left
  if (g.int8 && len % dbi::kKGroup != 0 && len != kv->n_seen)
    return fail(DBI_ERR_INVALID,
                "an int8 kv prefix must end on a 32-token group boundary or at n_seen");

  const size_t elems = size_t(g.n_layers) * len * g.nkv * g.hd;
  if (dbi_status st = need_pinned(kv)) return st;
  const uint32_t version = g.int8 ? kVersionInt8 : kVersion;
  const size_t nh = g.int8 ? 7 : 5;
  std::vector<unsigned char> hdr(8 + nh * 4 + size_t(len) * 4);
  std::memcpy(hdr.data(), kMagic, 8);
  const uint32_t h[7] = {version, kv->cfg.n_layers, kv->cfg.n_kv_heads, kv->cfg.head_dim, len,
                         DBI_KV_INT8, kv->cfg.n_sink};
  std::memcpy(hdr.data() + 8, h, nh * 4);
  std::memcpy(hdr.data() + 8 + nh * 4, tokens, size_t(len) * 4);

  // the payload packed on the device in file order, then streamed out
  unsigned char* dev = nullptr;
  const size_t payload = g.int8 ? int8_payload(g, len).bytes() : 2 * elems * sizeof(float);
  if (hipMalloc(reinterpret_cast<void**>(&dev), payload) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "prefix staging allocation failed");
  hipError_t e = hipSuccess;
  if (g.int8) {
    e = int8_sections(kv, dev, len, false);
  } else {
    float* devf = reinterpret_cast<float*>(dev);
    e = dbi::launch_prefix_pack(g, kv->store.k, devf, static_cast<int>(len), true, kv->stream);
    if (e == hipSuccess)
      e = dbi::launch_prefix_pack(g, kv->store.v, devf + elems, static_cast<int>(len), false,
                                  kv->stream);
  }
  std::FILE* f = nullptr;
  if (e == hipSuccess) {
    f = std::fopen(path, "wb");
    if (f == nullptr) {
      (void)hipStreamSynchronize(kv->stream);
      (void)hipFree(dev);
      return fail(DBI_ERR_IO, std::string("cannot open kv prefix cache for writing ") + path);
    }
  }
  bool ok = f != nullptr && std::fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
  for (size_t off = 0; ok && e == hipSuccess && off < payload; off += kPinChunk) {
    const size_t n = payload - off < kPinChunk ? payload - off : kPinChunk;
    e = hipMemcpyAsync(kv->ws.pinned, dev + off, n, hipMemcpyDeviceToHost, kv->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
    if (e == hipSuccess) ok = std::fwrite(kv->ws.pinned, 1, n, f) == n;
  }
  if (e != hipSuccess) (void)hipStreamSynchronize(kv->stream);
  (void)hipFree(dev);
  ok = ok && f != nullptr && std::ferror(f) == 0;
  if (f != nullptr && std::fclose(f) != 0) ok = false;
  if (e != hipSuccess) return hip_fail(e, "prefix readback");
  if (!ok) return fail(DBI_ERR_IO, std::string("write error on kv prefix cache ") + path);
  return DBI_OK;
}

dbi_status dbi_kv_prefix_load(dbi_kv* kv, const char* path, const int32_t* tokens,
                              uint32_t n_tokens, uint32_t* out_len) {
  if (kv == nullptr || path == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  if (kv->geom.ring)
    return fail(DBI_ERR_UNSUPPORTED, "kv prefix cache supports only the dense fp32 cache");
  std::FILE* f = std::fopen(path, "rb");
  if (f == nullptr) return fail(DBI_ERR_IO, std::string("cannot open kv prefix cache ") + path);
  struct Closer {
    std::FILE* f;
    ~Closer() { std::fclose(f); }
  } closer{f};
  // the file size stands for the reference's whole-file read; the header
  // and token list are read in front, the payload streamed to the device
  bool rd_ok = std::fseek(f, 0, SEEK_END) == 0;
  const long fsize = rd_ok ? std::ftell(f) : -1;
  rd_ok = rd_ok && fsize >= 0 && std::fseek(f, 0, SEEK_SET) == 0;
  if (!rd_ok) return fail(DBI_ERR_IO, std::string("read error on kv prefix cache ") + path);
  const size_t total = static_cast<size_t>(fsize);
  size_t p = 0;  // bytes consumed
  auto need = [&](size_t n) { return p + n <= total; };
  auto take = [&](void* dst, size_t n) {
    if (std::fread(dst, 1, n, f) != n) return false;
    p += n;
    return true;
  };
  auto io_fail = [&] { return fail(DBI_ERR_IO, std::string("read error on kv prefix cache ") + path); };

  // validation in the order of model.cpp:1117-1148; v2 adds its layout
  // fields after the hyperparameters
  for (int i = 0; i < 8; ++i) {
    if (!need(1)) return fail(DBI_ERR_FORMAT, "kv prefix cache truncated");
    unsigned char ch;
    if (!take(&ch, 1)) return io_fail();
    if (ch != kMagic[i]) return fail(DBI_ERR_FORMAT, "kv prefix cache bad magic");
  }
  uint32_t u[7] = {};
  int nh = 5;
  for (int i = 0; i < nh; ++i) {
    if (!need(4)) return fail(DBI_ERR_FORMAT, "kv prefix cache truncated");
    if (!take(&u[i], 4)) return io_fail();
    if (i == 0) {
      if (u[0] != kVersion && u[0] != kVersionInt8)
        return fail(DBI_ERR_FORMAT,
                    "kv prefix cache version " + std::to_string(u[0]) + " unsupported");
      if (u[0] == kVersionInt8) nh = 7;
    }
  }
  const bool v2 = u[0] == kVersionInt8;
  const uint32_t n_layers = u[1], n_kv = u[2], hd = u[3], prefix_len = u[4];
  const dbi::KvGeom& g = kv->geom;
  if (n_layers != kv->cfg.n_layers || n_kv != kv->cfg.n_kv_heads || hd != kv->cfg.head_dim)
    return fail(DBI_ERR_FORMAT, "kv prefix cache hyperparams do not match this model");
  if (v2 && !g.int8)
    return fail(DBI_ERR_FORMAT, "kv prefix cache holds an int8 cache; this cache is dense fp32");
  if (v2 && (u[5] != DBI_KV_INT8 || u[6] != kv->cfg.n_sink))
    return fail(DBI_ERR_FORMAT, "kv prefix cache int8 layout does not match this cache");
  if (prefix_len == 0) return fail(DBI_ERR_FORMAT, "kv prefix cache has a zero-length prefix");
  if (prefix_len > n_tokens) return fail(DBI_ERR_FORMAT, "kv prefix is longer than the prompt");
  if (prefix_len > static_cast<uint32_t>(g.cap))
    return fail(DBI_ERR_FORMAT, "kv prefix exceeds cache capacity");
  if (tokens == nullptr) return fail(DBI_ERR_INVALID, "null tokens");
  for (uint32_t i = 0; i < prefix_len; ++i) {
    if (!need(4)) return fail(DBI_ERR_FORMAT, "kv prefix cache truncated");
    int32_t saved;
    if (!take(&saved, 4)) return io_fail();
    if (saved != tokens[i])
      return fail(DBI_ERR_FORMAT,
                  "prompt prefix differs from saved cache at token " + std::to_string(i));
  }
  const size_t P = size_t(g.nkv) * g.hd;
  const size_t elems = size_t(g.n_layers) * prefix_len * P;
  const size_t payload = v2 ? int8_payload(g, prefix_len).bytes() : 2 * elems * sizeof(float);
  if (p + payload != total) return fail(DBI_ERR_FORMAT, "kv prefix cache payload size mismatch");
  if (dbi_status st = need_pinned(kv)) return st;

  // payload to the device in pinned chunks, then unpacked (the cache is
  // untouched until every byte has arrived)
  unsigned char* dev = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&dev), payload) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "prefix staging allocation failed");
  hipError_t e = hipSuccess;
  bool ok = true;
  for (size_t off = 0; ok && e == hipSuccess && off < payload; off += kPinChunk) {
    const size_t n = payload - off < kPinChunk ? payload - off : kPinChunk;
    ok = std::fread(kv->ws.pinned, 1, n, f) == n;
    if (ok) e = hipMemcpyAsync(dev + off, kv->ws.pinned, n, hipMemcpyHostToDevice, kv->stream);
    if (ok && e == hipSuccess) e = hipStreamSynchronize(kv->stream);
  }
  const float* devf = reinterpret_cast<const float*>(dev);
  const int n = static_cast<int>(prefix_len);
  if (ok && e == hipSuccess) {
    if (v2) {
      e = int8_sections(kv, dev, prefix_len, true);
    } else if (g.int8) {
      // a v1 (fp32) prefix into an int8 cache: the prefix's appends,
      // quantized on append exactly as KVCache::append would
      for (int l = 0; l < g.n_layers && e == hipSuccess; ++l)
        e = dbi::launch_append(g, kv->store, l, 0, n, devf + size_t(l) * n * P,
                               devf + elems + size_t(l) * n * P, kv->stream);
    } else {
      e = dbi::launch_prefix_unpack(g, devf, kv->store.k, n, true, kv->stream);
      if (e == hipSuccess)
        e = dbi::launch_prefix_unpack(g, devf + elems, kv->store.v, n, false, kv->stream);
    }
  }
  if (ok && e == hipSuccess) e = hipStreamSynchronize(kv->stream);
  if (e != hipSuccess) (void)hipStreamSynchronize(kv->stream);
  (void)hipFree(dev);
  if (!ok) return io_fail();
  if (e != hipSuccess) return hip_fail(e, "prefix upload");
  kv->n_seen = prefix_len;
  if (out_len) *out_len = prefix_len;
  return DBI_OK;
}

// ---------------------------------------------------------------------------
// readback in the reference's layout

size_t dbi_kv_export_bytes(const dbi_kv* kv, uint32_t what) {
  if (kv == nullptr) return 0;
  const dbi::KvGeom& g = kv->geom;
  const size_t P = size_t(g.nkv) * g.hd;
  switch (what) {
    case DBI_EXPORT_K:
    case DBI_EXPORT_V: return g.int8 ? 0 : size_t(g.cap) * P * 4;
    case DBI_EXPORT_K8:
    case DBI_EXPORT_V8: return g.int8 ? size_t(g.cap) * P : 0;
    case DBI_EXPORT_V_SCALE: return g.int8 ? size_t(g.cap) * g.nkv * g.nb * 4 : 0;
    case DBI_EXPORT_K_SCALE:
      if (!g.int8) return 0;
      return g.ring ? size_t(g.cap) * g.nkv * g.nb * 4 : size_t(g.ngroups) * P * 4;
    case DBI_EXPORT_K_SINK:
    case DBI_EXPORT_V_SINK: return (g.int8 && !g.ring) ? size_t(g.n_sink) * P * 4 : 0;
    case DBI_EXPORT_K_RAW: return (g.int8 && !g.ring) ? size_t(dbi::kKGroup) * P * 4 : 0;
    default: return 0;
  }
}

dbi_status dbi_kv_export(dbi_kv* kv, uint32_t what, uint32_t layer, void* dst, size_t bytes) {
  if (kv == nullptr || dst == nullptr) return fail(DBI_ERR_INVALID, "null argument");
  if (dbi_status st = check_layer(kv, layer)) return st;
  const size_t need = dbi_kv_export_bytes(kv, what);
  if (need == 0) return fail(DBI_ERR_UNSUPPORTED, "array not present in this layout");
  if (bytes != need) return fail(DBI_ERR_INVALID, "export size mismatch");
  const dbi::KvGeom& g = kv->geom;
  const dbi::KvStore& s = kv->store;
  // head-major device arrays -> reference [rows][nkv][inner]; K/V codes and
  // values are read back through the granule layout
  enum Map { kRows, kKeys, kValues, kFlat };
  const void* src = nullptr;
  size_t rows = 0, inner = 0, esz = 4, dev_rows = 0;
  Map map = kRows;
  switch (what) {
    case DBI_EXPORT_K: src = s.k; map = kKeys; break;
    case DBI_EXPORT_V: src = s.v; map = kValues; break;
    case DBI_EXPORT_K8: src = s.k8; map = kKeys; esz = 1; break;
    case DBI_EXPORT_V8: src = s.v8; map = kValues; esz = 1; break;
    case DBI_EXPORT_V_SCALE: src = s.v_scale; rows = g.cap; dev_rows = g.capg; inner = g.nb; break;
    case DBI_EXPORT_K_SCALE:
      src = s.k_scale;
      rows = g.ring ? g.cap : g.ngroups;
      dev_rows = g.ring ? g.capg : g.ngroups;
      inner = g.ring ? g.nb : g.hd;
      break;
    case DBI_EXPORT_K_SINK: src = s.k_sink; rows = dev_rows = g.n_sink; inner = g.hd; break;
    case DBI_EXPORT_V_SINK: src = s.v_sink; rows = dev_rows = g.n_sink; inner = g.hd; break;
    case DBI_EXPORT_K_RAW:
      src = s.k_raw; rows = dev_rows = dbi::kKGroup; inner = size_t(g.nkv) * g.hd; map = kFlat;
      break;
    default: return fail(DBI_ERR_UNSUPPORTED, "unknown export");
  }
  if (map == kKeys || map == kValues) {
    rows = g.cap;
    dev_rows = g.capg;
    inner = g.hd;
  }
  const size_t layer_bytes = (map == kFlat ? 1 : size_t(g.nkv)) * dev_rows * inner * esz;
  std::vector<unsigned char> tmp(layer_bytes);
  hipError_t e = hipMemcpyAsync(tmp.data(), static_cast<const unsigned char*>(src) + layer * layer_bytes,
                                layer_bytes, hipMemcpyDeviceToHost, kv->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
  if (e != hipSuccess) return hip_fail(e, "export readback");
  unsigned char* out = static_cast<unsigned char*>(dst);
  if (map == kFlat) {
    std::memcpy(out, tmp.data(), layer_bytes);
    return DBI_OK;
  }
  if (map == kRows) {
    const size_t row_bytes = inner * esz;
    for (size_t kh = 0; kh < size_t(g.nkv); ++kh)
      for (size_t r = 0; r < rows; ++r)
        std::memcpy(out + (r * g.nkv + kh) * row_bytes, tmp.data() + (kh * dev_rows + r) * row_bytes,
                    row_bytes);
    return DBI_OK;
  }
  const size_t he = dbi::head_elems(g);
  for (size_t kh = 0; kh < size_t(g.nkv); ++kh)
    for (int r = 0; r < g.cap; ++r)
      for (int d = 0; d < g.hd; ++d) {
        const size_t at = kh * he + (map == kKeys ? dbi::k_off(g, r, d) : dbi::v_off(g, r, d));
        const size_t to = (size_t(r) * g.nkv + kh) * g.hd + d;
        if (esz == 1)
          out[to] = tmp[at];
        else
          std::memcpy(out + to * 4, tmp.data() + at * 4, 4);
      }
  return DBI_OK;
}

/* ------------------------------------------------------------------ */
/* speculative verify round, token side                                */
/* ------------------------------------------------------------------ */

}  // extern "C"

namespace {

// verify workspace: slice keys, then the arrival counter, then int32 staging
// for the host variant (draft, verified argmaxes, accepted count)
constexpr size_t kVerifyKeysBytes =
    size_t(dbi::kMaxVerifyRows) * dbi::kMaxVerifySlices * sizeof(unsigned long long);
constexpr size_t kVerifyCounterAt = kVerifyKeysBytes;
constexpr size_t kVerifyIntsAt = kVerifyCounterAt + 256;
constexpr size_t kVerifyBytes =
    kVerifyIntsAt + sizeof(int32_t) * (dbi::kMaxVerifyDraft + dbi::kMaxVerifyRows + 1);

dbi_status ensure_verify(dbi_kv* kv) {
  if (kv->ws.verify != nullptr) return DBI_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(kv->stream, &cap), "capture status");
  if (cap != hipStreamCaptureStatusNone)
    return fail(DBI_ERR_INVALID,
                "the first verify call of a handle allocates its workspace and cannot be "
                "captured; make one call before capturing");
  unsigned char* w = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&w), kVerifyBytes) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "verify workspace allocation failed");
  // the kernel leaves the counter at zero; a fresh one starts there
  hipError_t e = hipMemsetAsync(w + kVerifyCounterAt, 0, sizeof(unsigned), kv->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
  if (e != hipSuccess) {
    (void)hipFree(w);
    return hip_fail(e, "verify counter clear");
  }
  kv->ws.verify = w;
  return DBI_OK;
}

dbi_status check_verify(const dbi_kv* kv, uint32_t k, uint32_t vocab) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (k == 0 || k > uint32_t(dbi::kMaxVerifyDraft))
    return fail(DBI_ERR_INVALID, "verify needs 1 <= k <= " +
                                     std::to_string(dbi::kMaxVerifyDraft) + " draft tokens");
  if (vocab == 0 || vocab > (uint32_t(1) << 30))
    return fail(DBI_ERR_INVALID, "verify needs 1 <= vocab <= 2^30");
  return DBI_OK;
}

dbi_status verify_impl(dbi_kv* kv, uint32_t k, uint32_t vocab, const float* logits_dev,
                       const int32_t* draft_dev, int32_t* verified_dev, int32_t* accepted_dev) {
  if (dbi_status st = ensure_verify(kv)) return st;
  dbi::VerifyCall c{};
  c.logits = logits_dev;
  c.draft = draft_dev;
  c.verified = verified_dev;
  c.accepted = accepted_dev;
  c.keys = reinterpret_cast<unsigned long long*>(kv->ws.verify);
  c.counter = reinterpret_cast<unsigned*>(kv->ws.verify + kVerifyCounterAt);
  c.rows = static_cast<int>(k) + 1;
  c.vocab = static_cast<int>(vocab);
  HIP_TRY(dbi::launch_verify(c, kv->stream), "verify launch");
  return DBI_OK;
}

}  // namespace

extern "C" {

dbi_status dbi_spec_verify_async(dbi_kv* kv, uint32_t k, uint32_t vocab, const float* logits_dev,
                                 const int32_t* draft_dev, int32_t* verified_dev,
                                 int32_t* accepted_dev) {
  if (dbi_status st = check_verify(kv, k, vocab)) return st;
  if (logits_dev == nullptr || draft_dev == nullptr || verified_dev == nullptr ||
      accepted_dev == nullptr)
    return fail(DBI_ERR_INVALID, "null verify argument");
  return verify_impl(kv, k, vocab, logits_dev, draft_dev, verified_dev, accepted_dev);
}

dbi_status dbi_kv_verify_commit(dbi_kv* kv, uint32_t pos, uint32_t k, uint32_t vocab,
                                const float* logits_dev, const int32_t* draft, int32_t* merged,
                                uint32_t* accepted) {
  if (dbi_status st = check_verify(kv, k, vocab)) return st;
  if (logits_dev == nullptr || draft == nullptr || merged == nullptr || accepted == nullptr)
    return fail(DBI_ERR_INVALID, "null verify argument");
  if (uint64_t(pos) + k + 1 > kv->n_seen)
    return fail(DBI_ERR_INVALID,
                "verify commit needs the round's k+1 rows in the cache (pos + k + 1 <= n_seen)");
  if (dbi_status st = ensure_verify(kv)) return st;
  int32_t* ints = reinterpret_cast<int32_t*>(kv->ws.verify + kVerifyIntsAt);
  int32_t* d_draft = ints;
  int32_t* d_ver = ints + dbi::kMaxVerifyDraft;
  int32_t* d_acc = d_ver + dbi::kMaxVerifyRows;
  HIP_TRY(hipMemcpyAsync(d_draft, draft, k * sizeof(int32_t), hipMemcpyHostToDevice, kv->stream),
          "copy draft");
  if (dbi_status st = verify_impl(kv, k, vocab, logits_dev, d_draft, d_ver, d_acc)) return st;
  // verified and the count are adjacent: one readback
  int32_t back[dbi::kMaxVerifyRows + 1];
  HIP_TRY(hipMemcpyAsync(back, d_ver, (dbi::kMaxVerifyRows + 1) * sizeof(int32_t),
                         hipMemcpyDeviceToHost, kv->stream),
          "copy verified");
  HIP_TRY(hipStreamSynchronize(kv->stream), "verify sync");
  const uint32_t acc = static_cast<uint32_t>(back[dbi::kMaxVerifyRows]);
  for (uint32_t i = 0; i <= acc; ++i) merged[i] = back[i];
  *accepted = acc;
  kv->n_seen = pos + acc + 1;
  return DBI_OK;
}

/* ------------------------------------------------------------------ */
/* output projection + residual add                                    */
/* ------------------------------------------------------------------ */

dbi_status dbi_oproj_residual_async(dbi_kv* kv, uint32_t wtype, const void* w_dev,
                                    const float* attn_dev, float* x_dev, uint32_t dim,
                                    uint32_t in) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  if (w_dev == nullptr || attn_dev == nullptr || x_dev == nullptr)
    return fail(DBI_ERR_INVALID, "null output-projection argument");
  if (dbi_status st = check_matvec(wtype, w_dev, attn_dev, dim, in, "output projection"))
    return st;
  HIP_TRY(run_matvec(kv, dbi_weight{w_dev, wtype}, attn_dev, x_dev, dim, in, true),
          "output projection launch");
  return DBI_OK;
}

// ---------------------------------------------------------------------------
// full-layer offload (backend.hpp:133-157; model.cpp:730-787, 896-917)

// owned: device copies the handle takes over on success (the host-row
// setup's), or null; either way the previous setup's copies are released.
static dbi_status offload_setup_impl(dbi_kv* kv, const dbi_offload_config* cfg,
                              const dbi_layer_weights* layers, uint32_t n_layers, void* owned) {
  if (kv == nullptr || cfg == nullptr || layers == nullptr)
    return fail(DBI_ERR_INVALID, "null offload argument");
  const uint32_t nkv = kv->cfg.n_kv_heads, hd = kv->cfg.head_dim;
  if (n_layers == 0 || n_layers > kv->cfg.n_layers)
    return fail(DBI_ERR_INVALID, "offload needs 1 to n_layers blocks");
  if (cfg->dim == 0 || cfg->ff == 0 || cfg->n_heads == 0 || cfg->n_heads % nkv != 0 ||
      cfg->dim > (uint32_t(1) << 20) || cfg->ff > (uint32_t(1) << 20) ||
      cfg->n_heads > 4096)
    return fail(DBI_ERR_INVALID,
                "offload needs dim, ff in [1, 2^20] and n_heads a multiple of n_kv_heads");
  if (!dbi::attention_supported(kv->geom, static_cast<int>(cfg->n_heads)))
    return fail(DBI_ERR_UNSUPPORTED, "no attention kernel for this shape");
  if (!(kv->cfg.rope_theta > 0.0f) && !kv->geom.ring)
    return fail(DBI_ERR_INVALID, "offload of a dense cache needs rope_theta > 0");
  const uint32_t qn = cfg->n_heads * hd, kvn = nkv * hd;
  for (uint32_t l = 0; l < n_layers; ++l) {
    const dbi_layer_weights& L = layers[l];
    if (L.attn_norm == nullptr || L.ffn_norm == nullptr)
      return fail(DBI_ERR_INVALID, "offload block " + std::to_string(l) + ": null norm weight");
    struct {
      const dbi_weight& w;
      uint32_t out, in;
      const char* name;
    } ws[] = {{L.wq, qn, cfg->dim, "wq"},      {L.wk, kvn, cfg->dim, "wk"},
              {L.wv, kvn, cfg->dim, "wv"},      {L.wo, cfg->dim, qn, "wo"},
              {L.wgate, cfg->ff, cfg->dim, "wgate"}, {L.wup, cfg->ff, cfg->dim, "wup"},
              {L.wdown, cfg->dim, cfg->ff, "wdown"}};
    for (const auto& w : ws) {
      // (the activation rows are the handle's own, 16-byte aligned)
      const std::string what = "offload block " + std::to_string(l) + " " + w.name;
      if (dbi_status st = check_matvec(w.w.type, w.w.data, nullptr, w.out, w.in, what.c_str()))
        return st;
    }
  }
  if (cfg->lm_head.data != nullptr) {
    if (cfg->output_norm == nullptr || cfg->vocab == 0)
      return fail(DBI_ERR_INVALID, "offload tail needs output_norm and vocab");
    if (dbi_status st =
            check_matvec(cfg->lm_head.type, cfg->lm_head.data, nullptr, cfg->vocab, cfg->dim,
                         "lm_head"))
      return st;
  }
  if (dbi_status st = refuse_capture(kv, "the offload scratch")) return st;
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  // the token calls allocate nothing: the rope table and the split workspace
  // of the largest decode plan at any position are in place from here on
  if (dbi_status st = ensure_rope_table(kv)) return st;
  if (dbi_status st = ensure_ws_sizes(
          kv, dbi::attention_workspace_bound(kv->geom, static_cast<int>(cfg->n_heads)),
          dbi::attention_counters_bound(kv->geom)))
    return st;
  OffloadState& o = kv->off;
  if (o.buf) (void)hipFree(o.buf);
  o.buf = nullptr;
  // rows rounded up to 64 floats: every row stays 256-byte aligned
  auto r64 = [](size_t n) { return (n + 63) / 64 * 64; };
  const size_t nlog = cfg->lm_head.data != nullptr ? cfg->vocab : 0;
  const size_t total =
      2 * r64(cfg->dim) + 2 * r64(qn) + 2 * r64(kvn) + 2 * r64(cfg->ff) + r64(nlog);
  if (hipMalloc(reinterpret_cast<void**>(&o.buf), total * sizeof(float)) != hipSuccess) {
    // the previous setup is gone with its scratch: leave no pointer into it
    o.buf = nullptr;
    o.layers.clear();
    o.logits = nullptr;
    o.cfg = dbi_offload_config{};
    if (o.owned) (void)hipFree(o.owned);
    o.owned = nullptr;
    return fail(DBI_ERR_NOMEM, "offload scratch allocation failed");
  }
  float* p = o.buf;
  o.normed = p; p += r64(cfg->dim);
  o.q = p; p += r64(qn);
  o.attn = p; p += r64(qn);
  o.k = p; p += r64(kvn);
  o.v = p; p += r64(kvn);
  o.gate = p; p += r64(cfg->ff);
  o.up = p; p += r64(cfg->ff);
  o.xrow = p; p += r64(cfg->dim);
  o.logits = nlog ? p : nullptr;
  o.cfg = *cfg;
  o.layers.assign(layers, layers + n_layers);
  if (o.owned) (void)hipFree(o.owned);
  o.owned = owned;
  return DBI_OK;
}

dbi_status dbi_offload_setup(dbi_kv* kv, const dbi_offload_config* cfg,
                             const dbi_layer_weights* layers, uint32_t n_layers) {
  return offload_setup_impl(kv, cfg, layers, n_layers, nullptr);
}

dbi_status dbi_decode_token_async(dbi_kv* kv, float* x_dev, uint32_t pos) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  return decode_token_impl(kv, x_dev, pos);
}

dbi_status dbi_decode_token_full_async(dbi_kv* kv, float* x_dev, uint32_t pos,
                                       float* logits_dev) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  const OffloadState& o = kv->off;
  if (o.cfg.lm_head.data == nullptr)
    return fail(DBI_ERR_INVALID, "decode_token_full needs an offload tail (lm_head)");
  if (logits_dev == nullptr) return fail(DBI_ERR_INVALID, "null logits");
  if (dbi_status st = decode_token_impl(kv, x_dev, pos)) return st;
  bool normed = false;
  HIP_TRY(run_matvec(kv, o.cfg.lm_head, x_dev, logits_dev, o.cfg.vocab, o.cfg.dim, false,
                     o.cfg.output_norm, &normed),
          "lm_head launch");
  return DBI_OK;
}

// ---- host-row forms (the reference's own Backend contract: setup_offload
// copies the weights to the device once, decode_token / decode_token_full
// take host rows)

dbi_status dbi_offload_setup_host(dbi_kv* kv, const dbi_offload_config* cfg,
                                  const dbi_layer_weights* layers, uint32_t n_layers) {
  if (kv == nullptr || cfg == nullptr || layers == nullptr)
    return fail(DBI_ERR_INVALID, "null offload argument");
  if (n_layers == 0 || n_layers > kv->cfg.n_layers)
    return fail(DBI_ERR_INVALID, "offload needs 1 to n_layers blocks");
  if (cfg->dim == 0 || cfg->ff == 0 || cfg->n_heads == 0 || cfg->dim > (uint32_t(1) << 20) ||
      cfg->ff > (uint32_t(1) << 20) || cfg->n_heads > 4096 ||
      (cfg->lm_head.data != nullptr && (cfg->vocab == 0 || cfg->vocab > (uint32_t(1) << 30))))
    return fail(DBI_ERR_INVALID, "offload needs dim, ff in [1, 2^20], n_heads in [1, 4096] "
                                 "and, with lm_head, vocab in [1, 2^30]");
  const size_t dim = cfg->dim, ff = cfg->ff;
  const size_t qn = size_t(cfg->n_heads) * kv->cfg.head_dim;
  const size_t kvn = size_t(kv->cfg.n_kv_heads) * kv->cfg.head_dim;
  // bytes of a [out][in] matrix of a served type (0: not served or a row
  // that is not a whole number of blocks; the device setup then reports it)
  auto wbytes = [](uint32_t type, size_t out, size_t in) -> size_t {
    switch (type) {
      case DBI_W_F32: return out * in * 4;
      case DBI_W_F16: return out * in * 2;
      case DBI_W_Q8_0: return in % 32 == 0 ? out * (in / 32) * 34 : 0;
      case DBI_W_Q4_0: return in % 32 == 0 ? out * (in / 32) * 18 : 0;
      default: return 0;
    }
  };
  struct Piece {
    const void* src;
    size_t bytes;
    std::function<void(const void*)> bind;  // stores the device address
  };
  std::vector<dbi_layer_weights> dev(layers, layers + n_layers);
  dbi_offload_config dcfg = *cfg;
  std::vector<Piece> pieces;
  auto add = [&](const void* src, size_t bytes, std::function<void(const void*)> bind,
                 const char* what, uint32_t l) -> dbi_status {
    if (src == nullptr) return DBI_OK;  // (the device setup checks what must be there)
    if (bytes == 0)
      return fail(DBI_ERR_UNSUPPORTED,
                  "offload block " + std::to_string(l) + " " + what +
                      ": the matvecs serve fp32, f16, Q8_0 and Q4_0 weights only (Q8_0 and "
                      "Q4_0 rows a multiple of 32)");
    pieces.push_back({src, bytes, std::move(bind)});
    return DBI_OK;
  };
  auto fset = [](const float** f) {
    return [f](const void* d) { *f = static_cast<const float*>(d); };
  };
  for (uint32_t l = 0; l < n_layers; ++l) {
    dbi_layer_weights& L = dev[l];
    const struct {
      dbi_weight* w;
      size_t out, in;
      const char* name;
    } ws[] = {{&L.wq, qn, dim, "wq"},      {&L.wk, kvn, dim, "wk"},   {&L.wv, kvn, dim, "wv"},
              {&L.wo, dim, qn, "wo"},      {&L.wgate, ff, dim, "wgate"},
              {&L.wup, ff, dim, "wup"},    {&L.wdown, dim, ff, "wdown"}};
    for (const auto& w : ws) {
      dbi_weight* wp = w.w;
      if (dbi_status st = add(wp->data, wbytes(wp->type, w.out, w.in),
                              [wp](const void* d) { wp->data = d; }, w.name, l))
        return st;
    }
    (void)add(L.attn_norm, dim * 4, fset(&L.attn_norm), "attn_norm", l);
    (void)add(L.ffn_norm, dim * 4, fset(&L.ffn_norm), "ffn_norm", l);
    (void)add(L.bq, qn * 4, fset(&L.bq), "bq", l);
    (void)add(L.bk, kvn * 4, fset(&L.bk), "bk", l);
    (void)add(L.bv, kvn * 4, fset(&L.bv), "bv", l);
  }
  if (cfg->lm_head.data != nullptr) {
    if (dbi_status st = add(cfg->lm_head.data, wbytes(cfg->lm_head.type, cfg->vocab, dim),
                            [&dcfg](const void* d) { dcfg.lm_head.data = d; }, "lm_head", 0))
      return st;
    (void)add(cfg->output_norm, dim * 4, fset(&dcfg.output_norm), "output_norm", 0);
  }
  if (dbi_status st = refuse_capture(kv, "the offload weights")) return st;
  // one device allocation, every piece 256-byte aligned
  size_t total = 0;
  for (const Piece& pc : pieces) total += (pc.bytes + 255) / 256 * 256;
  uint8_t* base = nullptr;
  if (total > 0 && hipMalloc(reinterpret_cast<void**>(&base), total) != hipSuccess)
    return fail(DBI_ERR_NOMEM, "offload weight allocation failed (" + std::to_string(total) +
                                   " bytes)");
  size_t at = 0;
  for (const Piece& pc : pieces) {
    const hipError_t e = hipMemcpy(base + at, pc.src, pc.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(base);
      return hip_fail(e, "offload weight upload");
    }
    pc.bind(base + at);
    at += (pc.bytes + 255) / 256 * 256;
  }
  const dbi_status st = offload_setup_impl(kv, &dcfg, dev.data(), n_layers, base);
  if (st != DBI_OK) (void)hipFree(base);
  return st;
}

dbi_status dbi_decode_token(dbi_kv* kv, float* x, uint32_t pos) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  const OffloadState& o = kv->off;
  if (o.layers.empty()) return fail(DBI_ERR_INVALID, "decode_token needs dbi_offload_setup first");
  if (x == nullptr) return fail(DBI_ERR_INVALID, "null residual row");
  const size_t bytes = size_t(o.cfg.dim) * sizeof(float);
  HIP_TRY(hipMemcpyAsync(o.xrow, x, bytes, hipMemcpyHostToDevice, kv->stream), "x upload");
  if (dbi_status st = decode_token_impl(kv, o.xrow, pos)) {
    (void)hipStreamSynchronize(kv->stream);  // the upload reads the caller's row
    return st;
  }
  HIP_TRY(hipMemcpyAsync(x, o.xrow, bytes, hipMemcpyDeviceToHost, kv->stream), "x readback");
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  return DBI_OK;
}

dbi_status dbi_decode_token_full(dbi_kv* kv, const float* x, uint32_t pos, float* logits) {
  if (kv == nullptr) return fail(DBI_ERR_INVALID, "null handle");
  const OffloadState& o = kv->off;
  if (o.cfg.lm_head.data == nullptr || o.logits == nullptr)
    return fail(DBI_ERR_INVALID, "decode_token_full needs an offload tail (lm_head)");
  if (x == nullptr || logits == nullptr) return fail(DBI_ERR_INVALID, "null row");
  HIP_TRY(hipMemcpyAsync(o.xrow, x, size_t(o.cfg.dim) * sizeof(float), hipMemcpyHostToDevice,
                         kv->stream),
          "x upload");
  if (dbi_status st = dbi_decode_token_full_async(kv, o.xrow, pos, o.logits)) {
    (void)hipStreamSynchronize(kv->stream);
    return st;
  }
  HIP_TRY(hipMemcpyAsync(logits, o.logits, size_t(o.cfg.vocab) * sizeof(float),
                         hipMemcpyDeviceToHost, kv->stream),
          "logits readback");
  HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
  return DBI_OK;
}

}  // extern "C"
