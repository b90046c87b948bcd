// C++ parity tests of the MI355X KV cache through the engine-facing host
// layer (dbinfer_amd/host), written like the reference's own ctest mains:
//   kv_ring_test.cpp:26-97        ring slots, residents, sinks, rope packing
//   kv_int8_test.cpp:33-137       per-channel K round trip, int8 vs fp32 attention
//   kv_prefix_cache_test.cpp:79-130  save -> load -> identical next attention
//   chunked_prefill_test.cpp:19-70   chunk == per-token (here within tolerance)
//   speculative_test.cpp:104-150     merge vectors, rollback state
// the Backend offload seam (backend.hpp:133-157) through backend.hpp, token
// by token against the oracle's decode_layer and logits,
// plus decode/chunk parity against the CPU oracle (oracle/kv_oracle.h), which
// is the checker only. `host_test --cpu-only` runs the parts that need no GPU.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "backend.hpp"
#include "kv_cache.hpp"
#include "kv_oracle.h"
#include "layer.hpp"

namespace {

using dbinfer_amd::model::Config;
using dbinfer_amd::model::KVCache;
using dbinfer_amd::model::KvDtype;
using dbinfer_amd::model::KvPolicy;

int g_failures = 0;

void check(bool ok, const std::string& what) {
  std::printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
  if (!ok) ++g_failures;
}

struct Lcg {  // kv_int8_test.cpp:24-31
  std::uint64_t s;
  float next() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    const auto hi = static_cast<std::uint32_t>(s >> 32);
    return static_cast<float>(hi) / 2147483648.0f - 1.0f;
  }
};

bool close(const std::vector<float>& got, const std::vector<float>& want, double* worst) {
  double w = 0.0;
  bool ok = got.size() == want.size();
  for (std::size_t i = 0; ok && i < got.size(); ++i) {
    const double err = std::fabs(static_cast<double>(got[i]) - want[i]);
    const double bound = 1e-5 + 1e-4 * std::fabs(static_cast<double>(want[i]));
    w = std::max(w, err / bound);
    ok = ok && err <= bound;
  }
  if (worst) *worst = w;
  return ok;
}

// ---------------------------------------------------------------- CPU only

void test_speculative_merge() {
  using dbinfer_amd::model::speculative_merge;
  {
    const std::int32_t d[3] = {10, 20, 30}, t[4] = {10, 20, 30, 40};
    std::vector<std::int32_t> out;
    const std::size_t a = speculative_merge({d, 3}, {t, 4}, out);
    check(a == 3 && out == std::vector<std::int32_t>{10, 20, 30, 40}, "merge all-accept emits bonus");
  }
  {
    const std::int32_t d[3] = {10, 99, 30}, t[4] = {10, 20, 30, 40};
    std::vector<std::int32_t> out;
    const std::size_t a = speculative_merge({d, 3}, {t, 4}, out);
    check(a == 1 && out == std::vector<std::int32_t>{10, 20}, "merge reject-at-1 emits correction");
  }
  {
    const std::int32_t d[2] = {5, 6}, t[3] = {9, 8, 7};
    std::vector<std::int32_t> out;
    const std::size_t a = speculative_merge({d, 2}, {t, 3}, out);
    check(a == 0 && out == std::vector<std::int32_t>{9}, "merge reject-at-0 emits target argmax");
  }
}

void test_rope_matches_oracle() {
  const std::size_t heads = 3, hd = 128;
  const std::int32_t pos[2] = {7, 32767};
  Lcg rng{0x5EED};
  std::vector<float> a(heads * 2 * hd);
  for (auto& x : a) x = rng.next();
  std::vector<float> b = a;
  dbinfer_amd::model::rope(a.data(), pos, 1e6f, heads, 2, hd);
  ok_rope(b.data(), pos, 1e6f, heads, 2, hd);
  check(std::memcmp(a.data(), b.data(), a.size() * 4) == 0, "host rope bitwise == oracle rope");
}

// ---------------------------------------------------------------- GPU

void test_ring_case(std::size_t n_sink, std::size_t window, std::size_t n_seen) {
  KVCache kv(1, 0, 1, 1, KvPolicy{n_sink, window, KvDtype::F32}, 1e6f);
  bool slots_ok = true;
  for (std::size_t t = 0; t < n_seen; ++t) {
    const float payload = static_cast<float>(t);
    const std::size_t want = t < n_sink ? t : n_sink + (t - n_sink) % window;
    slots_ok = slots_ok && kv.slot_for(t) == want;
    kv.append(0, t, &payload, &payload);
  }
  char name[160];
  std::snprintf(name, sizeof name, "(sink=%zu win=%zu seen=%zu)", n_sink, window, n_seen);
  check(kv.ok() && slots_ok, std::string("slot_for matches reference ") + name);
  std::vector<KVCache::Resident> res(kv.capacity());
  const std::size_t n_res = kv.residents(res.data());
  const std::vector<float> keys = kv.export_f32(DBI_EXPORT_K, 0);
  const std::size_t sinks = std::min(n_seen, n_sink);
  std::size_t ws = n_sink;
  if (n_seen > n_sink && n_seen - n_sink > window) ws = n_seen - window;
  const std::size_t wlen = n_seen > n_sink ? n_seen - ws : 0;
  check(n_res == sinks + wlen, std::string("n_res == sinks+window ") + name);
  bool pinned = true, recent = true, packed = true;
  for (std::size_t r = 0; r < sinks; ++r)
    pinned = pinned && res[r].slot == r && keys[res[r].slot] == static_cast<float>(r);
  for (std::size_t r = sinks; r < n_res; ++r)
    recent = recent && keys[res[r].slot] == static_cast<float>(ws + (r - sinks));
  std::vector<std::size_t> slots;
  for (std::size_t r = 0; r < n_res; ++r) {
    packed = packed && res[r].rope_pos == static_cast<std::int32_t>(r);
    slots.push_back(res[r].slot);
  }
  std::sort(slots.begin(), slots.end());
  check(pinned, std::string("sinks never evicted ") + name);
  check(recent, std::string("window holds most recent tokens ") + name);
  check(packed, std::string("rope positions pack to [0,n_res) ") + name);
  check(std::adjacent_find(slots.begin(), slots.end()) == slots.end(),
        std::string("resident slots are distinct ") + name);
}

void test_int8_roundtrip() {
  const std::size_t nkv = 3, hd = 40, slots = 5;
  Lcg rng{0xC0FFEE};
  KVCache kv(1, slots, nkv, hd, KvPolicy{0, 0, KvDtype::Int8});
  std::vector<float> k(nkv * hd), v(nkv * hd);
  bool ok = true;
  for (std::size_t s = 0; s < slots; ++s) {
    for (auto& x : k) x = rng.next() * 7.0f;
    for (auto& x : v) x = rng.next() * 0.03f;
    kv.append(0, s, k.data(), v.data());
    const auto k8 = kv.export_i8(DBI_EXPORT_K8, 0);
    const auto ks = kv.export_f32(DBI_EXPORT_K_SCALE, 0);
    for (std::size_t h = 0; h < nkv; ++h)
      for (std::size_t i = 0; i < hd; ++i) {
        const float sc = ks[(s / 32 * nkv + h) * hd + i];
        const float err = std::fabs(k[h * hd + i] - sc * static_cast<float>(k8[(s * nkv + h) * hd + i]));
        ok = ok && err <= sc + 1e-6f;
      }
  }
  check(kv.ok() && ok, "per-channel key quant/dequant error within one scale step");
}

void test_int8_attention_vs_fp32() {
  const std::size_t hd = 64, keys = 48;
  Lcg rng{0x1357};
  std::vector<float> q(hd), k(keys * hd), v(keys * hd);
  for (auto& x : q) x = rng.next();
  for (auto& x : k) x = rng.next();
  for (auto& x : v) x = rng.next();
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  KVCache f(1, keys, 1, hd), i8(1, keys, 1, hd, KvPolicy{0, 0, KvDtype::Int8});
  f.append_n(0, 0, keys, k.data(), v.data());
  i8.append_n(0, 0, keys, k.data(), v.data());
  std::vector<float> ref(hd), got(hd);
  f.check(dbi_attn_decode(f.handle(), 0, keys - 1, 1, scale, q.data(), ref.data()));
  i8.check(dbi_attn_decode(i8.handle(), 0, keys - 1, 1, scale, q.data(), got.data()));
  double num = 0, den = 0;
  for (std::size_t j = 0; j < hd; ++j) {
    num += (got[j] - ref[j]) * (got[j] - ref[j]);
    den += ref[j] * ref[j];
  }
  const double rel = std::sqrt(num / den);
  std::printf("int8 attention relative L2 = %.5f\n", rel);
  check(f.ok() && i8.ok() && rel <= 0.006, "int8 attention within 0.6% relative L2 of fp32");
}

// decode_layer's attention half on the device vs the oracle's reference flow
void test_decode_layer_parity(KvPolicy pol, const Config& cfg, std::size_t layers,
                              std::size_t steps, const char* name) {
  const std::size_t cap = pol.window ? 0 : steps + 1;
  KVCache kv(layers, cap, cfg.n_kv_heads, cfg.head_dim, pol, cfg.rope_theta);
  okv* o = okv_create(layers, cap, cfg.n_kv_heads, cfg.head_dim, pol.n_sink, pol.window,
                      pol.dtype == KvDtype::Int8 ? OKV_INT8 : OKV_F32);
  const std::size_t qn = cfg.n_heads * cfg.head_dim, kn = cfg.n_kv_heads * cfg.head_dim;
  const float scale = 1.0f / std::sqrt(static_cast<float>(cfg.head_dim));
  Lcg rng{0xABC + steps};
  bool ok = kv.ok();
  double worst = 0;
  for (std::size_t t = 0; t < steps && ok; ++t) {
    for (std::size_t l = 0; l < layers && ok; ++l) {
      std::vector<float> q(qn), k(kn), v(kn), out(qn), want(qn);
      for (auto& x : q) x = rng.next();
      for (auto& x : k) x = rng.next();
      for (auto& x : v) x = rng.next();
      std::vector<float> q0 = q, k0 = k;  // un-roped copies for the oracle
      const auto pos = static_cast<std::int32_t>(t);
      ok = dbinfer_amd::model::decode_attention(kv, cfg, l, pos, q.data(), k.data(), v.data(),
                                                out.data());
      if (pol.window) {
        okv_attend_ring(o, l, t, cfg.n_heads, scale, cfg.rope_theta, q0.data(), k0.data(),
                        v.data(), want.data(), 1);
      } else {
        ok_rope(q0.data(), &pos, cfg.rope_theta, cfg.n_heads, 1, cfg.head_dim);
        ok_rope(k0.data(), &pos, cfg.rope_theta, cfg.n_kv_heads, 1, cfg.head_dim);
        okv_append(o, l, t, k0.data(), v.data());
        if (pol.dtype == KvDtype::Int8)
          okv_attend_dense_int8(o, l, t, cfg.n_heads, scale, q0.data(), want.data(), 1);
        else
          okv_attend_dense_f32(o, l, t, cfg.n_heads, scale, q0.data(), want.data(), 1);
      }
      double w = 0;
      ok = ok && close(out, want, &w);
      worst = std::max(worst, w);
    }
  }
  std::printf("  %s worst err/bound %.3f\n", name, worst);
  check(ok, std::string("decode_layer attention parity: ") + name);
  okv_destroy(o);
}

// chunk attention (append all, then causal rows) vs the oracle chunk, and vs
// per-token decode on a second cache
void test_chunk_parity(KvDtype dt) {
  const Config cfg{32, 8, 64, 5e5f};
  const std::size_t pos0 = 40, n = 24, cap = 80;
  KVCache kv(1, cap, cfg.n_kv_heads, cfg.head_dim, KvPolicy{4, 0, dt});
  KVCache tok(1, cap, cfg.n_kv_heads, cfg.head_dim, KvPolicy{4, 0, dt});
  okv* o = okv_create(1, cap, cfg.n_kv_heads, cfg.head_dim, 4, 0,
                      dt == KvDtype::Int8 ? OKV_INT8 : OKV_F32);
  const std::size_t qn = cfg.n_heads * cfg.head_dim, kn = cfg.n_kv_heads * cfg.head_dim;
  Lcg rng{0x77};
  std::vector<float> pk(pos0 * kn), pv(pos0 * kn);
  for (auto& x : pk) x = rng.next();
  for (auto& x : pv) x = rng.next();
  kv.append_n(0, 0, pos0, pk.data(), pv.data());
  tok.append_n(0, 0, pos0, pk.data(), pv.data());
  for (std::size_t p = 0; p < pos0; ++p) okv_append(o, 0, p, pk.data() + p * kn, pv.data() + p * kn);
  std::vector<float> q(n * qn), k(n * kn), v(n * kn), out(n * qn), want(n * qn);
  for (auto& x : q) x = rng.next();
  for (auto& x : k) x = rng.next();
  for (auto& x : v) x = rng.next();
  std::vector<float> q0 = q, k0 = k, q1 = q, k1 = k;
  dbinfer_amd::model::chunk_attention(kv, cfg, 0, pos0, n, q.data(), k.data(), v.data(), out.data());
  for (std::size_t c = 0; c < n; ++c) {
    const auto p = static_cast<std::int32_t>(pos0 + c);
    ok_rope(q0.data() + c * qn, &p, cfg.rope_theta, cfg.n_heads, 1, cfg.head_dim);
    ok_rope(k0.data() + c * kn, &p, cfg.rope_theta, cfg.n_kv_heads, 1, cfg.head_dim);
    okv_append(o, 0, pos0 + c, k0.data() + c * kn, v.data() + c * kn);
  }
  okv_attend_chunk(o, 0, pos0, n, cfg.n_heads, 1.0f / 8.0f, q0.data(), want.data(), 1);
  double w = 0;
  const bool ok_oracle = kv.ok() && close(out, want, &w);
  // per-token decode on the second cache (fp32: the chunk's rows see the
  // same keys; int8: a row attends the cache as it stands after all n
  // appends, so per-token decode differs by design and is not compared)
  bool ok_tok = true;
  if (dt == KvDtype::F32) {
    for (std::size_t c = 0; c < n; ++c) {
      std::vector<float> row(qn);
      dbinfer_amd::model::decode_attention(tok, cfg, 0, static_cast<std::int32_t>(pos0 + c),
                                           q1.data() + c * qn, k1.data() + c * kn,
                                           v.data() + c * kn, row.data());
      std::vector<float> ch(out.begin() + c * qn, out.begin() + (c + 1) * qn);
      ok_tok = ok_tok && close(row, ch, nullptr);
    }
  }
  check(ok_oracle, std::string("chunk attention parity vs oracle ") +
                       (dt == KvDtype::Int8 ? "int8" : "fp32"));
  check(ok_tok, std::string("chunk rows == per-token decode ") +
                    (dt == KvDtype::Int8 ? "int8" : "fp32"));
  okv_destroy(o);
}

// decode_layer / decode_layer_chunk from the raw projections with biases
// (model.cpp:747-755, 935-953): the device producer against the host flow
// (bias adds, rope, then decode_attention / chunk_attention) on a second
// cache; outputs bitwise equal, since the device rope reproduces the host's
void test_producer_parity(KvPolicy pol, const Config& cfg, std::size_t steps, const char* name) {
  const std::size_t cap = pol.window ? 0 : steps + 8;
  KVCache dev(1, cap, cfg.n_kv_heads, cfg.head_dim, pol, cfg.rope_theta);
  KVCache host(1, cap, cfg.n_kv_heads, cfg.head_dim, pol, cfg.rope_theta);
  const std::size_t qn = cfg.n_heads * cfg.head_dim, kn = cfg.n_kv_heads * cfg.head_dim;
  Lcg rng{0xB1A5 + steps};
  std::vector<float> qb(qn), kb(kn), vb(kn);
  for (auto& x : qb) x = rng.next();
  for (auto& x : kb) x = rng.next();
  for (auto& x : vb) x = rng.next();
  const dbinfer_amd::model::AttnBias bias{qb.data(), kb.data(), vb.data()};
  auto biased = [](std::vector<float> x, const std::vector<float>& b) {
    for (std::size_t i = 0; i < x.size(); ++i) x[i] += b[i % b.size()];
    return x;
  };
  bool ok = dev.ok() && host.ok(), same = true;
  for (std::size_t t = 0; t < steps && ok; ++t) {
    std::vector<float> q(qn), k(kn), v(kn), oa(qn), ob(qn);
    for (auto& x : q) x = rng.next();
    for (auto& x : k) x = rng.next();
    for (auto& x : v) x = rng.next();
    const auto pos = static_cast<std::int32_t>(t);
    ok = dbinfer_amd::model::decode_attention_qkv(dev, cfg, 0, pos, q.data(), k.data(), v.data(),
                                                  bias, oa.data());
    std::vector<float> q1 = biased(q, qb), k1 = biased(k, kb), v1 = biased(v, vb);
    ok = ok && dbinfer_amd::model::decode_attention(host, cfg, 0, pos, q1.data(), k1.data(),
                                                    v1.data(), ob.data());
    same = same && std::memcmp(oa.data(), ob.data(), qn * 4) == 0;
  }
  if (!pol.window && ok) {  // one chunk after the decode steps
    const std::size_t n = 6, pos0 = steps;
    std::vector<float> q(n * qn), k(n * kn), v(n * kn), oa(n * qn), ob(n * qn);
    for (auto& x : q) x = rng.next();
    for (auto& x : k) x = rng.next();
    for (auto& x : v) x = rng.next();
    ok = dbinfer_amd::model::chunk_attention_qkv(dev, cfg, 0, static_cast<std::int32_t>(pos0), n,
                                                 q.data(), k.data(), v.data(), bias, oa.data());
    std::vector<float> q1 = biased(q, qb), k1 = biased(k, kb), v1 = biased(v, vb);
    ok = ok && dbinfer_amd::model::chunk_attention(host, cfg, 0, static_cast<std::int32_t>(pos0),
                                                   n, q1.data(), k1.data(), v1.data(), ob.data());
    same = same && std::memcmp(oa.data(), ob.data(), n * qn * 4) == 0;
  }
  check(ok && same, std::string("q/k/v producer == host bias + rope flow (bitwise): ") + name);
}

void test_prefix_cache() {
  const Config cfg{14, 2, 64, 1e6f};
  const std::size_t L = 3, cap = 64, n = 20;
  const std::vector<std::int32_t> prompt = {40, 1079, 264, 4128, 1614, 13, 7, 7, 9, 11,
                                            12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22};
  KVCache a(L, cap, cfg.n_kv_heads, cfg.head_dim), b(L, cap, cfg.n_kv_heads, cfg.head_dim);
  const std::size_t qn = cfg.n_heads * cfg.head_dim, kn = cfg.n_kv_heads * cfg.head_dim;
  Lcg rng{0x9797};
  std::vector<float> k(n * kn), v(n * kn);
  for (auto& x : k) x = rng.next();
  for (auto& x : v) x = rng.next();
  for (std::size_t l = 0; l < L; ++l) a.append_n(l, 0, n, k.data(), v.data());
  const std::string path = "/tmp/dbi_host_test_prefix.kv";
  auto saved = dbinfer_amd::model::save_kv_prefix(a, path, {prompt.data(), n});
  check(static_cast<bool>(saved), "save_kv_prefix succeeds");
  auto loaded = dbinfer_amd::model::load_kv_prefix(b, path, {prompt.data(), prompt.size()});
  check(loaded && *loaded == n && b.n_seen() == n, "load_kv_prefix restores length");
  // next token's attention after resume is bitwise equal (kv_prefix_cache_test.cpp:90-130)
  std::vector<float> q(qn), kk(kn), vv(kn);
  for (auto& x : q) x = rng.next();
  for (auto& x : kk) x = rng.next();
  for (auto& x : vv) x = rng.next();
  bool same = true;
  for (std::size_t l = 0; l < L; ++l) {
    std::vector<float> qa = q, qb = q, ka = kk, kb = kk, oa(qn), ob(qn);
    dbinfer_amd::model::decode_attention(a, cfg, l, n, qa.data(), ka.data(), vv.data(), oa.data());
    dbinfer_amd::model::decode_attention(b, cfg, l, n, qb.data(), kb.data(), vv.data(), ob.data());
    same = same && std::memcmp(oa.data(), ob.data(), qn * 4) == 0;
  }
  check(a.ok() && b.ok() && same, "resumed cache: next-token attention bitwise equal");
  auto missing = dbinfer_amd::model::load_kv_prefix(b, "/tmp/does/not/exist.kv",
                                                    {prompt.data(), prompt.size()});
  check(!missing && missing.error().message.rfind("cannot open kv prefix cache", 0) == 0,
        "missing prefix file is an error");
  std::remove(path.c_str());
}

void test_speculative_rollback() {
  // verify round: append [last, d1..d4] at pos, attend, accept a, commit;
  // the next round's attention equals a cache that only ever saw the
  // accepted rows (stale rejected rows are beyond n_seen and never read)
  const Config cfg{32, 8, 128, 1e6f};
  const std::size_t cap = 64, pos = 30, k = 4, accepted = 2;
  const std::size_t qn = cfg.n_heads * cfg.head_dim, kn = cfg.n_kv_heads * cfg.head_dim;
  KVCache spec(1, cap, cfg.n_kv_heads, cfg.head_dim), ref(1, cap, cfg.n_kv_heads, cfg.head_dim);
  Lcg rng{0x5150};
  std::vector<float> pk(pos * kn), pv(pos * kn);
  for (auto& x : pk) x = rng.next();
  for (auto& x : pv) x = rng.next();
  spec.append_n(0, 0, pos, pk.data(), pv.data());
  ref.append_n(0, 0, pos, pk.data(), pv.data());
  std::vector<float> q((k + 1) * qn), kk((k + 1) * kn), vv((k + 1) * kn), out((k + 1) * qn);
  for (auto& x : q) x = rng.next();
  for (auto& x : kk) x = rng.next();
  for (auto& x : vv) x = rng.next();
  std::vector<float> kref = kk;
  dbinfer_amd::model::chunk_attention(spec, cfg, 0, pos, k + 1, q.data(), kk.data(), vv.data(),
                                      out.data());
  const std::int32_t next = dbinfer_amd::model::speculative_commit(spec, pos, accepted);
  check(next == static_cast<std::int32_t>(pos + accepted + 1) && spec.n_seen() == pos + accepted + 1,
        "rollback keeps pos + accepted + 1 positions");
  // ref: the same rows, roped the same way, but only the accepted ones
  for (std::size_t c = 0; c <= accepted; ++c) {
    const auto p = static_cast<std::int32_t>(pos + c);
    dbinfer_amd::model::rope(kref.data() + c * kn, &p, cfg.rope_theta, cfg.n_kv_heads, 1,
                             cfg.head_dim);
  }
  ref.append_n(0, pos, accepted + 1, kref.data(), vv.data());
  std::vector<float> qn1(qn), kn1(kn), vn1(kn);
  for (auto& x : qn1) x = rng.next();
  for (auto& x : kn1) x = rng.next();
  for (auto& x : vn1) x = rng.next();
  std::vector<float> qa = qn1, qb = qn1, ka = kn1, kb = kn1, oa(qn), ob(qn);
  dbinfer_amd::model::decode_attention(spec, cfg, 0, next, qa.data(), ka.data(), vn1.data(), oa.data());
  dbinfer_amd::model::decode_attention(ref, cfg, 0, next, qb.data(), kb.data(), vn1.data(), ob.data());
  check(spec.ok() && ref.ok() && std::memcmp(oa.data(), ob.data(), qn * 4) == 0,
        "next round after rollback == cache without the rejected rows (bitwise)");
}

void test_speculative_verify() {
  // a verify round's tokens on the device: argmax of the k+1 logit rows
  // (ties planted), merge against a draft that diverges at 2, then commit
  const std::size_t cap = 64, pos = 30, k = 4, vocab = 50000, kn = 2 * 64;
  KVCache kv(1, cap, 2, 64);
  Lcg rng{0x7e57};
  std::vector<float> kk((pos + k + 1) * kn), vv((pos + k + 1) * kn);
  for (auto& x : kk) x = rng.next();
  for (auto& x : vv) x = rng.next();
  kv.append_n(0, 0, pos + k + 1, kk.data(), vv.data());
  std::vector<float> logits((k + 1) * vocab);
  for (auto& x : logits) x = rng.next();
  std::vector<std::int32_t> want(k + 1);
  for (std::size_t r = 0; r <= k; ++r) {
    logits[r * vocab + 4000 + r] = 3.0f;  // tied maximum: the earlier index wins
    logits[r * vocab + 30000 + r] = 3.0f;
    want[r] = ok_argmax(logits.data() + r * vocab, vocab);
  }
  const std::vector<std::int32_t> draft = {want[0], want[1], want[2] + 1, want[3]};
  std::vector<std::int32_t> out(k + 1);
  std::size_t n_out = 0;
  const std::size_t acc = ok_spec_merge(draft.data(), k, want.data(), out.data(), &n_out);
  out.resize(n_out);
  float* d = nullptr;
  const bool dev = hipMalloc(reinterpret_cast<void**>(&d), logits.size() * sizeof(float)) ==
                       hipSuccess &&
                   hipMemcpy(d, logits.data(), logits.size() * sizeof(float),
                             hipMemcpyHostToDevice) == hipSuccess;
  check(dev, "verify: device logits");
  if (!dev) return;
  std::vector<std::int32_t> merged;
  const auto r = dbinfer_amd::model::speculative_verify(kv, static_cast<std::int32_t>(pos), vocab,
                                                        d, draft, merged);
  check(want[0] == 4000 && acc == 2, "verify: oracle argmax keeps the first of a tie");
  check(r && *r == acc && merged == out && kv.n_seen() == pos + acc + 1,
        "verify: device argmax + merge == oracle, cache keeps pos + accepted + 1");
  const auto e = dbinfer_amd::model::speculative_verify(kv, static_cast<std::int32_t>(pos), vocab,
                                                        d, draft, merged);
  check(!e && merged.empty() && kv.n_seen() == pos + acc + 1,
        "verify: a round whose rows are not in the cache is refused, cache unchanged");
  (void)hipFree(d);
}

void test_output_projection() {
  // x += W_o · attn on the device for fp32, f16 and Q8_0 weights; integer
  // data (Q8_0: unit block scales, activation blocks whose max is 127) keeps
  // every partial sum exact, so the device equals the oracle bit for bit
  const std::size_t dim = 64, in = 256, nb = in / 32;
  KVCache kv(1, 16, 1, 64);
  Lcg rng{0x0b0e};
  auto small = [&](int range) {
    return static_cast<float>(static_cast<int>((rng.next() + 1.0f) * 0.5f * (2 * range + 1)) - range);
  };
  std::vector<float> attn(in), x(dim), wf(dim * in);
  for (std::size_t i = 0; i < in; ++i) attn[i] = i % 32 == 0 ? 127.0f : small(127);
  for (auto& v : x) v = small(100);
  for (auto& v : wf) v = small(8);
  std::vector<std::uint16_t> wh(dim * in);
  for (std::size_t i = 0; i < wf.size(); ++i) wh[i] = ok_f32_to_f16(wf[i]);
  std::vector<std::uint8_t> wq(dim * nb * 34);
  const std::uint16_t one = ok_f32_to_f16(1.0f);
  for (std::size_t o = 0; o < dim; ++o)
    for (std::size_t b = 0; b < nb; ++b) {
      std::uint8_t* blk = wq.data() + (o * nb + b) * 34;
      std::memcpy(blk, &one, 2);
      for (int i = 0; i < 32; ++i)
        blk[2 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(wf[o * in + b * 32 + i]));
    }
  struct Case {
    std::uint32_t wtype;
    int oracle_type;
    const void* host;
    std::size_t bytes;
    const char* name;
  } cases[] = {{DBI_W_F32, 0, wf.data(), wf.size() * 4, "fp32"},
               {DBI_W_F16, 1, wh.data(), wh.size() * 2, "f16"},
               {DBI_W_Q8_0, 8, wq.data(), wq.size(), "Q8_0"}};
  void *dw = nullptr, *da = nullptr, *dx = nullptr;
  bool ok = hipMalloc(&dw, wf.size() * 4) == hipSuccess && hipMalloc(&da, in * 4) == hipSuccess &&
            hipMalloc(&dx, dim * 4) == hipSuccess &&
            hipMemcpy(da, attn.data(), in * 4, hipMemcpyHostToDevice) == hipSuccess;
  check(ok, "output projection: device buffers");
  for (const Case& c : cases) {
    if (!ok) break;
    std::vector<float> want = x, got(dim);
    ok_oproj_residual(c.host, c.oracle_type, attn.data(), want.data(), dim, in);
    const bool up = hipMemcpy(dw, c.host, c.bytes, hipMemcpyHostToDevice) == hipSuccess &&
                    hipMemcpy(dx, x.data(), dim * 4, hipMemcpyHostToDevice) == hipSuccess;
    const bool ran = up && dbinfer_amd::model::output_projection(
                               kv, c.wtype, dw, static_cast<const float*>(da),
                               static_cast<float*>(dx), dim, in);
    const bool back = ran && dbi_kv_sync(kv.handle()) == DBI_OK &&
                      hipMemcpy(got.data(), dx, dim * 4, hipMemcpyDeviceToHost) == hipSuccess;
    check(back && std::memcmp(got.data(), want.data(), dim * 4) == 0,
          std::string("output projection ") + c.name + ": device == oracle (bitwise)");
  }
  check(!dbinfer_amd::model::output_projection(kv, 5, dw, static_cast<const float*>(da),
                                               static_cast<float*>(dx), dim, in),
        "output projection: an unserved weight type is refused");
  (void)hipFree(dw);
  (void)hipFree(da);
  (void)hipFree(dx);
}

}  // namespace

// The offload seam (Backend::setup_offload / decode_token /
// decode_token_full, backend.hpp:133-157) through the C++ mirror, token by
// token against the oracle's Model::decode_layer (okv_decode_layer) and
// forward's tail (ok_logits). Host weights, copied once by setup_offload.
// Q8_0 blocks: random codes and f16 scales written as bit patterns
// 2^(e-15) (1 + m/1024), e in {3, 4} (scales ~2.4e-4 .. 9.8e-4); f16
// weights: random signs and mantissas at e in {9, 10} (|w| in [0.016, 0.06]).
// Tolerance: fp32 sums in trees (1e-5 + 1e-4 |b|); for Q8_0 an activation
// code can flip at a rounding boundary (1e-2 (1 + |b|), as test_gpu_layer.py
// derives).
void test_offload(bool q8) {
  namespace be = dbinfer_amd::backend;
  constexpr std::size_t D = 256, FF = 512, NH = 4, NKV = 2, HD = 64, NL = 2, V = 300, CAP = 8;
  constexpr float EPS = 1e-5f, THETA = 1e4f;
  Lcg rng{q8 ? 0x51u : 0x52u};
  auto u32 = [&]() {
    return static_cast<std::uint32_t>((rng.next() + 1.0f) * 1048576.0f);
  };
  auto mat = [&](std::size_t out, std::size_t in) {
    std::vector<std::uint8_t> m;
    if (q8) {
      m.resize(out * (in / 32) * 34);
      for (std::size_t b = 0; b < out * (in / 32); ++b) {
        const std::uint16_t h = static_cast<std::uint16_t>(((3 + (u32() & 1)) << 10) | (u32() & 1023));
        std::memcpy(&m[b * 34], &h, 2);
        for (int i = 0; i < 32; ++i)
          m[b * 34 + 2 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(
              static_cast<int>(u32() % 255) - 127));
      }
    } else {
      m.resize(out * in * 2);
      for (std::size_t i = 0; i < out * in; ++i) {
        const std::uint16_t h = static_cast<std::uint16_t>(
            ((u32() & 1) << 15) | ((9 + (u32() & 1)) << 10) | (u32() & 1023));
        std::memcpy(&m[i * 2], &h, 2);
      }
    }
    return m;
  };
  auto vec = [&](std::size_t n, float base, float amp) {
    std::vector<float> v(n);
    for (auto& x : v) x = base + amp * rng.next();
    return v;
  };
  const std::size_t qn = NH * HD, kvn = NKV * HD;
  struct Block {
    std::vector<float> an, fn, bq, bk, bv;
    std::vector<std::uint8_t> w[7];
  };
  std::vector<Block> blk(NL);
  const std::size_t shapes[7][2] = {{qn, D}, {kvn, D}, {kvn, D}, {D, qn}, {FF, D}, {FF, D}, {D, FF}};
  const be::WeightType wt = q8 ? be::WeightType::Q8_0 : be::WeightType::F16;
  const int owt = q8 ? 8 : 1;  // GGUF type ids (oracle)
  std::vector<be::LayerQ> lq(NL);
  std::vector<ok_layer> ol(NL);
  for (std::size_t l = 0; l < NL; ++l) {
    Block& b = blk[l];
    b.an = vec(D, 1.0f, 0.1f);
    b.fn = vec(D, 1.0f, 0.1f);
    b.bq = vec(qn, 0.0f, 0.1f);
    b.bk = vec(kvn, 0.0f, 0.1f);
    b.bv = vec(kvn, 0.0f, 0.1f);
    for (int i = 0; i < 7; ++i) b.w[i] = mat(shapes[i][0], shapes[i][1]);
    auto qw = [&](int i) { return be::QWeight{reinterpret_cast<const std::byte*>(b.w[i].data()), wt}; };
    lq[l] = be::LayerQ{b.an.data(), b.fn.data(), qw(0), qw(1), qw(2), qw(3), qw(4), qw(5), qw(6),
                       b.bq.data(), b.bk.data(), b.bv.data(), D, FF, NH, NKV, HD, EPS, THETA};
    ol[l].attn_norm = b.an.data();
    ol[l].ffn_norm = b.fn.data();
    for (int i = 0; i < 7; ++i) {
      ol[l].w[i] = b.w[i].data();
      ol[l].wtype[i] = owt;
    }
    ol[l].bq = b.bq.data();
    ol[l].bk = b.bk.data();
    ol[l].bv = b.bv.data();
  }
  const std::vector<float> onorm = vec(D, 1.0f, 0.1f);
  const std::vector<std::uint8_t> lm = mat(V, D);
  const char* name = q8 ? "Q8_0" : "f16";
  auto within = [&](const float* got, const std::vector<float>& want, double* worst) {
    bool ok = true;
    for (std::size_t i = 0; i < want.size(); ++i) {
      const double b = std::fabs(static_cast<double>(want[i]));
      const double bound = q8 ? 1e-2 * (1.0 + b) : 1e-5 + 1e-4 * b;
      const double err = std::fabs(static_cast<double>(got[i]) - want[i]);
      *worst = std::max(*worst, err / bound);
      ok = ok && err <= bound;
    }
    return ok;
  };
  // decode_token on one cache, decode_token_full on another (each token
  // appends at pos)
  KVCache kv(NL, CAP, NKV, HD, {}, THETA), kv2(NL, CAP, NKV, HD, {}, THETA);
  be::HipBackend b1(kv), b2(kv2);
  auto s1 = b1.setup_offload(lq, nullptr, nullptr, 0, 0, nullptr, be::QWeight{}, 0);
  auto s2 = b2.setup_offload(lq, nullptr, nullptr, CAP, NKV * HD, onorm.data(),
                             be::QWeight{reinterpret_cast<const std::byte*>(lm.data()), wt}, V);
  check(static_cast<bool>(s1) && static_cast<bool>(s2),
        std::string("setup_offload copies the weights once: ") + name +
            (s1 ? "" : " (" + s1.error().message + ")") + (s2 ? "" : " (" + s2.error().message + ")"));
  if (!s1 || !s2) return;
  okv* o = okv_create(NL, CAP, NKV, HD, 0, 0, OKV_F32);
  okv* o2 = okv_create(NL, CAP, NKV, HD, 0, 0, OKV_F32);
  bool ok = true, ok_full = true;
  double worst = 0, worst_full = 0;
  for (std::int32_t pos = 0; pos < 5; ++pos) {
    const std::vector<float> x = vec(D, 0.0f, 1.0f);
    std::vector<float> got = x, want = x, want2 = x;
    auto r = b1.decode_token(got.data(), pos);
    ok = ok && static_cast<bool>(r);
    for (std::size_t l = 0; l < NL; ++l) {
      okv_decode_layer(o, l, want.data(), pos, &ol[l], D, FF, NH, EPS, THETA, 1);
      okv_decode_layer(o2, l, want2.data(), pos, &ol[l], D, FF, NH, EPS, THETA, 1);
    }
    okv_truncate(o, pos + 1);
    okv_truncate(o2, pos + 1);
    ok = ok && within(got.data(), want, &worst);
    auto lg = b2.decode_token_full(x.data(), pos);
    ok_full = ok_full && static_cast<bool>(lg);
    if (lg) {
      std::vector<float> wl(V);
      ok_logits(want2.data(), onorm.data(), lm.data(), owt, EPS, wl.data(), D, V);
      ok_full = ok_full && within(*lg, wl, &worst_full);
    }
  }
  std::printf("  offload %s worst err/bound %.3f (residual), %.3f (logits)\n", name, worst,
              worst_full);
  check(ok, std::string("Backend::decode_token == decode_layer over every block: ") + name);
  check(ok_full, std::string("Backend::decode_token_full == blocks + rmsnorm + lm_head: ") + name);
  // errors come back as the reference's Error, not as aborts
  float xx[D] = {};
  check(!b1.decode_token_full(xx, 5), "decode_token_full without an lm_head is an error");
  std::vector<be::LayerQ> bad = lq;
  bad[1].dim = D + 64;
  check(!b1.setup_offload(bad, nullptr, nullptr, 0, 0, nullptr, be::QWeight{}, 0),
        "setup_offload rejects blocks of different shapes");
  okv_destroy(o);
  okv_destroy(o2);
}

int main(int argc, char** argv) {
  const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0;
  test_speculative_merge();
  test_rope_matches_oracle();
  if (!cpu_only) {
    const std::size_t ring_cases[8][3] = {{4, 8, 40}, {4, 8, 12}, {4, 8, 11}, {0, 8, 40},
                                          {1, 4, 40}, {4, 8, 4},  {4, 8, 2},  {4, 8, 100}};
    for (const auto& c : ring_cases) test_ring_case(c[0], c[1], c[2]);
    test_int8_roundtrip();
    test_int8_attention_vs_fp32();
    test_decode_layer_parity({0, 0, KvDtype::F32}, {32, 4, 64, 1e4f}, 2, 40, "dense fp32 gqa8 hd64");
    test_decode_layer_parity({4, 0, KvDtype::Int8}, {24, 8, 128, 5e5f}, 2, 40, "dense int8 gqa3 hd128");
    test_decode_layer_parity({4, 16, KvDtype::F32}, {28, 4, 128, 1e6f}, 2, 50, "ring fp32 gqa7 hd128");
    test_decode_layer_parity({4, 16, KvDtype::Int8}, {28, 4, 128, 1e6f}, 2, 50, "ring int8 gqa7 hd128");
    test_chunk_parity(KvDtype::F32);
    test_chunk_parity(KvDtype::Int8);
    test_producer_parity({0, 0, KvDtype::F32}, {32, 8, 128, 1e6f}, 20, "dense fp32 gqa4 hd128");
    test_producer_parity({4, 0, KvDtype::Int8}, {24, 8, 128, 5e5f}, 40, "dense int8 gqa3 hd128");
    test_producer_parity({4, 16, KvDtype::F32}, {28, 4, 128, 1e6f}, 30, "ring fp32 gqa7 hd128");
    test_prefix_cache();
    test_speculative_rollback();
    test_speculative_verify();
    test_output_projection();
    test_offload(true);
    test_offload(false);
  }
  std::printf("---\n%d checks failed\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
