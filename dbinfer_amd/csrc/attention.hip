// Planning and launch of the GQA attention kernel (attn_kernel.hpp): the
// split-K plan of a call, the kernel instance it needs, and its arguments.
#include "attn_kernel.hpp"

namespace dbi {
namespace {

void* pick_kernel(int hd, int kind, int G, bool prod = false, int cpw = 1) {
  switch (kind * 2 + (prod ? 1 : 0)) {
    case 0: return attn_instance_0_0(hd, G, cpw);
    case 1: return attn_instance_0_1(hd, G, cpw);
    case 2: return attn_instance_1_0(hd, G, cpw);
    case 3: return attn_instance_1_1(hd, G, cpw);
    case 4: return attn_instance_2_0(hd, G, cpw);
    case 5: return attn_instance_2_1(hd, G, cpw);
    case 6: return attn_instance_3_0(hd, G, cpw);
    case 7: return attn_instance_3_1(hd, G, cpw);
    default: return nullptr;
  }
}


int kind_of(const KvGeom& g) { return (g.ring ? 2 : 0) + (g.int8 ? 1 : 0); }

// positions per chunk of the kernel instance (Cfg::CHUNK)
int chunk_of(const KvGeom& g) { return g.int8 && !g.ring ? 2 * kGranule : kGranule; }

// Workgroups one launch aims for (split-K fan-out: one 8-wave workgroup per
// CU).
constexpr int kTargetBlocks = 256;

// Dense chunks of two or more rows run on the matrix-core rows kernels
// (attn_rows.hpp for fp32, attn_i8_rows.hpp for int8): nvt 16-vector tiles
// per workgroup (nvt 3: one, and a remainder tile), rows_vectors / G
// rows each.
bool rows_kernel(const KvGeom& g, const AttnCall& c) { return !g.ring && c.rows > 1; }
// 1: one 16-column tile; 2: two; 3: one, plus a remainder tile for a few
// more vectors (int8: (query, channel block) columns for up to 16 / (hd / 32);
// fp32: 4 x 4 blocks for up to 4)
int rows_rem(const KvGeom& g) { return g.int8 ? 16 / (g.hd / 32) : 4; }
int rows_nvt(const KvGeom& g, int G, int rows) {
  if (rows * G <= 16) return 1;
  return rows * G <= 16 + rows_rem(g) ? 3 : 2;
}
// query vectors a workgroup of the instance serves
int rows_vectors(const KvGeom& g, int nvt) { return nvt == 3 ? 16 + rows_rem(g) : 16 * nvt; }

struct Plan {
  int nsplit, chunks_per_split;
  int nvt;     // rows kernel: vector tiles per workgroup (0: not the rows kernel)
  int cpw;     // kernel instance: chunks per wave (1, 2, 4; 0 = runtime loop)
  int nr;      // query rows per workgroup (rows kernels; else 1)
  int zgroups; // workgroups per (split, kv head): ceil(rows / nr)
  bool merge;  // several splits: the last to finish merges them
};

Plan plan(const KvGeom& g, const AttnCall& c) {
  const int G = c.n_heads / g.nkv;
  const bool rowsk = rows_kernel(g, c);
  const int chunk = rowsk && !g.int8 ? kGranule : chunk_of(g);
  const int nkeys_max = g.ring ? c.ring.n_res : c.pos0 + c.rows;
  const int nchunks = (nkeys_max + chunk - 1) / chunk;
  const int nvt = rowsk ? rows_nvt(g, G, c.rows) : 0;
  const int nr = rowsk ? (rows_vectors(g, nvt) / G < c.rows ? rows_vectors(g, nvt) / G : c.rows) : 1;
  const int zgroups = (c.rows + nr - 1) / nr;
  const int units = g.nkv * zgroups;
  // whole waves of workgroups only: a launch of target + a few would run a
  // second, nearly empty round on the CUs
  int want = kTargetBlocks / units;
  // (every wave of both kernels serves all G heads of its chunks)
  const int wpg = kWaves;
  // at least one chunk per wave; a short context may go down to one chunk
  // per two waves (more CUs share the stream, some waves idle) while that
  // keeps one merging workgroup within 32 records, or within 64 where the
  // merge is spread over several workgroups anyway (records beyond
  // kOneMergerBytes at 64 splits; measured: 64 records read by one
  // workgroup cost the C4 ring more than the wider spread gains)
  const int rec_cap = 64 * G * g.hd * 4 > kOneMergerBytes && !rowsk ? 64 : 32;
  const int strict = (nchunks + wpg - 1) / wpg;
  const int relaxed = (nchunks + wpg / 2 - 1) / (wpg / 2);
  const int relaxed_c = relaxed < rec_cap ? relaxed : rec_cap;
  const int max_by_chunks = strict > relaxed_c ? strict : relaxed_c;
  if (want > max_by_chunks) want = max_by_chunks;
  if (want > kMaxSplits) want = kMaxSplits;
  if (want < 1) want = 1;
  Plan p;
  p.nvt = nvt;
  p.nr = nr;
  p.zgroups = zgroups;
  p.chunks_per_split = (nchunks + want - 1) / want;
  p.nsplit = (nchunks + p.chunks_per_split - 1) / p.chunks_per_split;
  // (dense int8 rows: the merge launch also attends the fp32 sinks)
  p.merge = p.nsplit > 1 || (rowsk && g.int8 && g.n_sink > 0);
  const int per_wave = (p.chunks_per_split + wpg - 1) / wpg;
  p.cpw = per_wave <= 1 ? 1 : per_wave <= 2 ? 2 : per_wave <= 4 ? 4 : 0;
  return p;
}

}  // namespace

bool attention_supported(const KvGeom& g, int n_heads) {
  if (n_heads <= 0 || n_heads % g.nkv != 0 || !g.tiled) return false;
  return pick_kernel(g.hd, kind_of(g), n_heads / g.nkv) != nullptr;
}

int attention_split_count(const KvGeom& g, const AttnCall& c) { return plan(g, c).nsplit; }

size_t attention_counters_need(const KvGeom& g, const AttnCall& c) {
  const Plan p = plan(g, c);  // (the rows kernel's merge is a second launch: no counters)
  return p.merge && p.nvt == 0 ? static_cast<size_t>(c.rows) * g.nkv * kCounterStride : 0;
}

size_t attention_workspace_need(const KvGeom& g, const AttnCall& c) {
  const Plan p = plan(g, c);
  const int G = c.n_heads / g.nkv;
  return p.merge ? static_cast<size_t>(c.rows) * g.nkv * record_region(p.nsplit, G, g.hd) : 0;
}

size_t attention_workspace_bound(const KvGeom& g, int n_heads) {
  return static_cast<size_t>(g.nkv) * record_region(kMaxSplits, n_heads / g.nkv, g.hd);
}

size_t attention_counters_bound(const KvGeom& g) {
  return static_cast<size_t>(g.nkv) * kCounterStride;
}

hipError_t launch_attention(const KvGeom& g, const KvStore& s, Workspace& ws, const AttnCall& c,
                            hipStream_t st) {
  const int G = c.n_heads / g.nkv;
  const bool prod = c.rows == 1 && (c.q_bias != nullptr || c.k_bias != nullptr ||
                                    c.v_bias != nullptr || c.rope_row != nullptr);
  const Plan pl = plan(g, c);
  void* fn = pl.nvt > 0 ? (g.int8 ? attn_instance_i8_rows(g.hd, G, pl.nvt)
                                  : attn_instance_f32_rows(g.hd, G, pl.nvt))
                        : pick_kernel(g.hd, kind_of(g), G, prod, pl.cpw);
  if (fn == nullptr || !g.tiled) return hipErrorNotSupported;
  AttnParams p{};
  const size_t layer_heads = static_cast<size_t>(c.layer) * g.nkv;
  const size_t layer_el = layer_heads * head_elems(g);
  if (!g.int8) {
    p.kf = s.k + layer_el;
    p.vf = s.v + layer_el;
  } else {
    p.k8 = reinterpret_cast<const uint8_t*>(s.k8) + layer_el;
    p.v8 = reinterpret_cast<const uint8_t*>(s.v8) + layer_el;
    p.vs = s.v_scale + layer_heads * g.capg * g.nb;
    if (g.ring) {
      p.ks = s.k_scale + layer_heads * g.capg * g.nb;
    } else {
      p.ks = s.k_scale + layer_heads * g.ngroups * g.hd;
      if (g.n_sink > 0) {
        p.ksink = s.k_sink + layer_heads * g.n_sink * g.hd;
        p.vsink = s.v_sink + layer_heads * g.n_sink * g.hd;
      }
    }
  }
  p.rope = s.rope_cs;
  p.rope_rows = g.ring ? g.cap : 0;
  p.q = c.q;
  p.out = c.out;
  p.part = ws.part;
  p.cnt = ws.counters;
  p.capg = g.capg;
  p.ng = g.ngroups;
  p.n_sink = g.int8 && !g.ring ? g.n_sink : 0;
  p.nkv = g.nkv;
  p.n_heads = c.n_heads;
  p.rows = c.rows;
  p.pos0 = c.pos0;
  p.ring_nres = c.ring.n_res;
  p.ring_s = c.ring.s;
  p.ring_W = c.ring.W > 0 ? c.ring.W : 1;
  p.ring_base = c.ring.base;
  p.nsplit = pl.nsplit;
  p.direct = pl.merge ? 0 : 1;
  p.chunks_per_split = pl.chunks_per_split;
  p.qscale = c.scale * kLog2e;
  if (c.rows == 1) {
    p.qb = c.q_bias;
    p.qcs = c.rope_row;
  }
  AppendArgs a{};
  a.slot = -1;
  if (c.app_slot >= 0 && c.app_k != nullptr && c.app_v != nullptr && c.rows == 1) {
    a.k = c.app_k;
    a.v = c.app_v;
    a.slot = c.app_slot;
    a.pos = c.app_pos;
    a.kb = c.k_bias;
    a.vb = c.v_bias;
    a.kcs = c.rope_row;
    a.prod = c.k_bias != nullptr || c.v_bias != nullptr || c.rope_row != nullptr;
    a.nkv = g.nkv;
    a.n_sink = g.n_sink;
    a.capg = g.capg;
    a.ng = g.ngroups;
    if (!g.int8) {
      a.kf = s.k + layer_el;
      a.vf = s.v + layer_el;
    } else {
      a.k8 = reinterpret_cast<uint8_t*>(s.k8) + layer_el;
      a.v8 = reinterpret_cast<uint8_t*>(s.v8) + layer_el;
      a.vs = s.v_scale + layer_heads * g.capg * g.nb;
      if (g.ring) {
        a.ks = s.k_scale + layer_heads * g.capg * g.nb;
      } else {
        a.ks = s.k_scale + layer_heads * g.ngroups * g.hd;
        a.k_raw = s.k_raw + static_cast<size_t>(c.layer) * kKGroup * g.nkv * g.hd;
        if (g.n_sink > 0) {
          a.ksink = s.k_sink + layer_heads * g.n_sink * g.hd;
          a.vsink = s.v_sink + layer_heads * g.n_sink * g.hd;
        }
      }
    }
  }
  void* args[] = {&p, &a};
  if (pl.nvt > 0) {  // rows kernel: records, then the merge launch
    void* rargs[] = {&p};
    const hipError_t e =
        hipLaunchKernel(fn, dim3(p.nsplit, g.nkv, pl.zgroups), dim3(kThreads), rargs, 0, st);
    if (e != hipSuccess || !pl.merge) return e;
    void* mfn = attn_instance_f32_rows_merge(g.hd, G);
    if (mfn == nullptr) return hipErrorNotSupported;
    return hipLaunchKernel(mfn, dim3(c.rows * c.n_heads), dim3(64), rargs, 0, st);
  }
  return hipLaunchKernel(fn, dim3(p.nsplit, g.nkv, pl.zgroups), dim3(kThreads), args, 0, st);
}

}  // namespace dbi
