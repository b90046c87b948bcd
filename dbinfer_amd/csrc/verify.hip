// Token side of one speculative verify round on the device: the greedy argmax
// of each of the k+1 logit rows the target model produced for the verify
// chunk (speculative.cpp:69-70 calling sample::argmax, sample.cpp:11-28), then
// the merge of the k draft proposals against those argmaxes
// (speculative_merge, speculative.cpp:10-23). One launch: the logits stay in
// HBM and only the k+1 argmaxes and the accepted count are written.
//
// Argmax semantics. The reference scans a row and replaces its best only on a
// strictly greater value, so the answer is the earliest index whose value
// equals the largest non-NaN value of the row, and 0 when slot 0 holds a NaN
// (no comparison with a NaN best is true). -0.0 and +0.0 compare equal.
// Each workgroup reduces a slice of a row to one 64-bit key,
//   (order(value) << 32) | (0xffffffff - index),
// whose unsigned maximum is exactly that answer: order() is monotone in the
// float value, maps both zeros alike and maps NaN below -inf, and the low word
// makes the earlier index win between equal values. The slot-0 NaN rule is
// applied once per row at the end.
//
// Grid: (slices per row, rows). Each workgroup stores its key with an
// agent-coherent store, waits for it, then counts itself with one agent-scope
// atomic; the last to arrive reads every key with agent-coherent loads,
// writes the argmaxes, runs the merge and sets the counter back to zero. No
// memory fence is used (an agent-scope fence writes back or invalidates a
// whole L2 on this multi-XCD part), and no clear is needed between calls
// (none is recorded when the call is captured).
#include "kv_internal.hpp"

namespace dbi {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPerThread = 32;  // loads in flight per thread (one batch)

using u64 = unsigned long long;

struct VerifyArgs {
  const float* logits;  // [rows][vocab]
  const int32_t* draft;  // [rows - 1]
  int32_t* verified;     // [rows]
  int32_t* accepted;     // [1]
  u64* keys;             // [rows][nb]
  unsigned* counter;
  int rows, vocab, nb, span;
};

__device__ inline unsigned order_of(float v) {
  if (v != v) return 0u;
  const unsigned b = v == 0.0f ? 0u : __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ inline u64 key_of(float v, int i) {
  return (static_cast<u64>(order_of(v)) << 32) | (0xffffffffu - static_cast<unsigned>(i));
}

__device__ inline u64 wave_max(u64 x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const u64 o = __shfl_xor(x, off);
    x = o > x ? o : x;
  }
  return x;
}

__global__ __launch_bounds__(kThreads) void verify_kernel(VerifyArgs a) {
  __shared__ u64 s_w[kWaves];
  __shared__ int s_last;
  __shared__ int s_best[kMaxVerifyRows];
  const int b = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  const float* row = a.logits + static_cast<size_t>(r) * a.vocab;
  const int lo = b * a.span;
  const int hi = min(lo + a.span, a.vocab);
  u64 best = 0;
  // every load of a slice is issued before the first key is formed: one
  // memory round trip per kThreads * kPerThread elements
  for (int base = lo + t; base < hi; base += kThreads * kPerThread) {
    float v[kPerThread];
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int j = base + u * kThreads;
      v[u] = j < hi ? row[j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int j = base + u * kThreads;
      if (j < hi) {
        const u64 k = key_of(v[u], j);
        best = k > best ? k : best;
      }
    }
  }
  best = wave_max(best);
  if (lane == 0) s_w[w] = best;
  __syncthreads();
  if (t == 0) {
    u64 m = s_w[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) m = s_w[i] > m ? s_w[i] : m;
    __hip_atomic_store(&a.keys[static_cast<size_t>(r) * a.nb + b], m, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    // the key has reached the coherence point before the arrival is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const unsigned total = static_cast<unsigned>(a.nb) * static_cast<unsigned>(a.rows);
    const unsigned prev =
        __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == total - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // the draft goes to LDS while the waves reduce the slice keys
  __shared__ int s_draft[kMaxVerifyDraft];
  if (t < a.rows - 1) s_draft[t] = a.draft[t];
  // wave w owns rows w, w + kWaves, ...; one lane per slice key (nb <= 64).
  // All of a wave's loads are issued before the first reduction.
  constexpr int kRowsPerWave = (kMaxVerifyRows + kWaves - 1) / kWaves;
  u64 kk[kRowsPerWave];
  float first[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int rr = w + i * kWaves;
    kk[i] = 0;
    first[i] = 0.0f;
    if (rr < a.rows) {
      first[i] = a.logits[static_cast<size_t>(rr) * a.vocab];
      if (lane < a.nb)
        kk[i] = __hip_atomic_load(&a.keys[static_cast<size_t>(rr) * a.nb + lane],
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int rr = w + i * kWaves;
    if (rr < a.rows) {
      const u64 k = wave_max(kk[i]);
      if (lane == 0) {
        const int idx = first[i] != first[i]
                            ? 0
                            : static_cast<int>(0xffffffffu - static_cast<unsigned>(k));
        s_best[rr] = idx;
        a.verified[rr] = idx;
      }
    }
  }
  __syncthreads();
  if (t == 0) {
    const int kd = a.rows - 1;
    int j = 0;
    while (j < kd && s_draft[j] == s_best[j]) ++j;
    a.accepted[0] = j;
    __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

hipError_t launch_verify(const VerifyCall& c, hipStream_t st) {
  VerifyArgs a{};
  a.logits = c.logits;
  a.draft = c.draft;
  a.verified = c.verified;
  a.accepted = c.accepted;
  a.keys = c.keys;
  a.counter = c.counter;
  a.rows = c.rows;
  a.vocab = c.vocab;
  // slices of one load batch (kThreads * kPerThread elements) while a row
  // fits in kMaxVerifySlices of them, longer slices past that; halving the
  // slice (twice the workgroups and arrivals) measured slower
  const long per = static_cast<long>(kThreads) * kPerThread;
  long nb = (static_cast<long>(c.vocab) + per - 1) / per;
  nb = nb < 1 ? 1 : (nb > kMaxVerifySlices ? kMaxVerifySlices : nb);
  a.span = static_cast<int>((c.vocab + nb - 1) / nb);
  // every slice is non-empty: (nb - 1) * span < vocab
  a.nb = static_cast<int>((c.vocab + a.span - 1) / a.span);
  hipLaunchKernelGGL(verify_kernel, dim3(a.nb, a.rows), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace dbi
