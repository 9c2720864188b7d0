// Multi-workgroup radix select: the k-th largest 32-bit key of each segment
// (a batch row, or one chunk), spread over the whole GPU.
//
// Three launches of one digit each (bits 31..21, 20..10, 9..0).  Every
// workgroup takes kSpan consecutive keys, counts the digit of the keys that
// share the bits fixed so far in an LDS histogram and adds its non-empty
// bins to the segment's global histogram.  The last workgroup to finish (an
// acquire-release counter) reads the global histogram, fixes the digit that
// holds the target rank, clears the histogram for the next launch and resets
// the counter.  The third launch also keeps each workgroup's own histogram,
// so that its last workgroup can hand every workgroup the number of tied keys
// (keys equal to the final cut) in the workgroups before it: the callers'
// emit kernels then admit ties by ascending index with no further pass.
//
// Everything is integer counting, so the result does not depend on the order
// in which workgroups run.  The state lives in the caller's workspace; an init
// launch sets it, and each pass leaves the histogram zeroed behind it.
//
// Cross-workgroup visibility: everything the last workgroup reads is written
// by agent-scope atomics (the histogram adds, the per-workgroup histograms of
// the third pass) and read by agent-scope atomic loads, and every workgroup
// waits for its own memory operations to complete before it moves the
// counter (arrive()).  No agent-scope release fence is needed, which on this
// chip would write back the whole L2 of the workgroup's XCD.
#pragma once

#include "pfa_common.h"

namespace pfa {
namespace rsel {

constexpr int kThreads = 256;
constexpr int kPer = 4;                 // consecutive keys per thread
constexpr int kSpan = kThreads * kPer;  // keys per workgroup
constexpr int kBins = 2048;             // the first two digits have 11 bits
constexpr int kLastBins = 1024;         // the last one 10
constexpr int kPasses = 3;

__host__ __device__ constexpr int digit_shift(int pass) { return pass == 0 ? 21 : (pass == 1 ? 10 : 0); }
__host__ __device__ constexpr int digit_bins(int pass) { return pass == 2 ? kLastBins : kBins; }

// Per segment, at the start of its workspace region (64 bytes).
struct State {
  uint32_t prefix;    // key bits fixed by the passes so far
  int32_t remaining;  // rank of the target among the keys sharing `prefix` (1-based)
  uint32_t done;      // workgroups finished with the current pass
  int32_t need;       // keys to select: <= 0 none, >= n all (no pass runs)
  uint32_t slot;      // emit: slots handed out to keys above the cut
  uint32_t max_ord;   // emit: largest key seen (order key of a float)
  int32_t finite;     // emit: finite scores seen
  int32_t count;      // scores at or above a threshold (token top-k)
  uint32_t pad[8];
};
static_assert(sizeof(State) == 64, "State is 64 bytes");

__host__ __device__ inline int64_t groups_of(int64_t n) { return n > 0 ? (n + kSpan - 1) / kSpan : 1; }

// byte offsets within one segment's region
struct Layout {
  size_t ghist, tiebase, wstat, whist, bytes;
};
__host__ __device__ inline Layout layout(int64_t groups) {
  Layout L;
  L.ghist = sizeof(State);
  L.tiebase = L.ghist + (size_t)kBins * 4;
  L.wstat = L.tiebase + (size_t)((groups * 4 + 255) / 256) * 256;      // per-workgroup statistics (2 words)
  L.whist = L.wstat + (size_t)((groups * 8 + 255) / 256) * 256;
  L.bytes = L.whist + (size_t)((groups * kLastBins * 4 + 255) / 256) * 256;
  return L;
}
__host__ inline size_t segment_bytes(int64_t n) { return layout(groups_of(n)).bytes; }

__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This workgroup is done with the current launch: once all of its memory
// operations have completed (vmcnt 0 in every wave, then the barrier), thread
// 0 moves the counter.  True in the workgroup that arrives last.
__device__ __forceinline__ bool arrive(uint32_t* done, uint32_t groups, int* s_last) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = old == groups - 1u ? 1 : 0;
  }
  __syncthreads();
  return *s_last != 0;
}

// Exclusive scan over the 256 threads of a workgroup, in thread order.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* sm, uint32_t& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) sm[wv] = x;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < kThreads / 64; ++k) {
    pre += k < wv ? sm[k] : 0u;
    tot += sm[k];
  }
  total = tot;
  return pre + x - v;
}

// Sets every segment's state (need and the target rank as given: a later
// launch may still finalise them) and clears its histogram.
// grid = (segments).
template <class Src>
__global__ void __launch_bounds__(kThreads) init_kernel(unsigned char* ws, size_t seg_bytes, int64_t need) {
  unsigned char* base = ws + (size_t)blockIdx.x * seg_bytes;
  State* st = reinterpret_cast<State*>(base);
  uint32_t* ghist = reinterpret_cast<uint32_t*>(base + sizeof(State));
  for (int j = threadIdx.x; j < kBins; j += kThreads) ghist[j] = 0u;
  if (threadIdx.x == 0) {
    st->prefix = 0u;
    st->remaining = (int32_t)need;
    st->done = 0u;
    st->need = (int32_t)need;
    st->slot = 0u;
    st->max_ord = 0u;
    st->finite = 0;
    st->count = 0;
  }
}

// One digit pass.  grid = (groups_of(n), segments); Src::key(seg, i) gives the
// 32-bit order key of element i of segment seg.
template <class Src>
__global__ void __launch_bounds__(kThreads) pass_kernel(Src src, int64_t n, int pass, unsigned char* ws,
                                                         size_t seg_bytes) {
  __shared__ uint32_t lh[kBins];
  __shared__ uint32_t sm[kThreads / 64];
  __shared__ int s_last, s_digit;
  const int seg = blockIdx.y, w = blockIdx.x, tid = threadIdx.x;
  const int64_t G = gridDim.x;
  unsigned char* base = ws + (size_t)seg * seg_bytes;
  State* st = reinterpret_cast<State*>(base);
  const Layout Lo = layout(G);
  uint32_t* ghist = reinterpret_cast<uint32_t*>(base + Lo.ghist);
  int32_t* tiebase = reinterpret_cast<int32_t*>(base + Lo.tiebase);
  uint32_t* whist = reinterpret_cast<uint32_t*>(base + Lo.whist);
  const int need = st->need;
  if (need <= 0 || (int64_t)need >= n) return;  // uniform over the grid: nothing to resolve
  const uint32_t prefix = st->prefix;
  const int remaining = st->remaining;
  const int sh = digit_shift(pass), nb = digit_bins(pass);
  const int hs = sh + (pass == 2 ? 10 : 11);  // the bits above this digit (32 for the first pass)
  for (int j = tid; j < nb; j += kThreads) lh[j] = 0u;
  __syncthreads();
  const int64_t i0 = (int64_t)w * kSpan + (int64_t)tid * kPer;
  uint32_t kv[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) kv[e] = i0 + e < n ? src.key(seg, i0 + e) : 0u;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const bool match = i0 + e < n && (pass == 0 || (kv[e] >> hs) == (prefix >> hs));
    if (match) atomicAdd(&lh[(kv[e] >> sh) & (uint32_t)(nb - 1)], 1u);
  }
  __syncthreads();
  if (pass == kPasses - 1)
    for (int j = tid; j < nb; j += kThreads) store_agent(&whist[(int64_t)w * kLastBins + j], lh[j]);
  for (int j = tid; j < nb; j += kThreads) {
    const uint32_t c = lh[j];
    if (c != 0u) __hip_atomic_fetch_add(&ghist[j], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!arrive(&st->done, (uint32_t)G, &s_last)) return;
  // last workgroup: thread t holds bins nb-1-per*t .. nb-per*(t+1) (highest first)
  const int per = nb / kThreads;
  uint32_t cnt[kBins / kThreads];
  uint32_t c = 0u;
#pragma unroll
  for (int q = 0; q < kBins / kThreads; ++q) {
    cnt[q] = q < per ? load_agent(&ghist[nb - 1 - (tid * per + q)]) : 0u;
    c += cnt[q];
  }
  if (tid == 0) s_digit = 0;
  uint32_t total = 0u;
  const uint32_t before = block_excl_scan(c, sm, total);
  if (before < (uint32_t)remaining && before + c >= (uint32_t)remaining) {
    uint32_t cum = before;
    int d = 0;
#pragma unroll
    for (int q = 0; q < kBins / kThreads; ++q) {
      if (q < per && cum + cnt[q] >= (uint32_t)remaining) {
        d = nb - 1 - (tid * per + q);
        break;
      }
      cum += cnt[q];
    }
    st->prefix = prefix | ((uint32_t)d << sh);
    st->remaining = remaining - (int)cum;
    s_digit = d;
  }
  __syncthreads();
  for (int j = tid; j < kBins; j += kThreads) ghist[j] = 0u;
  if (tid == 0) st->done = 0u;
  if (pass == kPasses - 1) {
    // ties before each workgroup: exclusive scan of its count of the final digit
    const int d = s_digit;
    uint32_t carry = 0u;
    for (int64_t b0 = 0; b0 < G; b0 += kThreads) {
      const int64_t wq = b0 + tid;
      const uint32_t v = wq < G ? load_agent(&whist[wq * kLastBins + d]) : 0u;
      uint32_t tot = 0u;
      const uint32_t ex = block_excl_scan(v, sm, tot);
      if (wq < G) tiebase[wq] = (int32_t)(carry + ex);
      carry += tot;
    }
  }
}

// The selection rule of the emit kernels, for the kPer consecutive keys of
// this thread: sel[e] = key above the cut, or one of the first `remaining`
// keys equal to it in index order; rank[e] is a key's rank among the keys
// equal to the cut (index order).  Collective over the workgroup.
__device__ __forceinline__ void select_keys(const uint32_t (&kv)[kPer], int64_t i0, int64_t n, uint32_t cut,
                                            int remaining, int32_t tiebase, uint32_t* sm, bool (&sel)[kPer],
                                            bool (&above)[kPer], uint32_t (&rank)[kPer]) {
  bool eq[kPer];
  uint32_t t = 0u;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    above[e] = i0 + e < n && kv[e] > cut;
    eq[e] = i0 + e < n && kv[e] == cut;
    t += eq[e] ? 1u : 0u;
  }
  uint32_t tot = 0u;
  uint32_t r = (uint32_t)tiebase + block_excl_scan(t, sm, tot);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    rank[e] = r;
    sel[e] = above[e] || (eq[e] && r < (uint32_t)remaining);
    r += eq[e] ? 1u : 0u;
  }
}

template <class Src>
__host__ inline int run_passes(Src src, int64_t n, int segments, unsigned char* ws, size_t seg_bytes, hipStream_t s,
                               const char* what) {
  const dim3 grid((unsigned)groups_of(n), (unsigned)segments);
  for (int p = 0; p < kPasses; ++p) {
    pass_kernel<Src><<<grid, kThreads, 0, s>>>(src, n, p, ws, seg_bytes);
    PFA_CHECK_LAUNCH(what);
  }
  return PFA_OK;
}

}  // namespace rsel
}  // namespace pfa
