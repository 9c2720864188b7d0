// Shortlist candidates: prototype prefix top-k and the packed builder.
//
// Prototype prefix top-k (replaces the O(rows*T) masked torch.topk of
// sparse_attn.py:260-300).  For batch b and token t the set S(t) is the
// min(t+1, K) largest scores among positions 0..t under the order "larger
// value first, equal values -> smaller index first".  Scores map to 64-bit
// keys (order-preserving bits of the value, then the complemented index),
// distinct and ordered as that rule orders them.  Tokens are cut into
// blocks of 64 and blocks into superblocks of SB tokens; three launches:
//   1. sb_top    : per superblock, its top-K keys (a radix select of the
//                  K-th largest key over the superblock's keys, staged in
//                  LDS, then every key at or above it), in any order;
//   2. sb_prefix : per superblock s, R[s] = top-K of the earlier
//                  superblocks' lists (= the set entering s) and its K-th
//                  key th[s];
//   3. walk      : per block j of superblock s, P = S(64j - 1) = top-K of
//                  R[s] and the tokens of s before the block whose key is at
//                  least th[s] (the K-th best key of a prefix only rises, so
//                  no other token can be in P), selected in LDS and sorted
//                  best first.  P is written as the block's set table row
//                  (best first, or sorted by index when the per-token sets
//                  are wanted), and the block's tokens are resolved in
//                  parallel from exact rank counts (below);
//   3. expand : (optional) S(t) for every token, sorted by index.
//
// Block walk without a sequential loop.  Let P be the set entering block j
// (sorted best first, n = |P| <= K) and B the block's tokens.  A token t
// enters iff fewer than K elements of P U {q in B, q < t} are better than
// t.  The set after the block is F = top-K(P U B).  Every element of
// P U entered that is not in F leaves during the block; since the K-th best
// element only rises, they leave in increasing key order, and the i-th
// insertion that finds the set full evicts the i-th of them.  With ranks in
// P U B (F occupies ranks < K), the leaver at rank r is evicted by entered
// token number max(0, K - n) + #(leavers with rank >= r) - 1.  Hence
//   evict[p] = first token at which p is no longer in the set, p if it never
//   enters, INT32_MAX if it is still in the set at the end,
// and p is in S(t) exactly when p <= t < evict[p]; so
//   S(t) = { p in P(block of t) U {64j .. t} : evict[p] > t }.
//
// Builder (replaces sparse_attn.py:376-596).  Per row, everything below the
// local window start `lo` (strided anchors in closed form, the prototype set
// prefix below lo, extra candidates) is merged with a merge-path co-rank,
// de-duplicated, and followed by the window lo..t and t-padding.  One wave
// per row; the row of L indices is written with 16-byte stores.
#include "pfa_common.h"

namespace pfa {

constexpr int kBlk = 64;  // tokens per prefix block (one wave)
constexpr int kBins = 2048;  // radix-select histogram bins (11-bit digits)

// Superblock size: the smallest power of two in [1024, 4096] whose lists
// (ceil(T/SB) of min(K, SB) keys) fit the LDS stage of sb_prefix; a sort of
// SB keys runs in one workgroup, so smaller superblocks spread the sorting
// over more CUs.
constexpr int kPrefixStage = 16384;  // list keys staged in LDS by sb_prefix (128 KB)
static int64_t prefix_sb_tokens(int64_t T, int K) {
  for (int64_t sb = 1024; sb < 4096; sb <<= 1)
    if ((T + sb - 1) / sb * (sb < K ? sb : (int64_t)K) <= kPrefixStage) return sb;
  return 4096;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PrefixWs {
  uint64_t* skey;  // (B, nsb, SB) each superblock's keys, best first
  uint64_t* rkey;  // (B, nsb, K) R[s]: top-K of the superblocks before s, best first
  int32_t* rlen;   // (B, nsb)
  int32_t* blk;    // (B, nb, K) set table (used by pfa_proto_prefix_topk)
  int32_t* evict;  // (B, T) (used when the caller passes no evict array)
};

static size_t prefix_ws_bytes(int64_t B, int64_t T, int64_t nb, int64_t nsb, int64_t SB, int64_t K, PrefixWs* w,
                              char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align256(bytes); return base ? base + o : nullptr; };
  char* p;
  p = take((size_t)B * nsb * SB * 8);  if (w) w->skey = (uint64_t*)p;
  p = take((size_t)B * nsb * K * 8);   if (w) w->rkey = (uint64_t*)p;
  p = take((size_t)B * nsb * 4);       if (w) w->rlen = (int32_t*)p;
  p = take((size_t)B * nb * K * 4);    if (w) w->blk = (int32_t*)p;
  p = take((size_t)B * T * 4);         if (w) w->evict = (int32_t*)p;
  return off;
}

// Order-preserving key of (score, position): larger key = better under
// `better` (value desc, then position asc; NaN below everything, two NaNs by
// position; -0 and +0 equal).  Every real key is > 0 (the complemented
// position is >= 2^31), so 0 pads.
__device__ __forceinline__ uint64_t score_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  uint32_t ord;
  if (v != v) ord = 0u;
  else if (v == 0.f) ord = 0x80000000u;
  else ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(~(uint32_t)idx);
}
__device__ __forceinline__ int key_index(uint64_t k) { return (int)(~(uint32_t)k); }
__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t ord = (uint32_t)(k >> 32);
  const uint32_t u = (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord;  // ord 0 -> a NaN
  return __uint_as_float(u);
}

// Radix select over the keys get(i), i < n, in one workgroup of NT threads
// (256 or 1024): returns a threshold th such that exactly `need` keys are
// >= th (need <= the number of keys, keys distinct).  The digits start at
// the highest bit in which the keys differ (found first: the OR of every key
// XOR the first one), so that keys concentrated in a narrow value range
// still spread over the bins; digits of 11 bits, down to bit 0, stopping at
// the first digit whose chosen bin holds exactly the keys still needed.
// hist: kBins LDS words; sh: NT/64 (at least 4) LDS words; sx: NT/64 LDS u64.
template <int NT, typename Get>
__device__ __forceinline__ uint64_t block_select(int n, int need, Get get, uint32_t* hist, int* sh, uint64_t* sx) {
  constexpr int NW = NT / 64, BPT = kBins / NT;  // waves, bins per thread
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // highest differing bit
  const uint64_t k0 = get(0);  // a real key (the first candidate always is)
  uint64_t x = 0;
  for (int i = tid; i < n; i += NT) {
    const uint64_t k = get(i);
    if (k != 0ull) x |= k ^ k0;  // padding (0) is below every real key and never selected
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x |= __shfl_xor(x, o, 64);
  if (lane == 0) sx[wid] = x;
  __syncthreads();
  x = 0;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) x |= sx[w2];
  __syncthreads();
  int top = x ? 63 - __clzll((long long)x) : 0;  // digits cover bits top .. 0
  uint64_t pmask = top < 63 ? ~((2ull << top) - 1ull) : 0ull;  // bits above top: common to every key
  uint64_t pval = k0 & pmask;
  while (true) {
    const int bits = top + 1 < 11 ? top + 1 : 11;
    const int shift = top + 1 - bits;
    const uint32_t dmask = (1u << bits) - 1u;
    for (int e = tid; e < kBins; e += NT) hist[e] = 0u;
    __syncthreads();
    for (int i = tid; i < n; i += NT) {
      const uint64_t k = get(i);
      if ((k & pmask) == pval) atomicAdd(&hist[(uint32_t)(k >> shift) & dmask], 1u);
    }
    __syncthreads();
    // bins from the top: thread t owns bins kBins-1-BPT*t .. kBins-BPT-BPT*t
    uint32_t c[BPT];
    uint32_t tot = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      c[q] = hist[kBins - 1 - BPT * tid - q];
      tot += c[q];
    }
    // inclusive scan of the thread totals (wave scans, then the wave sums)
    uint32_t incl = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) sh[wid] = (int)incl;
    __syncthreads();
    uint32_t before = incl - tot;
    for (int w2 = 0; w2 < wid; ++w2) before += (uint32_t)sh[w2];
    __syncthreads();
    if (before < (uint32_t)need && before + tot >= (uint32_t)need) {
      uint32_t acc = before;
#pragma unroll
      for (int q = 0; q < BPT; ++q) {
        if (acc < (uint32_t)need && acc + c[q] >= (uint32_t)need) {
          sh[0] = kBins - 1 - BPT * tid - q;  // chosen digit
          sh[1] = need - (int)acc;            // still needed inside it
          sh[2] = (int)c[q];                  // keys in it
        }
        acc += c[q];
      }
    }
    __syncthreads();
    const uint32_t d = (uint32_t)sh[0];
    const int still = sh[1], inbin = sh[2];
    __syncthreads();
    pmask |= (uint64_t)dmask << shift;
    pval |= (uint64_t)d << shift;
    need = still;
    if (inbin == still || shift == 0) break;  // every key of the bin is taken: threshold = prefix
    top = shift - 1;
  }
  return pval;
}

// Bitonic sort of cap = NT*V (V a power of two, 1..16) keys in LDS, largest
// first, by a workgroup of NT threads.  Thread t holds the V keys
// [V*t, V*t + V) in registers: strides below V are exchanged in registers,
// strides below 64*V with the partner lane of the same wave (shuffles), and
// the larger strides through LDS between barriers.  The caller has made the
// keys visible to every thread (a barrier) before the call; they are in LDS,
// sorted, and visible to every thread on return.
template <int NT, int V>
__device__ __forceinline__ void block_sort_desc_v(uint64_t* k) {
  constexpr int cap = NT * V;
  const int tid = threadIdx.x;
  uint64_t r[V];
#pragma unroll
  for (int i = 0; i < V; ++i) r[i] = k[V * tid + i];
  for (int kk = 2; kk <= cap; kk <<= 1) {
    // strides of V and more: partner lanes (shuffles) or other waves (LDS)
    for (int jj = kk >> 1; jj >= V; jj >>= 1) {
      if (jj < 64 * V) {
        const int lm = jj / V;  // partner lane distance (a power of two below 64)
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const uint64_t x = r[i];
          const uint64_t y = __shfl_xor((unsigned long long)x, lm, 64);
          const int e = V * tid + i;
          const bool desc = (e & kk) == 0, lower = (e & jj) == 0;
          const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
          r[i] = (lower == desc) ? hi : lo;
        }
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) k[V * tid + i] = r[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const int e = V * tid + i;
          const uint64_t x = r[i], y = k[e ^ jj];
          const bool desc = (e & kk) == 0, lower = (e & jj) == 0;
          const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
          r[i] = (lower == desc) ? hi : lo;
        }
        __syncthreads();
      }
    }
    // strides below V: inside the thread's registers (static indices)
#pragma unroll
    for (int jj = V >> 1; jj >= 1; jj >>= 1) {
      if (jj < kk) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
          if ((i & jj) == 0) {
            const int pi = i | jj;
            const int e = V * tid + i;
            const bool desc = (e & kk) == 0;
            const uint64_t x = r[i], y = r[pi];
            const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
            r[i] = desc ? hi : lo;
            r[pi] = desc ? lo : hi;
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i) k[V * tid + i] = r[i];
  __syncthreads();
}

// Element p of top-K(a U c) for best-first (descending) key lists a (na)
// and c (nc), by a merge-path co-rank.
__device__ __forceinline__ uint64_t merge_key_at(int p, const uint64_t* a, int na, const uint64_t* c, int nc) {
  int lo = max(0, p - nc), hi = min(p, na);
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] > c[p - 1 - mid]) lo = mid + 1;
    else hi = mid;
  }
  const int ia = lo, ic = p - lo;
  const bool take_a = ia < na && (ic >= nc || a[ia] > c[ic]);
  return take_a ? a[ia] : c[ic];
}

// Launch 1: superblock s's keys sorted best first (SB entries; the first
// K are its top-K), and the evict entries of its tokens initialised to
// "still in the set".  One 1024-thread workgroup per (s, b) (few
// superblocks: the sort's latency is hidden by four waves per SIMD), the
// keys sorted in LDS.
constexpr int kSbThreads = 1024;
template <int V>  // SB = 1024 * V
__global__ void __launch_bounds__(kSbThreads)
prefix_sb_sort(const float* __restrict__ scores, int64_t T, int64_t stride, int nsb,
               uint64_t* __restrict__ skey, int32_t* __restrict__ evict) {
  constexpr int NT = kSbThreads;
  constexpr int64_t SB = NT * V;
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ __align__(16) uint64_t stage[];
  const int sb = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int64_t t0 = (int64_t)sb * SB;
  const int n = (int)min<int64_t>(SB, T - t0);
  const float* sc = scores + (int64_t)b * stride + t0;
  float x[V];
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const int i = NT * u + tid;
    x[u] = i < n ? sc[i] : 0.f;  // loads issued together
  }
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const int i = NT * u + tid;
    if (i < n) evict[(int64_t)b * T + t0 + i] = INT32_MAX;
    stage[i] = i < n ? score_key(x[u], (int)(t0 + i)) : 0ull;
  }
  __syncthreads();
  block_sort_desc_v<NT, V>(stage);
  uint64_t* out = skey + ((int64_t)b * nsb + sb) * SB;
  for (int i = tid; i < (int)SB; i += NT) out[i] = stage[i];
}

// Launch 2: R[s] = top-K of superblocks 0 .. s-1 (the set entering s),
// sorted best first, rlen[s] = |R[s]|: the K-th largest key of the first
// min(K, SB) entries of each earlier superblock's sorted list (radix
// select; up to kPrefixStage entries are staged in LDS), then those at or
// above it, sorted.  One 1024-thread workgroup per (s, b).
template <int V>  // cap = 1024 * V >= K
__global__ void __launch_bounds__(kSbThreads)
prefix_sb_prefix(int nsb, int64_t SB, int K, const uint64_t* __restrict__ skey,
                 uint64_t* __restrict__ rkey, int32_t* __restrict__ rlen) {
  constexpr int NT = kSbThreads;
  constexpr int cap = NT * V;
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ __align__(16) uint64_t dyn[];
  uint64_t* keys = dyn;         // cap: the selected keys, then sorted
  uint64_t* stage = dyn + cap;  // the staged list entries
  __shared__ uint32_t hist[kBins];
  __shared__ int sh[NT / 64];
  __shared__ uint64_t sx[NT / 64];
  __shared__ int s_cnt;
  const int sb = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int per = (int)min<int64_t>(K, SB);  // entries taken from each earlier list
  const int nl = sb * per;
  const uint64_t* sk = skey + (int64_t)b * nsb * SB;
  auto gslot = [&](int i) -> uint64_t {
    const int q = i / per, e = i - q * per;
    return sk[(int64_t)q * SB + e];
  };
  const bool staged = nl <= kPrefixStage;
  if (staged) {
    uint64_t x[kPrefixStage / NT];
#pragma unroll
    for (int u = 0; u < kPrefixStage / NT; ++u) {
      const int i = NT * u + tid;
      x[u] = i < nl ? gslot(i) : 0ull;  // loads issued together
    }
#pragma unroll
    for (int u = 0; u < kPrefixStage / NT; ++u) {
      const int i = NT * u + tid;
      if (i < nl) stage[i] = x[u];
    }
  }
  for (int p = tid; p < cap; p += NT) keys[p] = 0ull;
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  auto get = [&](int i) -> uint64_t { return staged ? stage[i] : gslot(i); };
  uint64_t th = 1;  // every real key is > 0
  if (nl > K) th = block_select<NT>(nl, K, get, hist, sh, sx);
  for (int i = tid; i < nl; i += NT) {
    const uint64_t k = get(i);
    if (k >= th) keys[atomicAdd(&s_cnt, 1)] = k;
  }
  __syncthreads();
  const int cnt = s_cnt;
  block_sort_desc_v<NT, V>(keys);
  uint64_t* out = rkey + ((int64_t)b * nsb + sb) * K;
  for (int p = tid; p < K; p += NT) out[p] = keys[p];
  if (tid == 0) rlen[(int64_t)b * nsb + sb] = cnt;
}

// Launch 3: one workgroup (256 threads) per (block j, batch b).  P =
// S(64j - 1) = top-K(R[s] U Q) best first, Q = the tokens of superblock s
// before the block, best first (the superblock's sorted list with its later
// positions dropped, an ordered compaction), by a merge-path co-rank.
// LDS: R[s], Q and P (cap keys each), P's positions, index-sorted copy and
// ranks (cap each).
template <bool SORT>
__global__ void __launch_bounds__(256)
prefix_block_walk(const float* __restrict__ scores, int64_t T, int64_t stride, int nb, int64_t SB, int nsb, int K,
                  int cap, const uint64_t* __restrict__ skey, const uint64_t* __restrict__ rkey,
                  const int32_t* __restrict__ rlen, int32_t* __restrict__ blk_out, int32_t* __restrict__ evict) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ __align__(16) char smem[];
  uint64_t* ra = (uint64_t*)smem;
  uint64_t* qa = ra + cap;
  uint64_t* pkey = qa + cap;  // P's keys, best first
  int32_t* ix = (int32_t*)(pkey + cap);
  int32_t* srt = ix + cap;  // index-sorted copy of P
  int32_t* rk = srt + cap;  // ranks of P
  __shared__ uint64_t bkey[kBlk];  // the block's keys by position
  __shared__ uint64_t sbk[kBlk];   // and sorted best first
  __shared__ int32_t flag[kBlk];
  __shared__ int32_t ent[kBlk];
  __shared__ uint64_t s_fl;
  __shared__ int s_nent;
  __shared__ int s_wsum[4];
  const int j = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t t0 = (int64_t)j * kBlk;
  const int s = (int)(t0 / SB);
  const float* sc = scores + (int64_t)b * stride;
  const int64_t sr = (int64_t)b * nsb + s;
  const int na = rlen[sr];
  const uint64_t* rk0 = rkey + sr * K;
  for (int i = tid; i < na; i += 256) ra[i] = rk0[i];
  // Q: ordered compaction of the superblock's sorted keys with position < t0
  // (thread t scans entries [t*E, t*E + E), E = SB / 256)
  const int E = (int)(SB >> 8);  // at most 16 (SB <= 4096)
  const uint64_t* sk = skey + sr * SB + (int64_t)tid * E;
  uint64_t kv[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) kv[e] = e < E ? sk[e] : 0ull;  // loads issued together
  int cnt = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) cnt += (kv[e] != 0ull && key_index(kv[e]) < t0) ? 1 : 0;
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wid] = incl;
  __syncthreads();
  int pos = incl - cnt;
  for (int w2 = 0; w2 < wid; ++w2) pos += s_wsum[w2];
  const int nq_all = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    if (pos < K && kv[e] != 0ull && key_index(kv[e]) < t0) qa[pos++] = kv[e];
  }
  __syncthreads();
  const int nq = min(K, nq_all);
  const int n = (int)min<int64_t>(K, t0);  // |S(64j - 1)| = min(K, na + nq)
  for (int p = tid; p < n; p += 256) {
    const uint64_t k = merge_key_at(p, ra, na, qa, nq);
    pkey[p] = k;
    ix[p] = key_index(k);
  }
  const int nB = (int)min<int64_t>(kBlk, T - t0);
  int32_t st = INT32_MAX;
  uint64_t bk = 0ull;  // this token's key (wave 0); 0 past the sequence
  if (tid < kBlk) {
    if (tid < nB) { st = (int32_t)(t0 + tid); bk = score_key(sc[t0 + tid], st); }
    bkey[tid] = bk;
    flag[tid] = 0;
    // the block's keys sorted best first across the wave (bitonic, shuffles)
    uint64_t x = bk;
#pragma unroll
    for (int kk = 2; kk <= 64; kk <<= 1) {
#pragma unroll
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        const uint64_t y = __shfl_xor((unsigned long long)x, jj, 64);
        const bool desc = (tid & kk) == 0, lower = (tid & jj) == 0;
        const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
        x = (lower == desc) ? hi : lo;
      }
    }
    sbk[tid] = x;
  }
  __syncthreads();
  int32_t* orow = blk_out + ((int64_t)b * nb + j) * K;
  if constexpr (SORT) {
    // the block's set table row sorted by index (bitonic over cap entries)
    for (int p = tid; p < cap; p += 256) srt[p] = p < n ? ix[p] : INT32_MAX;
    __syncthreads();
    for (int kk = 2; kk <= cap; kk <<= 1) {
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        for (int e = tid; e < cap; e += 256) {
          const int q = e ^ jj;
          if (q > e) {
            const int x = srt[e], y = srt[q];
            if (((e & kk) == 0) ? (x > y) : (x < y)) { srt[e] = y; srt[q] = x; }
          }
        }
        __syncthreads();
      }
    }
    for (int p = tid; p < K; p += 256) orow[p] = srt[p];
  } else {
    // best first
    for (int p = tid; p < K; p += 256) orow[p] = p < n ? ix[p] : INT32_MAX;
  }
  // ranks of P's elements in P U B: p + the block keys above it (the block
  // sorted best first, padding 0 below every real key: a binary search)
  for (int p = tid; p < n; p += 256) {
    const uint64_t kp = pkey[p];
    int lo = 0, hi = kBlk;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sbk[mid] > kp) lo = mid + 1;
      else hi = mid;
    }
    const int r = p + lo;
    rk[p] = r;
    if (r >= K) flag[r - K] = 1;
  }
  // the block's tokens (wave 0): the keys of P above it (binary search),
  // of the block above it (its place in the sorted block) and of the earlier
  // block tokens above it
  bool enters = false;
  int rt = 0;
  if (tid < kBlk && tid < nB) {
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pkey[mid] > bk) lo = mid + 1;
      else hi = mid;
    }
    int la = 0, ha = kBlk;
    while (la < ha) {
      const int mid = (la + ha) >> 1;
      if (sbk[mid] > bk) la = mid + 1;
      else ha = mid;
    }
    int rb = 0;
    for (int q = 0; q < tid; ++q) rb += bkey[q] > bk ? 1 : 0;
    enters = lo + rb < K;
    rt = lo + la;
    if (enters && rt >= K) flag[rt - K] = 1;
  }
  __syncthreads();
  if (tid < kBlk) {
    const uint64_t fl = __ballot(flag[tid] != 0);
    const uint64_t em = __ballot(enters);
    if (enters) ent[__popcll(em & ((1ull << tid) - 1))] = st;
    if (tid == 0) { s_fl = fl; s_nent = __popcll(em); }
  }
  __syncthreads();
  const uint64_t fl = s_fl;
  const int nent = s_nent;
  const int free_ins = max(0, K - n);
  int32_t* ev = evict + (int64_t)b * T;
  for (int p = tid; p < n; p += 256) {
    const int r = rk[p];
    if (r >= K) {
      const int e = free_ins + __popcll(fl >> (r - K)) - 1;
      if (e >= 0 && e < nent) ev[ix[p]] = ent[e];
    }
  }
  if (tid < kBlk && tid < nB) {
    if (!enters) {
      ev[st] = st;
    } else if (rt >= K) {
      const int e = free_ins + __popcll(fl >> (rt - K)) - 1;
      if (e >= 0 && e < nent) ev[st] = ent[e];
    }
  }
}

// S(t) for every token, sorted by index, entries past min(t+1, K) = t.
// One wave per token.
__global__ void __launch_bounds__(256)
prefix_expand(int64_t T, int nb, int K, const int32_t* __restrict__ blk, const int32_t* __restrict__ evict,
              int32_t* __restrict__ sets) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  if (t >= T) return;
  const int64_t j = t / kBlk;
  const int32_t* P = blk + ((int64_t)b * nb + j) * K;
  const int32_t* ev = evict + (int64_t)b * T;
  int32_t* out = sets + ((int64_t)b * T + t) * K;
  const uint64_t lt = (1ull << lane) - 1;
  int n = 0;
  for (int base = 0; base < K; base += 64) {
    const int p = base + lane;
    const int32_t x = p < K ? P[p] : INT32_MAX;
    const bool keep = x != INT32_MAX && ev[x] > t;
    const uint64_t m = __ballot(keep);
    const int pos = n + __popcll(m & lt);
    if (keep && pos < K) out[pos] = x;  // |set| = min(t+1, K): the guard never binds
    n += __popcll(m);
    if (__ballot(x == INT32_MAX)) break;
  }
  {
    const int64_t q = j * kBlk + lane;
    const bool keep = q <= t && ev[q] > t;
    const uint64_t m = __ballot(keep);
    const int pos = n + __popcll(m & lt);
    if (keep && pos < K) out[pos] = (int32_t)q;
    n += __popcll(m);
  }
  for (int p = n + lane; p < K; p += 64) out[p] = (int32_t)t;
}

// ------------------------------------------------------------------
// Builder
// ------------------------------------------------------------------
constexpr int kBuildWaves = 4;

struct Anchors {
  int64_t t, s, J;
  int n1;     // strided anchors below lo
  int zflag;  // extra 0 at the front
  __device__ __forceinline__ int count() const { return n1 + zflag; }
  __device__ __forceinline__ int64_t at(int i) const {
    if (zflag) { if (i == 0) return 0; i -= 1; }
    return t - s * (J - i);
  }
};

template <bool I64C, bool I64L>
__global__ void __launch_bounds__(64 * kBuildWaves)
shortlist_build_kernel(const int32_t* __restrict__ rows, const int32_t* __restrict__ row_batch, int64_t N,
                       const int32_t* __restrict__ n_rows_dev, int64_t seq_len, int L, int local_w, int stride, int slots,
                       const int32_t* __restrict__ proto_sets, int K, int64_t proto_len,
                       const int32_t* __restrict__ extra, const int32_t* __restrict__ extra_len, int ew,
                       int qcap, int bcap, int fcap, void* __restrict__ cand_out, void* __restrict__ len_out) {
  extern __shared__ __align__(16) int32_t lds_i[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int32_t* Q = lds_i + wid * (qcap + bcap + fcap / 4);
  int32_t* Bb = Q + qcap;
  const int64_t r = (int64_t)blockIdx.x * kBuildWaves + wid;
  // N is the launch size; a device row count, when given, bounds it
  const int64_t n = n_rows_dev ? min<int64_t>(N, (int64_t)n_rows_dev[0]) : N;
  if (r >= n) return;
  const int64_t t = rows[r];
  const int64_t b = row_batch ? row_batch[r] : 0;

  int64_t lo, wlen;
  if (local_w > 0) { wlen = min<int64_t>(t + 1, local_w); lo = t - wlen + 1; }
  else { wlen = 1; lo = t; }

  // anchors below lo
  Anchors A;
  A.t = t; A.s = stride; A.J = 0; A.n1 = 0; A.zflag = 0;
  if (slots > 0 && stride > 0) {
    int64_t q = t / stride;
    A.J = min<int64_t>(slots, q);
    int64_t j0 = (t - lo) / stride + 1;
    A.n1 = (int)max<int64_t>(0, A.J - j0 + 1);
    bool zero_extra = (slots > q) && !((t % stride) == 0 && q >= 1);
    A.zflag = (zero_extra && lo > 0) ? 1 : 0;
  }
  const int na = A.count();

  int64_t nB;  // entries below the window after merge + dedup, at most L
  if (extra == nullptr) {
    // Q = prototype entries below lo: a sorted prefix of the (sorted, unique)
    // set row.  Each Q entry's merged position is closed-form: the anchors
    // below it are counted directly (they form an arithmetic sequence plus
    // the zero anchor), an entry equal to an anchor is dropped (the anchor
    // stays), and the free slots are then filled with the anchors in order.
    uint8_t* F = reinterpret_cast<uint8_t*>(Bb + bcap);  // 1 = slot holds a Q entry
    const uint64_t lt = (1ull << lane) - 1ull;
    const int64_t a_first = t - A.s * A.J;  // smallest strided anchor when n1 > 0
    for (int p = 16 * lane; p < fcap; p += 16 * 64) *reinterpret_cast<uint4*>(F + p) = make_uint4(0, 0, 0, 0);
    wave_sync();
    int nq = 0, nd = 0;
    if (proto_sets != nullptr && K > 0) {
      const int64_t prow = min(t, proto_len - 1);
      const int32_t* P = proto_sets + (b * proto_len + prow) * K;
      for (int base = 0; base < K; base += 256) {
        int32_t v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int i = base + 64 * c + lane;
          v[c] = i < K ? P[i] : INT32_MAX;
        }
        bool more = true;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int i = base + 64 * c + lane;
          const int64_t x = v[c];
          const bool valid = x < lo;
          const uint64_t vb = __ballot(valid);
          if (vb == 0) {
            more = false;
            break;
          }
          bool dup = false;
          int64_t rank = 0;
          if (valid) {
            const bool strided = A.n1 > 0 && x >= a_first && (x - a_first) % A.s == 0 && (x - a_first) / A.s < A.n1;
            dup = strided || (A.zflag && x == 0);
            rank = (A.zflag && x > 0) ? 1 : 0;
            if (A.n1 > 0 && x > a_first) rank += min<int64_t>((x - a_first + A.s - 1) / A.s, A.n1);
          }
          const uint64_t db = __ballot(dup);
          if (valid && !dup) {
            const int64_t pos = (int64_t)(i - (nd + __popcll(db & lt))) + rank;
            if (pos < L) {
              Bb[pos] = (int32_t)x;
              F[pos] = 1;
            }
          }
          nq += __popcll(vb);
          nd += __popcll(db);
        }
        if (!more) break;
      }
    }
    nB = min<int64_t>((int64_t)na + nq - nd, L);
    wave_sync();
    int qb = 0;
    for (int64_t base = 0; base < nB; base += 64) {
      const int64_t p = base + lane;
      const bool isq = p < nB && F[p] != 0;
      const uint64_t qbal = __ballot(isq);
      if (p < nB && !isq) Bb[p] = (int32_t)A.at((int)(p - qb - __popcll(qbal & lt)));
      qb += __popcll(qbal);
    }
    wave_sync();
  } else {
    // Q := sorted (proto below lo) merged with sorted (extra below lo)
    int nq = 0;
    if (proto_sets != nullptr && K > 0) {
      int64_t prow = min(t, proto_len - 1);
      const int32_t* P = proto_sets + (b * proto_len + prow) * K;
      for (int base = 0; base < K; base += 64) {
        int p = base + lane;
        int val = (p < K) ? P[p] : INT32_MAX;
        bool below = p < K && val < lo;
        uint64_t m = __ballot(below);
        if (below) Q[nq + p - base] = val;  // sorted prefix: below entries are contiguous from 0
        nq += __popcll(m);
        if (!m) break;
      }
    }
    if (extra != nullptr && ew > 0) {
      // extras below lo, sorted, then merged into Q (Bb used as scratch)
      int64_t el = extra_len ? extra_len[r] : ew;
      int32_t* E = Bb;  // scratch
      int ecap = 1;
      while (ecap < ew) ecap <<= 1;
      for (int p = lane; p < ecap; p += 64) {
        int64_t vv = INT32_MAX;
        if (p < ew) {
          int64_t raw = (p < el) ? (int64_t)extra[r * ew + p] : t;
          raw = raw < 0 ? 0 : raw;
          raw = raw > seq_len - 1 ? seq_len - 1 : raw;
          raw = raw > t ? t : raw;
          vv = raw < lo ? raw : INT32_MAX;
        }
        E[p] = (int32_t)vv;
      }
      wave_sync();
      for (int k = 2; k <= ecap; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
          for (int e = lane; e < ecap; e += 64) {
            int p = e ^ j;
            if (p > e) {
              bool up = (e & k) == 0;
              int a = E[e], c = E[p];
              if (up ? (a > c) : (a < c)) { E[e] = c; E[p] = a; }
            }
          }
          wave_sync();
        }
      int ne = 0;
      for (int p = 0; p < ecap; p += 64) {
        int e = p + lane;
        bool ok = e < ecap && E[e] != INT32_MAX;
        ne += __popcll(__ballot(ok));
      }
      // merge Q[0..nq) and E[0..ne) -> tmp in registers then back to Q (sizes <= qcap)
      int tot = nq + ne;
      int32_t tmp[8];
      int cnt = 0;
      for (int p = lane; p < tot; p += 64, ++cnt) {
        int lo2 = max(0, p - ne), hi2 = min(p, nq);
        while (lo2 < hi2) {
          int mid = (lo2 + hi2) >> 1;
          if (Q[mid] <= E[p - 1 - mid]) lo2 = mid + 1; else hi2 = mid;
        }
        int ia = lo2, ib = p - lo2;
        tmp[cnt] = (ia < nq && (ib >= ne || Q[ia] <= E[ib])) ? Q[ia] : E[ib];
      }
      wave_sync();
      cnt = 0;
      for (int p = lane; p < tot; p += 64, ++cnt) Q[p] = tmp[cnt];
      nq = tot;
      wave_sync();
    }


    // merge anchors with Q, drop adjacent duplicates, keep the first L.
    const int tot = na + nq;
    int nb_out = 0;
    int64_t prev_last = -1;  // last value of previous chunk
    for (int base = 0; base < tot && nb_out < L; base += 64) {
      int p = base + lane;
      int64_t val = -1;
      if (p < tot) {
        int lo2 = max(0, p - nq), hi2 = min(p, na);
        while (lo2 < hi2) {
          int mid = (lo2 + hi2) >> 1;
          if (A.at(mid) <= (int64_t)Q[p - 1 - mid]) lo2 = mid + 1; else hi2 = mid;
        }
        int ia = lo2, ib = p - lo2;
        val = (ia < na && (ib >= nq || A.at(ia) <= (int64_t)Q[ib])) ? A.at(ia) : (int64_t)Q[ib];
      }
      int64_t left = __shfl_up(val, 1, 64);
      if (lane == 0) left = prev_last;
      bool keep = p < tot && val != left;
      uint64_t m = __ballot(keep);
      int pos = nb_out + __popcll(m & ((1ull << lane) - 1ull));
      if (keep && pos < L && pos < bcap) Bb[pos] = (int32_t)val;
      nb_out += __popcll(m);
      prev_last = __shfl(val, 63, 64);
    }
    wave_sync();
    nB = min<int64_t>(nb_out, L);
  }
  const int64_t length = max<int64_t>(1, min<int64_t>(nB + wlen, L));

  // write the row: [0,nB) merged list, [nB, nB+wlen) window, rest t.
  auto value_at = [&](int64_t p) -> int64_t {
    if (p < nB) return Bb[p];
    if (p < nB + wlen) return lo + (p - nB);
    return t;
  };
  if constexpr (!I64C) {
    int32_t* out = (int32_t*)cand_out + r * L;
    if ((L & 3) == 0 && (((uintptr_t)cand_out) & 15) == 0) {
      // streaming stores: the candidate rows are written once and read by a
      // later launch, so they bypass the caches
      typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
      i32x4_t* o4 = (i32x4_t*)out;
      for (int q = lane; q < L / 4; q += 64) {
        int64_t p = 4 * (int64_t)q;
        const i32x4_t w = {(int)value_at(p), (int)value_at(p + 1), (int)value_at(p + 2), (int)value_at(p + 3)};
        __builtin_nontemporal_store(w, o4 + q);
      }
    } else {
      for (int p = lane; p < L; p += 64) out[p] = (int32_t)value_at(p);
    }
  } else {
    int64_t* out = (int64_t*)cand_out + r * L;
    if ((L & 1) == 0 && (((uintptr_t)cand_out) & 15) == 0) {
      longlong2* o2 = (longlong2*)out;
      for (int q = lane; q < L / 2; q += 64) {
        int64_t p = 2 * (int64_t)q;
        longlong2 w;
        w.x = value_at(p);
        w.y = value_at(p + 1);
        o2[q] = w;
      }
    } else {
      for (int p = lane; p < L; p += 64) out[p] = value_at(p);
    }
  }
  if (lane == 0) {
    if constexpr (I64L) ((int64_t*)len_out)[r] = length;
    else ((int32_t*)len_out)[r] = (int32_t)length;
  }
}

}  // namespace pfa

using namespace pfa;

static constexpr int kPrefixMaxK = 2048;
static constexpr size_t kPrefixLds = 60 * 1024;  // dynamic LDS budget per workgroup

static int prefix_cap(int K) {
  int cap = 256;  // the LDS sort takes 256 .. 4096 keys
  while (cap < K) cap <<= 1;
  return cap;
}

extern "C" int pfa_proto_prefix_workspace_size(int B, int64_t T, int K, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && B >= 0 && T >= 0 && K > 0, "pfa_proto_prefix_workspace_size: bad arguments");
  int64_t nb = (T + kBlk - 1) / kBlk;
  if (nb < 1) nb = 1;
  const int64_t SB = prefix_sb_tokens(T, K);
  const int64_t nsb = (T + SB - 1) / SB > 0 ? (T + SB - 1) / SB : 1;
  *bytes = prefix_ws_bytes(B, T, nb, nsb, SB, K, nullptr, nullptr);
  return PFA_OK;
}

// Set table rows (B, nb, K) and evict (B, T): three launches.
static int prefix_blocks(const float* scores, int B, int64_t T, int64_t stride, int K, int32_t* blk,
                         int32_t* evict, const PrefixWs& w, int64_t nb, bool sorted_rows, hipStream_t s) {
  const int64_t SB = prefix_sb_tokens(T, K);
  const int64_t nsb = (T + SB - 1) / SB;
  const int cap = prefix_cap(K);
  const dim3 sgrid((unsigned)nsb, (unsigned)B);
  // (past 48 KB of dynamic LDS a launch declares it; static arrays add ~8 KB)
  auto lds_attr = [](const void* fn, size_t bytes) {
    if (bytes > 48 * 1024) hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  };
#define PFA_SB_SORT(V_)                                                                                   \
  do {                                                                                                    \
    lds_attr((const void*)prefix_sb_sort<V_>, (size_t)SB * 8);                                            \
    prefix_sb_sort<V_><<<sgrid, kSbThreads, (size_t)SB * 8, s>>>(scores, T, stride, (int)nsb, w.skey, evict); \
  } while (0)
  switch (SB) {
    case 1024: PFA_SB_SORT(1); break;
    case 2048: PFA_SB_SORT(2); break;
    default: PFA_SB_SORT(4); break;
  }
#undef PFA_SB_SORT
  PFA_CHECK_LAUNCH("pfa_proto_prefix/superblocks");
  // the largest staged list-slot count of sb_prefix (superblocks whose
  // lists exceed kPrefixStage slots read them from global memory)
  const int64_t nl = (nsb - 1) * (SB < K ? SB : (int64_t)K);
  const int pcap = cap < kSbThreads ? kSbThreads : cap;  // the sort takes multiples of 1024 keys
  const size_t lds_pre = (size_t)pcap * 8 + (size_t)(nl < 1 ? 1 : (nl < kPrefixStage ? nl : kPrefixStage)) * 8;
#define PFA_SB_PREFIX(V_)                                                                                 \
  do {                                                                                                    \
    lds_attr((const void*)prefix_sb_prefix<V_>, lds_pre);                                                 \
    prefix_sb_prefix<V_><<<sgrid, kSbThreads, lds_pre, s>>>((int)nsb, SB, K, w.skey, w.rkey, w.rlen);     \
  } while (0)
  switch (pcap) {
    case 1024: PFA_SB_PREFIX(1); break;
    default: PFA_SB_PREFIX(2); break;
  }
#undef PFA_SB_PREFIX
  PFA_CHECK_LAUNCH("pfa_proto_prefix/superblock prefix");
  const size_t lds = (size_t)cap * 36;
  dim3 grid((unsigned)nb, (unsigned)B);
  if (sorted_rows) {
    lds_attr((const void*)prefix_block_walk<true>, lds);
    prefix_block_walk<true><<<grid, 256, lds, s>>>(scores, T, stride, (int)nb, SB, (int)nsb, K, cap, w.skey, w.rkey,
                                                   w.rlen, blk, evict);
  } else {
    lds_attr((const void*)prefix_block_walk<false>, lds);
    prefix_block_walk<false><<<grid, 256, lds, s>>>(scores, T, stride, (int)nb, SB, (int)nsb, K, cap, w.skey,
                                                    w.rkey, w.rlen, blk, evict);
  }
  PFA_CHECK_LAUNCH("pfa_proto_prefix/walk");
  return PFA_OK;
}

#define PFA_PREFIX_SETUP(NAME)                                                                              \
  clear_error();                                                                                            \
  PFA_CHECK_ARG(proto_scores && workspace && B > 0 && T > 0 && K > 0 && K <= kPrefixMaxK,                   \
                NAME ": bad arguments (B=%d T=%lld K=%d, K <= %d)", B, (long long)T, K, kPrefixMaxK);       \
  PFA_CHECK_ARG(T < ((int64_t)1 << 31), NAME ": T too large");                                              \
  const int64_t nb = (T + kBlk - 1) / kBlk;                                                                 \
  const int64_t SBt = prefix_sb_tokens(T, K);                                                               \
  const int64_t nsb = (T + SBt - 1) / SBt;                                                                  \
  const size_t need = prefix_ws_bytes(B, T, nb, nsb, SBt, K, nullptr, nullptr);                             \
  if (ws_bytes < need) {                                                                                    \
    set_error(NAME ": workspace %zu < %zu", ws_bytes, need);                                               \
    return PFA_E_WORKSPACE;                                                                                 \
  }                                                                                                         \
  PrefixWs w;                                                                                               \
  prefix_ws_bytes(B, T, nb, nsb, SBt, K, &w, (char*)workspace);                                             \
  hipStream_t s = as_stream(stream)

extern "C" int pfa_proto_prefix_blocks(const float* proto_scores, int B, int64_t T, int64_t score_stride, int K,
                                       int32_t* blocks_out, int32_t* evict_out, void* workspace, size_t ws_bytes,
                                       void* stream) {
  PFA_PREFIX_SETUP("pfa_proto_prefix_blocks");
  PFA_CHECK_ARG(blocks_out && evict_out, "pfa_proto_prefix_blocks: null output");
  return prefix_blocks(proto_scores, B, T, score_stride, K, blocks_out, evict_out, w, nb, false, s);
}

extern "C" int pfa_proto_prefix_topk(const float* proto_scores, int B, int64_t T, int64_t score_stride, int K,
                                     int32_t* sets_out, int32_t* evict_out, void* workspace, size_t ws_bytes,
                                     void* stream) {
  PFA_PREFIX_SETUP("pfa_proto_prefix_topk");
  PFA_CHECK_ARG(sets_out != nullptr, "pfa_proto_prefix_topk: null output");
  int32_t* ev = evict_out ? evict_out : w.evict;
  int rc = prefix_blocks(proto_scores, B, T, score_stride, K, w.blk, ev, w, nb, true, s);
  if (rc != PFA_OK) return rc;
  prefix_expand<<<dim3((unsigned)((T + 3) / 4), (unsigned)B), 256, 0, s>>>(T, (int)nb, K, w.blk, ev, sets_out);
  PFA_CHECK_LAUNCH("pfa_proto_prefix/expand");
  return PFA_OK;
}

extern "C" int pfa_shortlist_build(const int32_t* rows, const int32_t* row_batch, int64_t N,
                                   const int32_t* n_rows_dev, int64_t seq_len, int L,
                                   int local_w, int anchor_stride, int anchor_slots, const int32_t* proto_sets,
                                   int proto_k, int64_t proto_len, const int32_t* extra, const int32_t* extra_len,
                                   int extra_width, void* cand_out, int cand_is_i64, void* len_out, int len_is_i64,
                                   void* stream) {
  clear_error();
  PFA_CHECK_ARG(N >= 0 && seq_len > 0 && L > 0, "pfa_shortlist_build: bad sizes N=%lld T=%lld L=%d", (long long)N,
                (long long)seq_len, L);
  if (N == 0) return PFA_OK;
  PFA_CHECK_ARG(rows && cand_out && len_out, "pfa_shortlist_build: null pointer");
  PFA_CHECK_ARG(proto_sets == nullptr || (proto_k > 0 && proto_len > 0), "pfa_shortlist_build: bad proto_k");
  PFA_CHECK_ARG(extra == nullptr || (extra_width > 0 && extra_width <= 512), "pfa_shortlist_build: extra width");
  int qcap = (proto_sets ? proto_k : 0) + (extra ? extra_width : 0);
  int ecap = 1;
  while (extra && ecap < extra_width) ecap <<= 1;
  int64_t bound = (int64_t)anchor_slots + 1 + qcap;
  int bcap = (int)((int64_t)L < bound ? (int64_t)L : bound);
  if (extra && bcap < ecap) bcap = ecap;
  qcap = (qcap + 3) & ~3;
  bcap = (bcap + 3) & ~3;
  if (qcap == 0) qcap = 4;
  const int fcap = extra ? 0 : (bcap + 15) & ~15;  // Q-slot flags of the proto-only merge (bytes)
  size_t lds = (size_t)kBuildWaves * ((qcap + bcap) * 4 + fcap);
  PFA_CHECK_ARG(lds <= 160 * 1024, "pfa_shortlist_build: LDS need %zu too large (L=%d K=%d slots=%d)", lds, L,
                proto_k, anchor_slots);
  PFA_CHECK_ARG(!extra || (extra_width + proto_k) <= 64 * 8, "pfa_shortlist_build: extra merge too wide");
  unsigned blocks = (unsigned)((N + kBuildWaves - 1) / kBuildWaves);
  hipStream_t s = as_stream(stream);
#define PFA_BUILD(C64, L64)                                                                                   \
  shortlist_build_kernel<C64, L64><<<blocks, 64 * kBuildWaves, lds, s>>>(                                     \
      rows, row_batch, N, n_rows_dev, seq_len, L, local_w, anchor_stride, anchor_slots, proto_sets, proto_sets ? proto_k : 0, \
      proto_len, extra, extra_len, extra ? extra_width : 0, qcap, bcap, fcap, cand_out, len_out)
  if (cand_is_i64) {
    if (len_is_i64) PFA_BUILD(true, true); else PFA_BUILD(true, false);
  } else {
    if (len_is_i64) PFA_BUILD(false, true); else PFA_BUILD(false, false);
  }
#undef PFA_BUILD
  PFA_CHECK_LAUNCH("pfa_shortlist_build");
  return PFA_OK;
}
