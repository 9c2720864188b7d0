// Shortlist candidates: prototype prefix top-k and the packed builder.
//
// Prototype prefix top-k (replaces the O(rows*T) masked torch.topk of
// sparse_attn.py:260-300).  For batch b and token t the set S(t) is the
// min(t+1, K) largest scores among positions 0..t under the order "larger
// value first, equal values -> smaller index first".  Tokens are cut into
// blocks of 64 and blocks into superblocks of `sbs` blocks:
//   1. block_sort : each block's scores sorted best first (wave bitonic);
//   2. sb_local   : per superblock, one workgroup folds its blocks in order:
//                   Q[j] = top-K of the superblock's tokens up to block j;
//   3. scan_round : a log-depth scan over the superblock totals (ceil(log2
//                   nsb) rounds, every superblock in parallel):
//                   R[s] = top-K of all tokens before superblock s;
//   4. block_walk : per block j, P = top-K(R[s] U Q[j-1]) = S(64j - 1) is
//                   written as the block's set table row (best first, or
//                   sorted by index when the per-token sets are wanted), and
//                   the block's tokens are resolved in parallel from exact
//                   rank counts (below);
//   5. expand     : (optional) S(t) for every token, sorted by index.
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

// Superblock size: the local fold is a sequential chain of sbs merges, the
// superblock scan takes ceil(log2(nb / sbs)) parallel rounds.
static int64_t prefix_sbs(int64_t nb) {
  return nb < 8 ? (nb > 0 ? nb : 1) : 8;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PrefixWs {
  float* bval;
  int32_t* bidx;
  int32_t* blen;
  float* qval;
  int32_t* qidx;
  int32_t* qlen;
  float* rval;  // (B, nsb+1, K): row s+1 = top-K of superblocks 0..s, row 0 empty
  int32_t* ridx;
  int32_t* rlen;
  float* r2val;  // ping-pong partner of rval/ridx/rlen for the log-depth scan
  int32_t* r2idx;
  int32_t* r2len;
  int32_t* blk;    // (B, nb, K) set table (used by pfa_proto_prefix_topk)
  int32_t* evict;  // (B, T) (used when the caller passes no evict array)
};

static size_t prefix_ws_bytes(int64_t B, int64_t T, int64_t nb, int64_t nsb, int64_t K, PrefixWs* w, char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align256(bytes); return base ? base + o : nullptr; };
  char* p;
  p = take((size_t)B * nb * kBlk * 4); if (w) w->bval = (float*)p;
  p = take((size_t)B * nb * kBlk * 4); if (w) w->bidx = (int32_t*)p;
  p = take((size_t)B * nb * 4);        if (w) w->blen = (int32_t*)p;
  p = take((size_t)B * nb * K * 4);    if (w) w->qval = (float*)p;
  p = take((size_t)B * nb * K * 4);    if (w) w->qidx = (int32_t*)p;
  p = take((size_t)B * nb * 4);        if (w) w->qlen = (int32_t*)p;
  p = take((size_t)B * (nsb + 1) * K * 4);   if (w) w->rval = (float*)p;
  p = take((size_t)B * (nsb + 1) * K * 4);   if (w) w->ridx = (int32_t*)p;
  p = take((size_t)B * (nsb + 1) * 4);       if (w) w->rlen = (int32_t*)p;
  p = take((size_t)B * (nsb + 1) * K * 4);   if (w) w->r2val = (float*)p;
  p = take((size_t)B * (nsb + 1) * K * 4);   if (w) w->r2idx = (int32_t*)p;
  p = take((size_t)B * (nsb + 1) * 4);       if (w) w->r2len = (int32_t*)p;
  p = take((size_t)B * nb * K * 4);    if (w) w->blk = (int32_t*)p;
  p = take((size_t)B * T * 4);         if (w) w->evict = (int32_t*)p;
  return off;
}

// Sort (v, i) across the 64 lanes of a wave: best first.
__device__ __forceinline__ void wave_bitonic_best_first(float& v, int& i) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      float pv = __shfl_xor(v, j, 64);
      int pi = __shfl_xor(i, j, 64);
      bool up = (lane & k) == 0;
      bool lower = (lane & j) == 0;
      bool self_better = better(v, i, pv, pi);
      bool keep = (lower == up) ? self_better : !self_better;
      if (!keep) { v = pv; i = pi; }
    }
  }
}

__global__ void __launch_bounds__(64)
prefix_block_sort(const float* __restrict__ scores, int64_t T, int64_t stride, int nb, int K,
                  float* __restrict__ oval, int32_t* __restrict__ oidx, int32_t* __restrict__ olen,
                  int32_t* __restrict__ evict) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  int64_t t = (int64_t)j * kBlk + lane;
  if (t < T) evict[(int64_t)b * T + t] = INT32_MAX;
  float v = -INFINITY;
  int i = INT32_MAX;
  if (t < T) { v = scores[(int64_t)b * stride + t]; i = (int)t; }
  wave_bitonic_best_first(v, i);
  int64_t n = T - (int64_t)j * kBlk;
  if (n > kBlk) n = kBlk;
  if (n > K) n = K;
  int64_t base = ((int64_t)b * nb + j) * kBlk;
  if (lane < n) { oval[base + lane] = v; oidx[base + lane] = i; }
  if (lane == 0) olen[(int64_t)b * nb + j] = (int)n;
}

// Element p of top-K(a U c) for best-first lists a (na) and c (nc), by a
// merge-path co-rank.  Either list may live in LDS or global memory.
__device__ __forceinline__ void merge_at(int p, const float* av, const int32_t* ai, int na, const float* cv,
                                         const int32_t* ci, int nc, float& ov, int32_t& oi) {
  int lo = max(0, p - nc), hi = min(p, na);
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (better(av[mid], ai[mid], cv[p - 1 - mid], ci[p - 1 - mid])) lo = mid + 1;
    else hi = mid;
  }
  const int ia = lo, ic = p - lo;
  const bool take_a = ia < na && (ic >= nc || better(av[ia], ai[ia], cv[ic], ci[ic]));
  ov = take_a ? av[ia] : cv[ic];
  oi = take_a ? ai[ia] : ci[ic];
}

// Q[j] = top-K(Q[j-1] U block j) within each superblock (one workgroup).
// With `preload` every block list of the superblock is staged in LDS up
// front (one burst of loads); otherwise the next block is fetched one step
// ahead.  The sequential chain then runs on LDS only.
__global__ void __launch_bounds__(256)
prefix_sb_local(int nb, int sbs, int K, int preload, const float* __restrict__ bval,
                const int32_t* __restrict__ bidx, const int32_t* __restrict__ blen, float* __restrict__ qval,
                int32_t* __restrict__ qidx, int32_t* __restrict__ qlen) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ char smem[];
  float* cv0 = (float*)smem;
  int32_t* ci0 = (int32_t*)(cv0 + K);
  float* cv1 = (float*)(ci0 + K);
  int32_t* ci1 = (int32_t*)(cv1 + K);
  const int nslot = preload ? sbs : 2;
  float* kv = (float*)(ci1 + K);  // nslot x kBlk
  int32_t* ki = (int32_t*)(kv + nslot * kBlk);
  int32_t* kn = ki + nslot * kBlk;  // nslot lengths
  const int sb = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int j0 = sb * sbs, j1 = min(nb, j0 + sbs);
  if (j0 >= j1) return;
  const int cnt = j1 - j0;
  const int nfirst = preload ? cnt : 1;
  for (int e = tid; e < nfirst * kBlk; e += 256) {
    const int jj = e / kBlk, l = e % kBlk;
    const int64_t row = (int64_t)b * nb + j0 + jj;
    const int nbl = blen[row];
    if (l < nbl) { kv[jj * kBlk + l] = bval[row * kBlk + l]; ki[jj * kBlk + l] = bidx[row * kBlk + l]; }
    if (l == 0) kn[jj] = nbl;
  }
  __syncthreads();
  int n = 0, cur = 0;
  for (int i = 0; i < cnt; ++i) {
    const int j = j0 + i;
    const int slot = preload ? i : (i & 1);
    float pv = 0.f;
    int32_t pi = 0;
    int pn = 0;
    if (!preload && i + 1 < cnt) {
      const int64_t nrow = (int64_t)b * nb + j + 1;
      pn = blen[nrow];
      if (tid < pn) { pv = bval[nrow * kBlk + tid]; pi = bidx[nrow * kBlk + tid]; }
    }
    const int64_t row = (int64_t)b * nb + j;
    const int nbl = kn[slot];
    const float* bv = kv + slot * kBlk;
    const int32_t* bi = ki + slot * kBlk;
    const int m = min(K, n + nbl);
    const float* av = cur ? cv1 : cv0;
    const int32_t* ai = cur ? ci1 : ci0;
    float* ov = cur ? cv0 : cv1;
    int32_t* oi = cur ? ci0 : ci1;
    for (int p = tid; p < m; p += 256) {
      float vv;
      int32_t ii;
      merge_at(p, av, ai, n, bv, bi, nbl, vv, ii);
      ov[p] = vv;
      oi[p] = ii;
      qval[row * K + p] = vv;
      qidx[row * K + p] = ii;
    }
    if (tid == 0) qlen[row] = m;
    if (!preload && i + 1 < cnt) {
      const int ns = (i + 1) & 1;
      if (tid < pn) { kv[ns * kBlk + tid] = pv; ki[ns * kBlk + tid] = pi; }
      if (tid == 0) kn[ns] = pn;
    }
    __syncthreads();
    cur ^= 1;
    n = m;
  }
}

// One round of a log-depth radix-R (Hillis-Steele) inclusive scan over
// superblock totals: out[s] = top-K(in[s] U in[s-d] U ... U in[s-(R-1)d])
// over the terms with a non-negative index (d = R^round, so after round r
// row s covers superblocks s-R^(r+1)+1 .. s).  Rows are (nsb+1)-strided with
// row s+1 holding superblock s (row 0 stays empty, so that the walk reads
// row s as "everything before superblock s").  With `from_q` the input is
// the superblock totals themselves: the local prefix of each superblock's
// last block.  One workgroup per (superblock, batch): the (up to R <= 8)
// lists are staged in LDS together and reduced by a tree of pairwise
// co-rank merges (log2 R levels, the pairs of a level merged side by side,
// the last level written straight to the output row).  Top-K under the
// strict order `better` of distinct positions does not depend on the merge
// order.
__global__ void __launch_bounds__(256)
prefix_scan_round(int nb, int sbs, int nsb, int K, int d, int radix, int from_q, const float* __restrict__ qval,
                  const int32_t* __restrict__ qidx, const int32_t* __restrict__ qlen,
                  const float* __restrict__ ival, const int32_t* __restrict__ iidx, const int32_t* __restrict__ ilen,
                  float* __restrict__ oval, int32_t* __restrict__ oidx, int32_t* __restrict__ olen) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ char smem[];
  // entry arrays: radix input lists, then level-1 outputs (radix/2 lists),
  // then level-2 outputs (radix/4 lists); list i of a region at i*K
  float* ev = (float*)smem;
  const int cap_e = (radix + (radix > 2 ? radix / 2 : 0) + (radix > 4 ? radix / 4 : 0)) * K;
  int32_t* ei = (int32_t*)(ev + cap_e);
  __shared__ int s_off[8], s_len[8];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int64_t rb = (int64_t)b * (nsb + 1);
  // input row of superblock ss (entries at row * K) and its length
  auto row_of_sb = [&](int ss) -> int64_t {
    return from_q ? (int64_t)b * nb + min(nb, (ss + 1) * sbs) - 1 : rb + ss + 1;
  };
  const float* inv = from_q ? qval : ival;
  const int32_t* ini = from_q ? qidx : iidx;
  const int32_t* inl = from_q ? qlen : ilen;
  float* ov = oval + (rb + s + 1) * K;
  int32_t* oi = oidx + (rb + s + 1) * K;
  if (s == 0 && tid == 0) olen[rb] = 0;
  const int nl = min(radix, s / d + 1);  // terms s, s-d, ... that exist
  // all lengths in one round of loads, then every entry in one flat loop
  if (tid < nl) {
    s_off[tid] = tid * K;
    s_len[tid] = inl[row_of_sb(s - tid * d)];
  }
  __syncthreads();
  if (nl == 1) {
    const int64_t r0 = row_of_sb(s);
    const int n0 = s_len[0];
    for (int p = tid; p < n0; p += 256) { ov[p] = inv[r0 * K + p]; oi[p] = ini[r0 * K + p]; }
    if (tid == 0) olen[rb + s + 1] = n0;
    return;
  }
  for (int e = tid; e < nl * K; e += 256) {
    const int k = e / K, p = e - k * K;
    if (p < s_len[k]) {
      const int64_t r = row_of_sb(s - k * d);
      ev[e] = inv[r * K + p];
      ei[e] = ini[r * K + p];
    }
  }
  __syncthreads();
  int n = nl;
  int region = radix * K;  // where level 1 writes
  for (int level = 0; n > 1; ++level) {
    const int np = n >> 1;
    const bool last = n == 2;
    const int tpp = 256 / np;  // threads per pair (np <= 4)
    const int pr = tid / tpp, pt = tid % tpp;
    int m = 0;
    if (pr < np) {
      const int oa = s_off[2 * pr], na = s_len[2 * pr];
      const int oc = s_off[2 * pr + 1], nc = s_len[2 * pr + 1];
      m = min(K, na + nc);
      const int od = region + pr * K;
      for (int p = pt; p < m; p += tpp) {
        float vv;
        int32_t ii;
        merge_at(p, ev + oa, ei + oa, na, ev + oc, ei + oc, nc, vv, ii);
        if (last) {
          ov[p] = vv;
          oi[p] = ii;
        } else {
          ev[od + p] = vv;
          ei[od + p] = ii;
        }
      }
    }
    __syncthreads();
    if (last) {
      if (tid == 0) olen[rb + s + 1] = m;
      break;
    }
    // pair pr becomes list pr; an odd last list is carried as it is (the
    // descriptors are read before any is rewritten)
    int new_off = 0, new_len = 0, carry_off = 0, carry_len = 0;
    if (tid < np) {
      new_off = region + tid * K;
      new_len = min(K, s_len[2 * tid] + s_len[2 * tid + 1]);
    }
    if (tid == 0 && (n & 1)) {
      carry_off = s_off[n - 1];
      carry_len = s_len[n - 1];
    }
    __syncthreads();
    if (tid < np) {
      s_off[tid] = new_off;
      s_len[tid] = new_len;
    }
    if (tid == 0 && (n & 1)) {
      s_off[np] = carry_off;
      s_len[np] = carry_len;
    }
    __syncthreads();
    region += np * K;
    n = np + (n & 1);
  }
}

// One workgroup (256 threads) per (block j, batch b).  LDS: the entering set
// P best first (v, ix: cap entries each, cap = power of two >= K) and a
// staging area of 2*cap floats + 2*cap ints that first holds R[s] and
// Q[j-1] for the merge, then the index-sorted copy and the ranks of P.
template <bool SORT>
__global__ void __launch_bounds__(256)
prefix_block_walk(const float* __restrict__ scores, int64_t T, int64_t stride, int nb, int sbs, int nsb, int K,
                  int cap, const float* __restrict__ qval, const int32_t* __restrict__ qidx,
                  const int32_t* __restrict__ qlen, const float* __restrict__ rval, const int32_t* __restrict__ ridx,
                  const int32_t* __restrict__ rlen, int32_t* __restrict__ blk_out, int32_t* __restrict__ evict) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ char smem[];
  float* v = (float*)smem;
  int32_t* ix = (int32_t*)(v + cap);
  float* sav = (float*)(ix + cap);        // staging: R values   (cap)
  int32_t* sai = (int32_t*)(sav + cap);   //          R indices  (cap)
  float* sqv = (float*)(sai + cap);       //          Q values   (cap)
  int32_t* sqi = (int32_t*)(sqv + cap);   //          Q indices  (cap)
  int32_t* srt = sai;                     // after the merge: index-sorted copy
  int32_t* rk = sqi;                      //                  ranks of P
  __shared__ float bv[kBlk];
  __shared__ int32_t bi[kBlk];
  __shared__ int32_t flag[kBlk];
  __shared__ int32_t ent[kBlk];
  __shared__ uint64_t s_fl;
  __shared__ int s_nent;
  const int j = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int s = j / sbs, k = j % sbs;
  const int64_t rrow = (int64_t)b * (nsb + 1) + s;  // row s: top-K of superblocks 0..s-1
  const int64_t qrow = (int64_t)b * nb + j - 1;      // block j-1's local prefix (k > 0)
  // both lengths in one round of loads, then the entries of both rows
  const int na = rlen[rrow];
  const int nq = k > 0 ? qlen[qrow] : 0;
  for (int p = tid; p < K; p += 256) {
    if (p < na) { sav[p] = rval[rrow * K + p]; sai[p] = ridx[rrow * K + p]; }
    if (p < nq) { sqv[p] = qval[qrow * K + p]; sqi[p] = qidx[qrow * K + p]; }
  }
  const int64_t t0 = (int64_t)j * kBlk;
  const int nB = (int)min<int64_t>(kBlk, T - t0);
  float sv = -INFINITY;
  int32_t st = INT32_MAX;
  if (tid < kBlk) {
    if (tid < nB) { sv = scores[(int64_t)b * stride + t0 + tid]; st = (int32_t)(t0 + tid); }
    bv[tid] = sv;
    bi[tid] = st;
    flag[tid] = 0;
  }
  __syncthreads();
  const int n = min(K, na + nq);
  for (int p = tid; p < n; p += 256) {
    float vv;
    int32_t ii;
    merge_at(p, sav, sai, na, sqv, sqi, nq, vv, ii);
    v[p] = vv;
    ix[p] = ii;
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
    // best first, as merged
    for (int p = tid; p < K; p += 256) orow[p] = p < n ? ix[p] : INT32_MAX;
  }
  // ranks of P's elements in P U B (P is sorted best first)
  for (int p = tid; p < n; p += 256) {
    int c = 0;
    for (int q = 0; q < nB; ++q) c += better(bv[q], bi[q], v[p], ix[p]) ? 1 : 0;
    const int r = p + c;
    rk[p] = r;
    if (r >= K) flag[r - K] = 1;
  }
  // the block's tokens (wave 0)
  bool enters = false;
  int rt = 0;
  if (tid < kBlk && tid < nB) {
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (better(v[mid], ix[mid], sv, st)) lo = mid + 1;
      else hi = mid;
    }
    int ra = 0, rb = 0;
    for (int q = 0; q < nB; ++q) {
      if (better(bv[q], bi[q], sv, st)) {
        ++ra;
        if (q < tid) ++rb;
      }
    }
    enters = lo + rb < K;
    rt = lo + ra;
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

// Radix of the superblock scan: as many lists as fit the LDS budget (R
// inputs plus the tree's intermediate lists, 8 bytes per entry), at most 8.
static int prefix_round_entries(int radix) { return radix + (radix > 2 ? radix / 2 : 0) + (radix > 4 ? radix / 4 : 0); }
static int prefix_radix(int K) {
  for (int r = 8; r > 2; r >>= 1)
    if ((size_t)prefix_round_entries(r) * K * 8 <= kPrefixLds) return r;
  return 2;
}

static int prefix_cap(int K) {
  int cap = 64;
  while (cap < K) cap <<= 1;
  return cap;
}

extern "C" int pfa_proto_prefix_workspace_size(int B, int64_t T, int K, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && B >= 0 && T >= 0 && K > 0, "pfa_proto_prefix_workspace_size: bad arguments");
  int64_t nb = (T + kBlk - 1) / kBlk;
  if (nb < 1) nb = 1;
  const int64_t sbs = prefix_sbs(nb);
  const int64_t nsb = (nb + sbs - 1) / sbs;
  *bytes = prefix_ws_bytes(B, T, nb, nsb, K, nullptr, nullptr);
  return PFA_OK;
}

// Steps 1-4: set table rows (B, nb, K) and evict (B, T).
static int prefix_blocks(const float* scores, int B, int64_t T, int64_t stride, int K, int32_t* blk,
                         int32_t* evict, const PrefixWs& w, int64_t nb, bool sorted_rows, hipStream_t s) {
  const int64_t sbs = prefix_sbs(nb);
  const int64_t nsb = (nb + sbs - 1) / sbs;
  const int cap = prefix_cap(K);
  dim3 grid((unsigned)nb, (unsigned)B);
  prefix_block_sort<<<grid, 64, 0, s>>>(scores, T, stride, (int)nb, K, w.bval, w.bidx, w.blen, evict);
  PFA_CHECK_LAUNCH("pfa_proto_prefix/sort");
  const int preload = (size_t)K * 16 + (size_t)sbs * (kBlk * 8 + 4) <= kPrefixLds ? 1 : 0;
  const size_t lds_local = (size_t)K * 16 + (size_t)(preload ? sbs : 2) * (kBlk * 8 + 4);
  prefix_sb_local<<<dim3((unsigned)nsb, (unsigned)B), 256, lds_local, s>>>(
      (int)nb, (int)sbs, K, preload, w.bval, w.bidx, w.blen, w.qval, w.qidx, w.qlen);
  PFA_CHECK_LAUNCH("pfa_proto_prefix/local");
  // log-depth inclusive scan of the superblock totals (ping-pong between
  // the two R buffers; the last round lands in the buffer the walk reads)
  const int radix = prefix_radix(K);
  int rounds = 0;
  for (int64_t span = 1; span < nsb; span *= radix) ++rounds;
  if (rounds == 0) rounds = 1;
  const size_t lds_round = (size_t)prefix_round_entries(radix) * K * 8;
  const float* fin_v = nullptr;
  const int32_t* fin_i = nullptr;
  const int32_t* fin_l = nullptr;
  for (int r = 0; r < rounds; ++r) {
    const bool to_primary = ((rounds - 1 - r) & 1) == 0;
    float* ov = to_primary ? w.rval : w.r2val;
    int32_t* oi = to_primary ? w.ridx : w.r2idx;
    int32_t* ol = to_primary ? w.rlen : w.r2len;
    const float* iv = to_primary ? w.r2val : w.rval;
    const int32_t* ii = to_primary ? w.r2idx : w.ridx;
    const int32_t* il = to_primary ? w.r2len : w.rlen;
    int d = 1;
    for (int q = 0; q < r; ++q) d *= radix;
    prefix_scan_round<<<dim3((unsigned)nsb, (unsigned)B), 256, lds_round, s>>>(
        (int)nb, (int)sbs, (int)nsb, K, d, radix, r == 0 ? 1 : 0, w.qval, w.qidx, w.qlen, iv, ii, il, ov, oi, ol);
    PFA_CHECK_LAUNCH("pfa_proto_prefix/scan");
    fin_v = ov;
    fin_i = oi;
    fin_l = ol;
  }
  if (sorted_rows)
    prefix_block_walk<true><<<grid, 256, (size_t)cap * 24, s>>>(scores, T, stride, (int)nb, (int)sbs, (int)nsb, K,
                                                                cap, w.qval, w.qidx, w.qlen, fin_v, fin_i, fin_l,
                                                                blk, evict);
  else
    prefix_block_walk<false><<<grid, 256, (size_t)cap * 24, s>>>(scores, T, stride, (int)nb, (int)sbs, (int)nsb, K,
                                                                 cap, w.qval, w.qidx, w.qlen, fin_v, fin_i, fin_l,
                                                                 blk, evict);
  PFA_CHECK_LAUNCH("pfa_proto_prefix/walk");
  return PFA_OK;
}

#define PFA_PREFIX_SETUP(NAME)                                                                              \
  clear_error();                                                                                            \
  PFA_CHECK_ARG(proto_scores && workspace && B > 0 && T > 0 && K > 0 && K <= kPrefixMaxK,                   \
                NAME ": bad arguments (B=%d T=%lld K=%d, K <= %d)", B, (long long)T, K, kPrefixMaxK);       \
  PFA_CHECK_ARG(T < ((int64_t)1 << 31), NAME ": T too large");                                              \
  const int64_t nb = (T + kBlk - 1) / kBlk;                                                                 \
  const int64_t sbs = prefix_sbs(nb);                                                                       \
  const int64_t nsb = (nb + sbs - 1) / sbs;                                                                 \
  const size_t need = prefix_ws_bytes(B, T, nb, nsb, K, nullptr, nullptr);                                  \
  if (ws_bytes < need) {                                                                                    \
    set_error(NAME ": workspace %zu < %zu", ws_bytes, need);                                               \
    return PFA_E_WORKSPACE;                                                                                 \
  }                                                                                                         \
  PrefixWs w;                                                                                               \
  prefix_ws_bytes(B, T, nb, nsb, K, &w, (char*)workspace);                                                  \
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
