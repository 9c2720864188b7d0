// Shortlist candidates: prototype prefix top-k and the packed builder.
//
// Prototype prefix top-k (replaces the O(rows*T) masked torch.topk of
// sparse_attn.py:260-300).  For batch b and token t the set is the
// min(t+1, K) largest scores among positions 0..t, ties to the lowest
// index.  Tokens are cut into blocks of 64:
//   1. block_sort : each block's scores sorted (value desc, index asc) by a
//                   wave-wide bitonic network in registers, truncated to K;
//   2. scan_level : Hillis-Steele inclusive scan over blocks whose operator
//                   is "top-K of the union of two sorted lists" (merge path);
//   3. block_walk : one wave per block starts from the exclusive prefix
//                   (re-sorted by index in LDS) and walks its 64 tokens in
//                   order, replacing the current minimum whenever a better
//                   score arrives, writing each token's set sorted by index.
//
// Builder (replaces sparse_attn.py:376-596).  Per row, everything below the
// local window start `lo` (strided anchors in closed form, the prototype set
// prefix below lo, extra candidates) is merged with a merge-path co-rank,
// de-duplicated, and followed by the window lo..t and t-padding.  One wave
// per row; the row of L indices is written with 16-byte stores.
#include "pfa_common.h"

namespace pfa {

constexpr int kBlk = 64;  // tokens per prefix block (one wave)

struct PrefixWs {
  float* val[2];
  int32_t* idx[2];
  int32_t* len[2];
};

static size_t prefix_ws_bytes(int64_t B, int64_t nb, int64_t K) {
  size_t lists = (size_t)B * nb * K;
  size_t one = ((lists * 4 + 255) & ~(size_t)255);
  size_t lens = (((size_t)B * nb * 4 + 255) & ~(size_t)255);
  return 2 * (2 * one + lens);
}

static PrefixWs carve_prefix(void* ws, int64_t B, int64_t nb, int64_t K) {
  size_t lists = (size_t)B * nb * K;
  size_t one = ((lists * 4 + 255) & ~(size_t)255);
  size_t lens = (((size_t)B * nb * 4 + 255) & ~(size_t)255);
  char* p = (char*)ws;
  PrefixWs w;
  for (int i = 0; i < 2; ++i) {
    w.val[i] = (float*)p; p += one;
    w.idx[i] = (int32_t*)p; p += one;
    w.len[i] = (int32_t*)p; p += lens;
  }
  return w;
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
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  int64_t t = (int64_t)j * kBlk + lane;
  if (evict != nullptr && t < T) evict[(int64_t)b * T + t] = INT32_MAX;
  float v = -INFINITY;
  int i = INT32_MAX;
  if (t < T) { v = scores[(int64_t)b * stride + t]; i = (int)t; }
  wave_bitonic_best_first(v, i);
  int64_t n = T - (int64_t)j * kBlk;
  if (n > kBlk) n = kBlk;
  if (n > K) n = K;
  int64_t base = ((int64_t)b * nb + j) * K;
  if (lane < n) { oval[base + lane] = v; oidx[base + lane] = i; }
  if (lane == 0) olen[(int64_t)b * nb + j] = (int)n;
}

// out[j] = topK(in[j-d] U in[j]) for j >= d, else copy.  Both inputs are
// staged in LDS (2 x K x 8 bytes) so the co-rank searches stay on chip.
__global__ void __launch_bounds__(64)
prefix_scan_level(int nb, int K, int d, const float* __restrict__ ival, const int32_t* __restrict__ iidx,
                  const int32_t* __restrict__ ilen, float* __restrict__ oval, int32_t* __restrict__ oidx,
                  int32_t* __restrict__ olen) {
  extern __shared__ char smem[];
  float* av = (float*)smem;
  int32_t* ai = (int32_t*)(av + K);
  float* bv = (float*)(ai + K);
  int32_t* bi = (int32_t*)(bv + K);
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t rowj = (int64_t)b * nb + j;
  const int nbl = ilen[rowj];
  if (j < d) {
    for (int p = lane; p < nbl; p += 64) { oval[rowj * K + p] = ival[rowj * K + p]; oidx[rowj * K + p] = iidx[rowj * K + p]; }
    if (lane == 0) olen[rowj] = nbl;
    return;
  }
  const int64_t rowa = rowj - d;
  const int na = ilen[rowa];
  for (int p = lane; p < na; p += 64) { av[p] = ival[rowa * K + p]; ai[p] = iidx[rowa * K + p]; }
  for (int p = lane; p < nbl; p += 64) { bv[p] = ival[rowj * K + p]; bi[p] = iidx[rowj * K + p]; }
  __syncthreads();
  const int m = min(K, na + nbl);
  for (int p = lane; p < m; p += 64) {
    int lo = max(0, p - nbl), hi = min(p, na);
    while (lo < hi) {
      int mid = (lo + hi) >> 1;
      if (better(av[mid], ai[mid], bv[p - 1 - mid], bi[p - 1 - mid])) lo = mid + 1;
      else hi = mid;
    }
    int ia = lo, ib = p - lo;
    bool take_a = ia < na && (ib >= nbl || better(av[ia], ai[ia], bv[ib], bi[ib]));
    oval[rowj * K + p] = take_a ? av[ia] : bv[ib];
    oidx[rowj * K + p] = take_a ? ai[ia] : bi[ib];
  }
  if (lane == 0) olen[rowj] = m;
}

// LDS bitonic sort by index ascending of n (<= cap, power of two) entries.
__device__ void lds_sort_by_index(float* v, int32_t* ix, int cap) {
  const int lane = threadIdx.x & 63;
  for (int k = 2; k <= cap; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int e = lane; e < cap; e += 64) {
        int p = e ^ j;
        if (p > e) {
          bool up = (e & k) == 0;
          int a = ix[e], c = ix[p];
          bool swap = up ? (a > c) : (a < c);
          if (swap) {
            ix[e] = c; ix[p] = a;
            float tv = v[e]; v[e] = v[p]; v[p] = tv;
          }
        }
      }
      __syncthreads();
    }
  }
}

// One wave per (batch, block).  LDS: value + index arrays of `cap` entries
// (cap = next power of two >= K).
__global__ void __launch_bounds__(64)
prefix_block_walk(const float* __restrict__ scores, int64_t T, int64_t stride, int nb, int K, int cap,
                  const float* __restrict__ pval, const int32_t* __restrict__ pidx, const int32_t* __restrict__ plen,
                  int32_t* __restrict__ sets, int32_t* __restrict__ evict) {
  extern __shared__ char smem[];
  float* v = (float*)smem;
  int32_t* ix = (int32_t*)(v + cap);
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  int n = 0;
  if (j > 0) {
    const int64_t row = (int64_t)b * nb + (j - 1);
    n = plen[row];
    for (int p = lane; p < cap; p += 64) {
      if (p < n) { v[p] = pval[row * K + p]; ix[p] = pidx[row * K + p]; }
      else { v[p] = -INFINITY; ix[p] = INT32_MAX; }
    }
  } else {
    for (int p = lane; p < cap; p += 64) { v[p] = -INFINITY; ix[p] = INT32_MAX; }
  }
  __syncthreads();
  if (n > 1) lds_sort_by_index(v, ix, cap);
  const int64_t t0 = (int64_t)j * kBlk;
  const int64_t t1 = min(T, t0 + kBlk);
  for (int64_t t = t0; t < t1; ++t) {
    float s = scores[(int64_t)b * stride + t];
    if (n < K) {
      if (lane == 0) { v[n] = s; ix[n] = (int)t; }
      ++n;
      __syncthreads();
    } else {
      // worst element of the current set
      float wv = INFINITY;
      int wi = -1, wp = -1;
      for (int p = lane; p < n; p += 64) {
        if (wp < 0 || better(wv, wi, v[p], ix[p])) { wv = v[p]; wi = ix[p]; wp = p; }
      }
      for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(wv, off, 64);
        int oi = __shfl_xor(wi, off, 64), op = __shfl_xor(wp, off, 64);
        bool take;
        if (op < 0) take = false;
        else if (wp < 0) take = true;
        else take = better(wv, wi, ov, oi);
        if (take) { wv = ov; wi = oi; wp = op; }
      }
      if (!better(s, (int)t, wv, wi)) {
        if (evict != nullptr && lane == 0) evict[(int64_t)b * T + t] = (int32_t)t;  // never enters
      } else {
        if (evict != nullptr && lane == 0) evict[(int64_t)b * T + wi] = (int32_t)t;  // wi leaves at t
        float tv[4];
        int ti[4];
        int cnt = 0;
        for (int p = wp + 1 + lane; p < n && cnt < 4; p += 64, ++cnt) { tv[cnt] = v[p]; ti[cnt] = ix[p]; }
        // n - wp - 1 may exceed 256: loop in rounds
        int p0 = wp + 1;
        while (true) {
          __syncthreads();
          int c = 0;
          for (int p = p0 + lane; p < n && c < 4; p += 64, ++c) { v[p - 1] = tv[c]; ix[p - 1] = ti[c]; }
          p0 += 256;
          __syncthreads();
          if (p0 >= n) break;
          c = 0;
          for (int p = p0 + lane; p < n && c < 4; p += 64, ++c) { tv[c] = v[p]; ti[c] = ix[p]; }
        }
        if (lane == 0) { v[n - 1] = s; ix[n - 1] = (int)t; }
        __syncthreads();
      }
    }
    int32_t* out = sets + ((int64_t)b * T + t) * K;
    for (int p = lane; p < K; p += 64) out[p] = (p < n) ? ix[p] : (int32_t)t;
  }
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
                       int64_t seq_len, int L, int local_w, int stride, int slots,
                       const int32_t* __restrict__ proto_sets, int K, int64_t proto_len,
                       const int32_t* __restrict__ extra, const int32_t* __restrict__ extra_len, int ew,
                       int qcap, int bcap, void* __restrict__ cand_out, void* __restrict__ len_out) {
  extern __shared__ int32_t lds_i[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int32_t* Q = lds_i + wid * (qcap + bcap);
  int32_t* Bb = Q + qcap;
  const int64_t r = (int64_t)blockIdx.x * kBuildWaves + wid;
  if (r >= N) return;
  const int64_t t = rows[r];
  const int64_t b = row_batch ? row_batch[r] : 0;

  int64_t lo, wlen;
  if (local_w > 0) { wlen = min<int64_t>(t + 1, local_w); lo = t - wlen + 1; }
  else { wlen = 1; lo = t; }

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
  const int64_t nB = min<int64_t>(nb_out, L);
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
      int4* o4 = (int4*)out;
      for (int q = lane; q < L / 4; q += 64) {
        int64_t p = 4 * (int64_t)q;
        o4[q] = make_int4((int)value_at(p), (int)value_at(p + 1), (int)value_at(p + 2), (int)value_at(p + 3));
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

extern "C" int pfa_proto_prefix_workspace_size(int B, int64_t T, int K, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && B >= 0 && T >= 0 && K > 0, "pfa_proto_prefix_workspace_size: bad arguments");
  int64_t nb = (T + kBlk - 1) / kBlk;
  if (nb < 1) nb = 1;
  *bytes = prefix_ws_bytes(B, nb, K);
  return PFA_OK;
}

extern "C" int pfa_proto_prefix_topk(const float* proto_scores, int B, int64_t T, int64_t score_stride, int K,
                                     int32_t* sets_out, int32_t* evict_out, void* workspace, size_t ws_bytes,
                                     void* stream) {
  clear_error();
  PFA_CHECK_ARG(proto_scores && sets_out && workspace && B > 0 && T > 0 && K > 0 && K <= 4096,
                "pfa_proto_prefix_topk: bad arguments (B=%d T=%lld K=%d)", B, (long long)T, K);
  int64_t nb = (T + kBlk - 1) / kBlk;
  PFA_CHECK_ARG(nb < 65536 * 64, "pfa_proto_prefix_topk: T too large");
  size_t need = prefix_ws_bytes(B, nb, K);
  if (ws_bytes < need) {
    set_error("pfa_proto_prefix_topk: workspace %zu < %zu", ws_bytes, need);
    return PFA_E_WORKSPACE;
  }
  PrefixWs w = carve_prefix(workspace, B, nb, K);
  hipStream_t s = as_stream(stream);
  dim3 grid((unsigned)nb, (unsigned)B);
  prefix_block_sort<<<grid, 64, 0, s>>>(proto_scores, T, score_stride, (int)nb, K, w.val[0], w.idx[0], w.len[0],
                                             evict_out);
  PFA_CHECK_LAUNCH("pfa_proto_prefix_topk/sort");
  int cur = 0;
  for (int64_t d = 1; d < nb; d <<= 1) {
    prefix_scan_level<<<grid, 64, (size_t)K * 16, s>>>((int)nb, K, (int)d, w.val[cur], w.idx[cur], w.len[cur], w.val[cur ^ 1],
                                          w.idx[cur ^ 1], w.len[cur ^ 1]);
    PFA_CHECK_LAUNCH("pfa_proto_prefix_topk/scan");
    cur ^= 1;
  }
  int cap = 1;
  while (cap < K) cap <<= 1;
  size_t lds = (size_t)cap * 8;
  PFA_CHECK_ARG(lds <= 160 * 1024, "pfa_proto_prefix_topk: K=%d too large for LDS", K);
  prefix_block_walk<<<grid, 64, lds, s>>>(proto_scores, T, score_stride, (int)nb, K, cap, w.val[cur], w.idx[cur],
                                          w.len[cur], sets_out, evict_out);
  PFA_CHECK_LAUNCH("pfa_proto_prefix_topk/walk");
  return PFA_OK;
}

extern "C" int pfa_shortlist_build(const int32_t* rows, const int32_t* row_batch, int64_t N, int64_t seq_len, int L,
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
  size_t lds = (size_t)kBuildWaves * (qcap + bcap) * 4;
  PFA_CHECK_ARG(lds <= 160 * 1024, "pfa_shortlist_build: LDS need %zu too large (L=%d K=%d slots=%d)", lds, L,
                proto_k, anchor_slots);
  PFA_CHECK_ARG(!extra || (extra_width + proto_k) <= 64 * 8, "pfa_shortlist_build: extra merge too wide");
  unsigned blocks = (unsigned)((N + kBuildWaves - 1) / kBuildWaves);
  hipStream_t s = as_stream(stream);
#define PFA_BUILD(C64, L64)                                                                                   \
  shortlist_build_kernel<C64, L64><<<blocks, 64 * kBuildWaves, lds, s>>>(                                     \
      rows, row_batch, N, seq_len, L, local_w, anchor_stride, anchor_slots, proto_sets, proto_sets ? proto_k : 0, \
      proto_len, extra, extra_len, extra ? extra_width : 0, qcap, bcap, cand_out, len_out)
  if (cand_is_i64) {
    if (len_is_i64) PFA_BUILD(true, true); else PFA_BUILD(true, false);
  } else {
    if (len_is_i64) PFA_BUILD(false, true); else PFA_BUILD(false, false);
  }
#undef PFA_BUILD
  PFA_CHECK_LAUNCH("pfa_shortlist_build");
  return PFA_OK;
}
