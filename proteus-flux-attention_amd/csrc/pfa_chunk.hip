// Device stages of the chunked shortlist pipeline:
//   * per-chunk salience top-k with nucleus truncation
//     (reference tools/chunked_shortlist.py:140-208),
//   * the global shortlist merge (chunked_shortlist.py:211-254),
//   * per-(head, row) symmetric int8 quantisation of shortlisted K/V,
//   * RoPE on arbitrary rows (a slice of queries, or gathered shortlist keys
//     at their original positions).
//
// Orders: every selection sorts 64-bit keys ascending.  A score s is mapped
// to the order-preserving u32 `ord(s)`; the key (~ord(s) << 32 | position)
// ascending is "score descending, then position ascending" (ties go to the
// lowest position, the contract of every top-k in this library).
//
// Sorting: a bitonic network over a power-of-two array of u64 keys.  Tiles
// of kSortTile keys are sorted in LDS by one workgroup; larger arrays add
// global compare-exchange passes for the strides >= kSortTile.  The whole
// array lives in the caller's workspace.
#include "pfa_common.h"
#include "pfa_radix.h"

// RoPE and quantisation round every elementwise product on its own, as the
// reference's separate tensor ops do: no fused multiply-add contraction.
#pragma clang fp contract(off)

namespace pfa {

constexpr int kSortTile = 8192;  // u64 keys per LDS tile (64 KiB)
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;

__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool finite_f(float f) { return (__float_as_uint(f) & 0x7f800000u) != 0x7f800000u; }

// ---------------------------------------------------------------------
// bitonic sort of u64 keys (ascending); n is a power of two
// ---------------------------------------------------------------------
// Bitonic stages k = 2 .. kmax over s[0, m) in LDS; element i of the tile is
// element base + i of the whole array (which fixes each pair's direction).
__device__ __forceinline__ void lds_bitonic(uint64_t* s, int m, int kmax, int64_t base) {
  for (int k = 2; k <= kmax; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < m; i += blockDim.x) {
        const int l = i ^ j;
        if (l > i) {
          const bool up = ((base + i) & k) == 0;
          const uint64_t a = s[i], b = s[l];
          if ((a > b) == up) {
            s[i] = b;
            s[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__global__ void __launch_bounds__(1024) bitonic_tile_sort(uint64_t* keys, int64_t n, int kmax) {
  __shared__ uint64_t s[kSortTile];
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  const int m = (int)(n - base < kSortTile ? n - base : kSortTile);
  for (int i = threadIdx.x; i < m; i += blockDim.x) s[i] = keys[base + i];
  __syncthreads();
  lds_bitonic(s, m, kmax, base);
  for (int i = threadIdx.x; i < m; i += blockDim.x) keys[base + i] = s[i];
}

// merge stage k, strides j < kSortTile, one tile per workgroup
__global__ void __launch_bounds__(1024) bitonic_tile_merge(uint64_t* keys, int64_t k) {
  __shared__ uint64_t s[kSortTile];
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += blockDim.x) s[i] = keys[base + i];
  __syncthreads();
  const bool up = (base & k) == 0;  // k > kSortTile: the direction is constant over the tile
  for (int j = kSortTile >> 1; j > 0; j >>= 1) {
    for (int i = threadIdx.x; i < kSortTile; i += blockDim.x) {
      const int l = i ^ j;
      if (l > i) {
        const uint64_t a = s[i], b = s[l];
        if ((a > b) == up) {
          s[i] = b;
          s[l] = a;
        }
      }
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < kSortTile; i += blockDim.x) keys[base + i] = s[i];
}

// merge stage k, one stride j >= kSortTile, over all n/2 pairs
__global__ void __launch_bounds__(256) bitonic_global_pass(uint64_t* keys, int64_t n, int64_t k, int64_t j) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n / 2) return;
  const int64_t i = (p / j) * 2 * j + (p % j);
  const int64_t l = i + j;
  const bool up = (i & k) == 0;
  const uint64_t a = keys[i], b = keys[l];
  if ((a > b) == up) {
    keys[i] = b;
    keys[l] = a;
  }
}

static int64_t pow2_ceil(int64_t n) {
  int64_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

static int sort_u64(uint64_t* keys, int64_t n, hipStream_t s, const char* what) {
  if (n <= 1) return PFA_OK;
  const int64_t tiles = (n + kSortTile - 1) / kSortTile;
  bitonic_tile_sort<<<(unsigned)tiles, 1024, 0, s>>>(keys, n, (int)(n < kSortTile ? n : kSortTile));
  PFA_CHECK_LAUNCH(what);
  for (int64_t k = 2 * (int64_t)kSortTile; k <= n; k <<= 1) {
    for (int64_t j = k >> 1; j >= kSortTile; j >>= 1) {
      const int64_t pairs = n / 2;
      bitonic_global_pass<<<(unsigned)((pairs + 255) / 256), 256, 0, s>>>(keys, n, k, j);
      PFA_CHECK_LAUNCH(what);
    }
    bitonic_tile_merge<<<(unsigned)tiles, 1024, 0, s>>>(keys, k);
    PFA_CHECK_LAUNCH(what);
  }
  return PFA_OK;
}

// ---------------------------------------------------------------------
// block-wide helpers for one 1024-thread workgroup
// ---------------------------------------------------------------------
struct BlockScratch {
  float f[kSelWaves];
  int i[kSelWaves];
  int carry;
  int total;
};

__device__ __forceinline__ float block_sum(float v, BlockScratch& sc) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sc.f[w] = v;
  __syncthreads();
  float r = 0.f;
  for (int k = 0; k < kSelWaves; ++k) r += sc.f[k];  // fixed order: deterministic
  return r;
}

__device__ __forceinline__ int block_count(bool flag, BlockScratch& sc) {
  const int w = threadIdx.x >> 6;
  const int c = __popcll(__ballot(flag));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sc.i[w] = c;
  __syncthreads();
  int r = 0;
  for (int k = 0; k < kSelWaves; ++k) r += sc.i[k];
  return r;
}

// Exclusive rank of `flag` among the flags of this 1024-element step in
// thread order; returns the step's total through `total`.
__device__ __forceinline__ int block_rank(bool flag, BlockScratch& sc, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t bal = __ballot(flag);
  __syncthreads();
  if (lane == 0) sc.i[w] = __popcll(bal);
  __syncthreads();
  int before = 0, tot = 0;
  for (int k = 0; k < kSelWaves; ++k) {
    before += k < w ? sc.i[k] : 0;
    tot += sc.i[k];
  }
  total = tot;
  return before + __popcll(bal & ((1ull << lane) - 1ull));
}

// ---------------------------------------------------------------------
// chunk salience top-k
// ---------------------------------------------------------------------
__device__ __forceinline__ float masked_score(const float* sc, const uint8_t* mk, int64_t i) {
  const float v = sc[i];
  return (mk != nullptr && mk[i] == 0) ? -INFINITY : v;
}
__device__ __forceinline__ float safe_score(float v) { return finite_f(v) ? v : -1e9f; }

struct ChunkKeys {
  const float* scores;
  const uint8_t* mask;
  __device__ __forceinline__ uint32_t key(int, int64_t i) const {
    return ord_key(safe_score(masked_score(scores, mask, i)));
  }
};

__device__ __forceinline__ float ord_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// After the radix passes: writes the selected keys (~ord(score) << 32 |
// position) into keys[0, limit) -- keys above the cut in any slot order,
// then the `remaining` lowest-position ties -- pads keys[limit, limit_pow2)
// with ~0, and gathers the emit statistics (largest safe score, finite
// count).  grid = groups_of(n).
__global__ void __launch_bounds__(rsel::kThreads) chunk_keys_kernel(ChunkKeys src, int64_t n, int64_t limit_pow2,
                                                                    unsigned char* ws, uint64_t* __restrict__ keys) {
  __shared__ uint32_t sm[rsel::kThreads / 64];
  __shared__ uint32_t s_base;
  const int w = blockIdx.x, tid = threadIdx.x;
  rsel::State* st = reinterpret_cast<rsel::State*>(ws);
  const int32_t* tiebase = reinterpret_cast<const int32_t*>(ws + rsel::layout(gridDim.x).tiebase);
  const int64_t i0 = (int64_t)w * rsel::kSpan + (int64_t)tid * rsel::kPer;
  uint32_t kv[rsel::kPer];
  int nfin = 0;
#pragma unroll
  for (int e = 0; e < rsel::kPer; ++e) {
    kv[e] = 0u;
    if (i0 + e < n) {
      const float v = masked_score(src.scores, src.mask, i0 + e);
      nfin += finite_f(v) ? 1 : 0;
      kv[e] = ord_key(safe_score(v));
    }
  }
  // statistics of this workgroup (reduced by the emit kernel)
  uint32_t mx = 0u;
#pragma unroll
  for (int e = 0; e < rsel::kPer; ++e) mx = i0 + e < n && kv[e] > mx ? kv[e] : mx;
  for (int o = 32; o > 0; o >>= 1) {
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, o, 64));
    nfin += __shfl_xor(nfin, o, 64);
  }
  __shared__ uint32_t s_mx[rsel::kThreads / 64];
  __shared__ int s_fin[rsel::kThreads / 64];
  if ((tid & 63) == 0) {
    s_mx[tid >> 6] = mx;
    s_fin[tid >> 6] = nfin;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t m2 = 0u;
    int f2 = 0;
    for (int k = 0; k < rsel::kThreads / 64; ++k) {
      m2 = max(m2, s_mx[k]);
      f2 += s_fin[k];
    }
    uint32_t* ws2 = reinterpret_cast<uint32_t*>(ws + rsel::layout(gridDim.x).wstat) + 2 * w;
    ws2[0] = m2;
    ws2[1] = (uint32_t)f2;
  }
  const int limit = st->need;
  if ((int64_t)limit >= n) {
    // everything is selected: key i in slot i
#pragma unroll
    for (int e = 0; e < rsel::kPer; ++e)
      if (i0 + e < n) keys[i0 + e] = ((uint64_t)(~kv[e]) << 32) | (uint64_t)(uint32_t)(i0 + e);
  } else {
    bool sel[rsel::kPer], above[rsel::kPer];
    uint32_t rank[rsel::kPer];
    const int remaining = st->remaining;
    rsel::select_keys(kv, i0, n, st->prefix, remaining, tiebase[w], sm, sel, above, rank);
    uint32_t na = 0u;
#pragma unroll
    for (int e = 0; e < rsel::kPer; ++e) na += above[e] ? 1u : 0u;
    uint32_t tot = 0u;
    uint32_t pos = rsel::block_excl_scan(na, sm, tot);
    if (tid == 0) s_base = tot != 0u ? atomicAdd(&st->slot, tot) : 0u;
    __syncthreads();
    pos += s_base;
    const uint32_t n_above = (uint32_t)(limit - remaining);
#pragma unroll
    for (int e = 0; e < rsel::kPer; ++e) {
      const uint64_t key = ((uint64_t)(~kv[e]) << 32) | (uint64_t)(uint32_t)(i0 + e);
      if (above[e]) {
        if (pos < n_above) keys[pos] = key;  // exactly n_above keys lie above the cut
        ++pos;
      } else if (sel[e]) {
        keys[n_above + rank[e]] = key;
      }
    }
  }
  if (w == 0)
    for (int64_t j = (limit < n ? limit : n) + tid; j < limit_pow2; j += rsel::kThreads) keys[j] = ~0ull;
}

// The selected keys in order, the nucleus cut and the outputs.  `keys` holds
// limit_pow2 keys; sort_here: they are not sorted yet (limit_pow2 <= kSortTile)
// and are sorted in LDS first.  wstat: the keys kernel's per-workgroup
// statistics (largest order key, finite count) of `groups` workgroups.
__global__ void __launch_bounds__(kSelThreads) chunk_emit_kernel(const float* __restrict__ scores,
                                                               const uint8_t* __restrict__ mask, int64_t n,
                                                               const uint64_t* __restrict__ keys, int limit,
                                                               int limit_pow2, int sort_here, float top_p,
                                                               const uint32_t* __restrict__ wstat, int groups,
                                                               int64_t offset, int drop_nonfinite,
                                                               float* __restrict__ vals_out,
                                                               int64_t* __restrict__ idx_out, int32_t* count_out) {
  __shared__ BlockScratch sc;
  __shared__ int s_keep;
  __shared__ uint64_t s_keys[kSortTile];
  const int tid = threadIdx.x;
  if (limit <= 0) {  // nothing selectable
    if (tid == 0) *count_out = 0;
    return;
  }
  // statistics over the workgroups of the keys kernel
  uint32_t mo = 0u;
  int fin = 0;
  for (int g = tid; g < groups; g += kSelThreads) {
    mo = max(mo, wstat[2 * g]);
    fin += (int)wstat[2 * g + 1];
  }
  for (int o = 32; o > 0; o >>= 1) {
    mo = max(mo, (uint32_t)__shfl_xor((int)mo, o, 64));
    fin += __shfl_xor(fin, o, 64);
  }
  if ((tid & 63) == 0) {
    sc.i[tid >> 6] = fin;
    sc.f[tid >> 6] = __uint_as_float(mo);
  }
  __syncthreads();
  fin = 0;
  mo = 0u;
  for (int k = 0; k < kSelWaves; ++k) {
    fin += sc.i[k];
    mo = max(mo, __float_as_uint(sc.f[k]));
  }
  if (fin <= 0) {  // no finite score
    if (tid == 0) *count_out = 0;
    return;
  }
  const uint64_t* K = keys;
  if (sort_here && limit <= kSelThreads) {
    // rank sort: the keys are distinct (they carry the position), so key t
    // goes to slot #(keys below it); one key per thread, kSortTile/2 slots
    // of LDS for the input
    uint64_t* in = s_keys + kSortTile / 2;
    if (tid < limit) in[tid] = keys[tid];
    __syncthreads();
    if (tid < limit) {
      const uint64_t k = in[tid];
      int r = 0;
      for (int j = 0; j < limit; ++j) r += in[j] < k ? 1 : 0;
      s_keys[r] = k;
    }
    __syncthreads();
    K = s_keys;
  } else if (sort_here) {
    for (int i = tid; i < limit_pow2; i += kSelThreads) s_keys[i] = keys[i];
    __syncthreads();
    lds_bitonic(s_keys, limit_pow2, limit_pow2, 0);
    K = s_keys;
  }
  const float mx = ord_to_float(mo);
  int keep = limit;
  if (top_p < 1.0f) {
    // softmax denominator over the chunk (each thread sums its strided
    // scores, then the fixed-order block sum)
    float acc = 0.f;
    for (int64_t i = tid; i < n; i += kSelThreads) acc += expf(safe_score(masked_score(scores, mask, i)) - mx);
    const float z = block_sum(acc, sc);
    // mass_r = cumulative softmax probability in selection order; keep =
    // #(mass < top_p) (+1 when that is not every token), clamped
    float carry = 0.f;
    int below = 0;
    for (int base = 0; base < limit; base += kSelThreads) {
      const int r = base + tid;
      float p = 0.f;
      if (r < limit) {
        const int64_t i = (int64_t)(uint32_t)(K[r] & 0xffffffffu);
        p = expf(safe_score(masked_score(scores, mask, i)) - mx) / z;
      }
      // inclusive scan of p over the step (wave scan, then wave totals)
      float x = p;
      const int lane = tid & 63, w = tid >> 6;
      for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
      }
      __syncthreads();
      if (lane == 63) sc.f[w] = x;
      __syncthreads();
      float before = carry;
      float tot = carry;
      for (int k = 0; k < kSelWaves; ++k) {
        before += k < w ? sc.f[k] : 0.f;
        tot += sc.f[k];
      }
      const float mass = before + x;
      below += block_count(r < limit && mass < top_p, sc);
      carry = tot;
    }
    if (below >= limit) keep = limit;
    else keep = min(limit, max(1, below + 1));
  }
  if (tid == 0) s_keep = keep;
  __syncthreads();
  keep = s_keep;
  // selected entries in order (non-finite values dropped on request)
  int out = 0;
  for (int base = 0; base < keep; base += kSelThreads) {
    const int r = base + tid;
    float v = 0.f;
    int64_t i = 0;
    if (r < keep) {
      i = (int64_t)(uint32_t)(K[r] & 0xffffffffu);
      v = masked_score(scores, mask, i);
    }
    const bool ok = r < keep && (!drop_nonfinite || finite_f(v));
    int tot = 0;
    const int pos = out + block_rank(ok, sc, tot);
    if (ok) {
      vals_out[pos] = v;
      idx_out[pos] = i + offset;
    }
    out += tot;
  }
  if (tid == 0) *count_out = out;
}

// ---------------------------------------------------------------------
// global shortlist merge
// ---------------------------------------------------------------------
__global__ void __launch_bounds__(256) fin_keys_score(const float* __restrict__ scores, int64_t n, int64_t n2,
                                                      uint64_t* __restrict__ a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n2) return;
  a[i] = i < n ? (((uint64_t)(~ord_key(scores[i])) << 32) | (uint64_t)(uint32_t)i) : ~0ull;
}

__global__ void __launch_bounds__(256) fin_keys_index(const uint64_t* __restrict__ a, const int64_t* __restrict__ idx,
                                                      int64_t n, int64_t n2, uint64_t* __restrict__ b) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n2) return;
  if (r < n) {
    const int64_t pos = (int64_t)(uint32_t)(a[r] & 0xffffffffu);
    const uint32_t ix = (uint32_t)((int32_t)idx[pos]) ^ 0x80000000u;  // signed order
    b[r] = ((uint64_t)ix << 32) | (uint64_t)(~(uint32_t)r);
  } else {
    b[r] = ~0ull;
  }
}

__global__ void __launch_bounds__(kSelThreads) fin_emit_kernel(const float* __restrict__ scores,
                                                             const int64_t* __restrict__ idx, int64_t n,
                                                             int64_t max_tokens, const uint64_t* __restrict__ a,
                                                             const uint64_t* __restrict__ b,
                                                             int32_t* __restrict__ ord, int64_t* __restrict__ keep_idx,
                                                             float* __restrict__ keep_score, int32_t* count_out) {
  __shared__ BlockScratch sc;
  const int tid = threadIdx.x;
  // survivors: the first entry of each index group in b (the last of that
  // index in score order); ord[r] = -1 unless rank r survives
  for (int64_t r = tid; r < n; r += kSelThreads) ord[r] = -1;
  __syncthreads();
  for (int64_t u = tid; u < n; u += kSelThreads) {
    const bool first = u == 0 || (b[u] >> 32) != (b[u - 1] >> 32);
    if (first) ord[(uint32_t)~(uint32_t)(b[u] & 0xffffffffu)] = 0;
  }
  __syncthreads();
  // ordinal of each survivor in score order
  int carry = 0;
  for (int64_t base = 0; base < n; base += kSelThreads) {
    const int64_t r = base + tid;
    const bool s = r < n && ord[r] == 0;
    int tot = 0;
    const int k = carry + block_rank(s, sc, tot);
    __syncthreads();
    if (s) ord[r] = k;
    carry += tot;
  }
  __syncthreads();
  // emit the selected survivors in index order (b's order)
  int out = 0;
  for (int64_t base = 0; base < n; base += kSelThreads) {
    const int64_t u = base + tid;
    bool take = false;
    uint32_t r = 0;
    if (u < n) {
      const bool first = u == 0 || (b[u] >> 32) != (b[u - 1] >> 32);
      r = ~(uint32_t)(b[u] & 0xffffffffu);
      take = first && (int64_t)ord[r] < max_tokens;
    }
    int tot = 0;
    const int pos = out + block_rank(take, sc, tot);
    if (take) {
      const int64_t p = (int64_t)(uint32_t)(a[r] & 0xffffffffu);
      keep_idx[pos] = idx[p];
      keep_score[pos] = scores[p];
    }
    out += tot;
  }
  if (tid == 0) *count_out = out;
}

// ---------------------------------------------------------------------
// per-(head, row) int8 quantisation: one wave per (row, head)
// ---------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) quant_rows_kernel(const typename Elem<DT>::T* __restrict__ src, int64_t n_rows,
                                                         int64_t row_stride, int H, int D, int8_t* __restrict__ dst,
                                                         float* __restrict__ scales) {
  const int64_t wv = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wv >= n_rows * H) return;
  const int64_t r = wv / H;
  const int h = (int)(wv % H);
  const typename Elem<DT>::T* row = src + r * row_stride + (int64_t)h * D;
  float amax = 0.f;
  for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(load_f<DT>(row + d)));
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  const float sc = fmaxf(__fdiv_rn(amax, 127.0f), 1e-6f);
  int8_t* out = dst + ((int64_t)h * n_rows + r) * D;
  for (int d = lane; d < D; d += 64) {
    float q = rintf(__fdiv_rn(load_f<DT>(row + d), sc));
    q = fminf(fmaxf(q, -127.f), 127.f);
    out[d] = (int8_t)(int)q;
  }
  if (lane == 0) scales[(int64_t)h * n_rows + r] = sc;
}

// ---------------------------------------------------------------------
// RoPE on rows: H heads of D elements at x + r*row_stride; table row =
// positions[r] (or pos_offset + r).  Same rounding as pfa_rope_qk_inplace.
// ---------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) rope_rows_kernel(typename Elem<DT>::T* x, int64_t n_rows, int64_t row_stride,
                                                        int H, int D, const typename Elem<DT>::T* cos_tab,
                                                        const typename Elem<DT>::T* sin_tab,
                                                        const int32_t* positions, int64_t pos_offset) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int half = D / 2;
  if (i >= n_rows * H * half) return;
  const int pair = (int)(i % half);
  const int64_t rest = i / half;
  const int h = (int)(rest % H);
  const int64_t r = rest / H;
  const int64_t t = positions ? (int64_t)positions[r] : pos_offset + r;
  typename Elem<DT>::T* base = x + r * row_stride + (int64_t)h * D + 2 * pair;
  const float xe = load_f<DT>(base), xo = load_f<DT>(base + 1);
  const float ce = load_f<DT>(cos_tab + t * D + 2 * pair), co = load_f<DT>(cos_tab + t * D + 2 * pair + 1);
  const float se = load_f<DT>(sin_tab + t * D + 2 * pair), so = load_f<DT>(sin_tab + t * D + 2 * pair + 1);
  store_f<DT>(base, round_to<DT>(round_to<DT>(xe * ce) + round_to<DT>(-xo * se)));
  store_f<DT>(base + 1, round_to<DT>(round_to<DT>(xo * co) + round_to<DT>(xe * so)));
}

// The same, 8 elements (4 pairs) per thread with 16-byte loads and stores,
// for D a multiple of 8 and 16-byte aligned rows and tables (rope_rotate8:
// the bits of the pair formula above).
template <int DT>
__global__ void __launch_bounds__(256) rope_rows8_kernel(typename Elem<DT>::T* x, int64_t n_rows,
                                                         int64_t row_stride, int H, int D,
                                                         const typename Elem<DT>::T* cos_tab,
                                                         const typename Elem<DT>::T* sin_tab,
                                                         const int32_t* positions, int64_t pos_offset) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = H * (D / 8);
  if (i >= n_rows * per_row) return;
  const int64_t r = i / per_row;
  const int e = (int)(i - r * per_row) * 8;  // element offset within the row's H*D
  const int d = e % D;
  const int64_t t = positions ? (int64_t)positions[r] : pos_offset + r;
  typename Elem<DT>::T* base = x + r * row_stride + e;
  float xv[8], cv[8], sv[8], o[8];
  load8<DT>(base, xv);
  load8<DT>(cos_tab + t * D + d, cv);
  load8<DT>(sin_tab + t * D + d, sv);
  rope_rotate8<DT>(xv, cv, sv, o);
  store8<DT>(base, o);
}

}  // namespace pfa

using namespace pfa;

// workspace of pfa_chunk_topk: pow2(min(budget, n)) keys, then the radix
// select's state (about 4n + 10 KB bytes)
static size_t chunk_keys_bytes(int64_t limit) { return ((size_t)pow2_ceil(limit > 0 ? limit : 1) * 8 + 255) / 256 * 256; }

extern "C" int pfa_chunk_topk_workspace_size(int64_t n, int budget, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && n >= 0 && budget >= 0, "pfa_chunk_topk_workspace_size: bad arguments");
  const int64_t limit = n < budget ? n : budget;
  *bytes = chunk_keys_bytes(limit) + rsel::segment_bytes(n);
  return PFA_OK;
}

extern "C" int pfa_chunk_topk(const float* scores, const uint8_t* keep_mask, int64_t n, int budget, float top_p,
                              int64_t index_offset, int drop_nonfinite, float* values_out, int64_t* indices_out,
                              int32_t* count_out, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n >= 0 && n < INT32_MAX && budget >= 0, "pfa_chunk_topk: bad sizes n=%lld budget=%d",
                (long long)n, budget);
  PFA_CHECK_ARG(count_out != nullptr, "pfa_chunk_topk: count_out is required");
  PFA_CHECK_ARG(top_p > 0.0f, "pfa_chunk_topk: top_p must be positive");
  hipStream_t s = as_stream(stream);
  const int64_t limit = n < budget ? n : budget;
  size_t need = 0;
  pfa_chunk_topk_workspace_size(n, budget, &need);
  PFA_CHECK_ARG(workspace && ws_bytes >= need, "pfa_chunk_topk: workspace of %zu bytes required", need);
  if (limit <= 0) {
    // nothing can be selected: count 0 (written by a one-lane emit)
    chunk_emit_kernel<<<1, kSelThreads, 0, s>>>(scores, keep_mask, n, nullptr, 0, 0, 0, top_p, nullptr, 0, 0, 0,
                                                 values_out, indices_out, count_out);
    PFA_CHECK_LAUNCH("pfa_chunk_topk");
    return PFA_OK;
  }
  PFA_CHECK_ARG(scores && values_out && indices_out, "pfa_chunk_topk: null pointer");
  const int64_t lp = pow2_ceil(limit);
  uint64_t* keys = (uint64_t*)workspace;
  unsigned char* sel_ws = (unsigned char*)workspace + chunk_keys_bytes(limit);
  const size_t seg = rsel::segment_bytes(n);
  const ChunkKeys src{scores, keep_mask};
  rsel::init_kernel<ChunkKeys><<<1, rsel::kThreads, 0, s>>>(sel_ws, seg, limit);
  PFA_CHECK_LAUNCH("pfa_chunk_topk/init");
  int rc = rsel::run_passes(src, n, 1, sel_ws, seg, s, "pfa_chunk_topk/select");
  if (rc != PFA_OK) return rc;
  chunk_keys_kernel<<<(unsigned)rsel::groups_of(n), rsel::kThreads, 0, s>>>(src, n, lp, sel_ws, keys);
  PFA_CHECK_LAUNCH("pfa_chunk_topk/keys");
  const int groups = (int)rsel::groups_of(n);
  const uint32_t* wstat = (const uint32_t*)(sel_ws + rsel::layout(groups).wstat);
  const bool sort_here = lp <= kSortTile;
  if (!sort_here) {
    rc = sort_u64(keys, lp, s, "pfa_chunk_topk/sort");
    if (rc != PFA_OK) return rc;
  }
  chunk_emit_kernel<<<1, kSelThreads, 0, s>>>(scores, keep_mask, n, keys, (int)limit, (int)lp, sort_here ? 1 : 0,
                                               top_p, wstat, groups, index_offset, drop_nonfinite ? 1 : 0, values_out,
                                               indices_out, count_out);
  PFA_CHECK_LAUNCH("pfa_chunk_topk/emit");
  return PFA_OK;
}

// workspace of pfa_shortlist_finalise: two key arrays of pow2(n) + n int32
extern "C" int pfa_shortlist_finalise_workspace_size(int64_t n, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && n >= 0, "pfa_shortlist_finalise_workspace_size: bad arguments");
  const size_t n2 = (size_t)pow2_ceil(n > 0 ? n : 1);
  *bytes = 2 * n2 * 8 + (size_t)(n > 0 ? n : 1) * 4;
  return PFA_OK;
}

extern "C" int pfa_shortlist_finalise(const float* scores, const int64_t* indices, int64_t n, int64_t max_tokens,
                                      int64_t* keep_indices_out, float* keep_scores_out, int32_t* count_out,
                                      void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n > 0 && n < INT32_MAX, "pfa_shortlist_finalise: candidate count must be in [1, 2^31) (got %lld)",
                (long long)n);
  PFA_CHECK_ARG(max_tokens >= 0, "pfa_shortlist_finalise: max_tokens must be >= 0");
  PFA_CHECK_ARG(scores && indices && keep_indices_out && keep_scores_out && count_out,
                "pfa_shortlist_finalise: null pointer");
  size_t need = 0;
  pfa_shortlist_finalise_workspace_size(n, &need);
  PFA_CHECK_ARG(workspace && ws_bytes >= need, "pfa_shortlist_finalise: workspace of %zu bytes required", need);
  hipStream_t s = as_stream(stream);
  const int64_t n2 = pow2_ceil(n);
  uint64_t* a = (uint64_t*)workspace;
  uint64_t* b = a + n2;
  int32_t* ord = (int32_t*)(b + n2);
  const unsigned g = (unsigned)((n2 + 255) / 256);
  fin_keys_score<<<g, 256, 0, s>>>(scores, n, n2, a);
  PFA_CHECK_LAUNCH("pfa_shortlist_finalise");
  int rc = sort_u64(a, n2, s, "pfa_shortlist_finalise/sort");
  if (rc != PFA_OK) return rc;
  fin_keys_index<<<g, 256, 0, s>>>(a, indices, n, n2, b);
  PFA_CHECK_LAUNCH("pfa_shortlist_finalise");
  rc = sort_u64(b, n2, s, "pfa_shortlist_finalise/sort");
  if (rc != PFA_OK) return rc;
  fin_emit_kernel<<<1, kSelThreads, 0, s>>>(scores, indices, n, max_tokens, a, b, ord, keep_indices_out,
                                             keep_scores_out, count_out);
  PFA_CHECK_LAUNCH("pfa_shortlist_finalise/emit");
  return PFA_OK;
}

extern "C" int pfa_quantize_rows_int8(const void* src, int dtype, int64_t n_rows, int64_t row_stride, int H, int D,
                                      int8_t* dst, float* scales, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n_rows >= 0 && H > 0 && D > 0 && row_stride >= (int64_t)H * D,
                "pfa_quantize_rows_int8: bad shape rows=%lld H=%d D=%d stride=%lld", (long long)n_rows, H, D,
                (long long)row_stride);
  if (n_rows == 0) return PFA_OK;
  PFA_CHECK_ARG(src && dst && scales, "pfa_quantize_rows_int8: null pointer");
  hipStream_t s = as_stream(stream);
  const int64_t waves = n_rows * H;
  const unsigned blocks = (unsigned)((waves * 64 + 255) / 256);
  switch (dtype) {
    case PFA_F32:
      quant_rows_kernel<PFA_F32><<<blocks, 256, 0, s>>>((const float*)src, n_rows, row_stride, H, D, dst, scales);
      break;
    case PFA_BF16:
      quant_rows_kernel<PFA_BF16><<<blocks, 256, 0, s>>>((const uint16_t*)src, n_rows, row_stride, H, D, dst,
                                                         scales);
      break;
    case PFA_F16:
      quant_rows_kernel<PFA_F16><<<blocks, 256, 0, s>>>((const uint16_t*)src, n_rows, row_stride, H, D, dst,
                                                        scales);
      break;
    default:
      set_error("pfa_quantize_rows_int8: unsupported dtype %d", dtype);
      return PFA_E_UNSUPPORTED;
  }
  PFA_CHECK_LAUNCH("pfa_quantize_rows_int8");
  return PFA_OK;
}

extern "C" int pfa_rope_rows_inplace(void* x, int dtype, int64_t n_rows, int64_t row_stride, int H, int D,
                                     const void* cos_tab, const void* sin_tab, const int32_t* positions,
                                     int64_t pos_offset, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n_rows >= 0 && H > 0 && D > 0 && D % 2 == 0 && row_stride >= (int64_t)H * D && pos_offset >= 0,
                "pfa_rope_rows_inplace: bad shape rows=%lld H=%d D=%d", (long long)n_rows, H, D);
  if (n_rows == 0) return PFA_OK;
  PFA_CHECK_ARG(x && cos_tab && sin_tab, "pfa_rope_rows_inplace: null pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = D % 8 == 0 && row_stride % 8 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)cos_tab % 16) == 0 &&
                   ((uintptr_t)sin_tab % 16) == 0 && (dtype == PFA_F32 || dtype == PFA_BF16 || dtype == PFA_F16);
  if (vec) {
    const int64_t work8 = n_rows * H * (D / 8);
    const unsigned blocks8 = (unsigned)((work8 + 255) / 256);
    if (dtype == PFA_F32)
      rope_rows8_kernel<PFA_F32><<<blocks8, 256, 0, s>>>((float*)x, n_rows, row_stride, H, D, (const float*)cos_tab,
                                                          (const float*)sin_tab, positions, pos_offset);
    else if (dtype == PFA_BF16)
      rope_rows8_kernel<PFA_BF16><<<blocks8, 256, 0, s>>>((uint16_t*)x, n_rows, row_stride, H, D,
                                                           (const uint16_t*)cos_tab, (const uint16_t*)sin_tab,
                                                           positions, pos_offset);
    else
      rope_rows8_kernel<PFA_F16><<<blocks8, 256, 0, s>>>((uint16_t*)x, n_rows, row_stride, H, D,
                                                          (const uint16_t*)cos_tab, (const uint16_t*)sin_tab,
                                                          positions, pos_offset);
    PFA_CHECK_LAUNCH("pfa_rope_rows_inplace");
    return PFA_OK;
  }
  const int64_t work = n_rows * H * (D / 2);
  const unsigned blocks = (unsigned)((work + 255) / 256);
  switch (dtype) {
    case PFA_F32:
      rope_rows_kernel<PFA_F32><<<blocks, 256, 0, s>>>((float*)x, n_rows, row_stride, H, D, (const float*)cos_tab,
                                                        (const float*)sin_tab, positions, pos_offset);
      break;
    case PFA_BF16:
      rope_rows_kernel<PFA_BF16><<<blocks, 256, 0, s>>>((uint16_t*)x, n_rows, row_stride, H, D,
                                                         (const uint16_t*)cos_tab, (const uint16_t*)sin_tab,
                                                         positions, pos_offset);
      break;
    case PFA_F16:
      rope_rows_kernel<PFA_F16><<<blocks, 256, 0, s>>>((uint16_t*)x, n_rows, row_stride, H, D,
                                                        (const uint16_t*)cos_tab, (const uint16_t*)sin_tab,
                                                        positions, pos_offset);
      break;
    default:
      set_error("pfa_rope_rows_inplace: unsupported dtype %d", dtype);
      return PFA_E_UNSUPPORTED;
  }
  PFA_CHECK_LAUNCH("pfa_rope_rows_inplace");
  return PFA_OK;
}
