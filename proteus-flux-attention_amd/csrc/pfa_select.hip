// Token top-k (radix select) and row packing.
#include "pfa_common.h"
#include "pfa_radix.h"

#include <mutex>

namespace pfa {

// ---------------------------------------------------------------------
// Token top-k.  Per batch row, the `need` largest values are found by the
// multi-workgroup radix select of pfa_radix.h on order-preserving 32-bit
// keys; of the values equal to the cut value, the lowest indices are taken.
// Replaces the per-batch torch.topk loop of aspa.py:823-840.
// ---------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int block_sum_int(int v, int* red) {
  // wave64 reduce then across waves (<= 16 waves)
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  int nw = (blockDim.x + 63) >> 6;
  int s = 0;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}

struct ImportanceKeys {
  const float* imp;
  int64_t T;
  __device__ __forceinline__ uint32_t key(int b, int64_t i) const { return order_key(imp[(int64_t)b * T + i]); }
};

// need = max(keep_count, #(imp >= threshold), guard) clamped to [1, T], when
// the threshold makes it data dependent.  grid = (groups, B); the last
// workgroup of a row finalises the row's state.
__global__ void __launch_bounds__(rsel::kThreads) topk_need_kernel(const float* __restrict__ imp, int64_t T,
                                                                   float threshold, int64_t keep_count, int guard,
                                                                   unsigned char* ws, size_t seg_bytes) {
  __shared__ int red[rsel::kThreads / 64];
  __shared__ int s_last;
  const int b = blockIdx.y;
  rsel::State* st = reinterpret_cast<rsel::State*>(ws + (size_t)b * seg_bytes);
  const int64_t i0 = (int64_t)blockIdx.x * rsel::kSpan + (int64_t)threadIdx.x * rsel::kPer;
  int c = 0;
#pragma unroll
  for (int e = 0; e < rsel::kPer; ++e)
    if (i0 + e < T) c += imp[(int64_t)b * T + i0 + e] >= threshold ? 1 : 0;
  c = block_sum_int(c, red);
  if (threadIdx.x == 0 && c != 0)
    __hip_atomic_fetch_add(&st->count, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!rsel::arrive(&st->done, gridDim.x, &s_last) || threadIdx.x != 0) return;
  const int64_t cnt = (int64_t)__hip_atomic_load(&st->count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int64_t need = keep_count;
  if (cnt > need) need = cnt;
  if (guard > need) need = guard;
  if (need < 1) need = 1;
  if (need > T) need = T;
  st->need = (int32_t)need;
  st->remaining = (int32_t)need;
  st->done = 0u;
}

// The mask: keys above the cut, the first `remaining` keys equal to it (by
// index), and the first `guard` tokens.  grid = (groups, B).
__global__ void __launch_bounds__(rsel::kThreads) topk_mask_kernel(ImportanceKeys src, int guard,
                                                                   const unsigned char* ws, size_t seg_bytes,
                                                                   uint8_t* __restrict__ mask) {
  __shared__ uint32_t sm[rsel::kThreads / 64];
  const int b = blockIdx.y, w = blockIdx.x;
  const int64_t T = src.T;
  const unsigned char* base = ws + (size_t)b * seg_bytes;
  const rsel::State* st = reinterpret_cast<const rsel::State*>(base);
  const int32_t* tiebase = reinterpret_cast<const int32_t*>(base + rsel::layout(gridDim.x).tiebase);
  uint8_t* mrow = mask + (int64_t)b * T;
  const int64_t i0 = (int64_t)w * rsel::kSpan + (int64_t)threadIdx.x * rsel::kPer;
  const int need = st->need;
  if ((int64_t)need >= T) {
#pragma unroll
    for (int e = 0; e < rsel::kPer; ++e)
      if (i0 + e < T) mrow[i0 + e] = 1;
    return;
  }
  uint32_t kv[rsel::kPer];
#pragma unroll
  for (int e = 0; e < rsel::kPer; ++e) kv[e] = i0 + e < T ? src.key(b, i0 + e) : 0u;
  bool sel[rsel::kPer], above[rsel::kPer];
  uint32_t rank[rsel::kPer];
  rsel::select_keys(kv, i0, T, st->prefix, st->remaining, tiebase[w], sm, sel, above, rank);
#pragma unroll
  for (int e = 0; e < rsel::kPer; ++e)
    if (i0 + e < T) mrow[i0 + e] = (sel[e] || i0 + e < guard) ? 1 : 0;
}

// ---------------------------------------------------------------------
// Row packing.  Tiles of kPackTile tokens of one (batch*head) row.
// ---------------------------------------------------------------------
constexpr int kPackThreads = 256;
constexpr int kPackTile = 1024;  // 4 tokens per thread

__global__ void __launch_bounds__(kPackThreads)
pack_count_routed(const int32_t* __restrict__ head_idx, int topk, const uint8_t* __restrict__ token_mask, int H,
                  int64_t T, int nblk, uint8_t* __restrict__ mask_out, int32_t* __restrict__ blockcounts,
                  int32_t* __restrict__ row_of) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  __shared__ int red[16];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  int cnt = 0;
  for (int j = 0; j < kPackTile / kPackThreads; ++j) {
    int64_t t = (int64_t)blk * kPackTile + j * kPackThreads + threadIdx.x;
    if (t < T) {
      int64_t bt = (int64_t)b * T + t;
      bool act = token_mask == nullptr || token_mask[bt] != 0;
      bool sel = false;
      for (int kk = 0; kk < topk; ++kk) sel |= head_idx[bt * topk + kk] == h;
      act = act && sel;
      mask_out[(int64_t)bh * T + t] = act ? 1 : 0;
      if (row_of != nullptr) row_of[(int64_t)bh * T + t] = -1;
      cnt += act ? 1 : 0;
    }
  }
  int s = block_sum_int(cnt, red);
  if (threadIdx.x == 0) blockcounts[(int64_t)bh * nblk + blk] = s;
}

// Token-parallel form for H <= kPackHeads: one workgroup per (tile, batch)
// reads each token's head list once and writes the mask, row_of = -1 and the
// tile counts of all H head rows (the per-row form above re-reads the head
// lists once per head row).  The counts are integer sums: the same in any
// order.
constexpr int kPackHeads = 16;
__global__ void __launch_bounds__(kPackThreads)
pack_count_routed_tok(const int32_t* __restrict__ head_idx, int topk, const uint8_t* __restrict__ token_mask, int H,
                      int64_t T, int nblk, uint8_t* __restrict__ mask_out, int32_t* __restrict__ blockcounts,
                      int32_t* __restrict__ row_of) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  __shared__ int cnt_s[kPackHeads];
  const int blk = blockIdx.x, b = blockIdx.y;
  if (threadIdx.x < kPackHeads) cnt_s[threadIdx.x] = 0;
  __syncthreads();
  int cnt[kPackHeads];
#pragma unroll
  for (int h = 0; h < kPackHeads; ++h) cnt[h] = 0;
  for (int j = 0; j < kPackTile / kPackThreads; ++j) {
    const int64_t t = (int64_t)blk * kPackTile + j * kPackThreads + threadIdx.x;
    if (t < T) {
      const int64_t bt = (int64_t)b * T + t;
      uint32_t sel = 0;
      if (token_mask == nullptr || token_mask[bt] != 0)
        for (int kk = 0; kk < topk; ++kk) {
          const int hv = head_idx[bt * topk + kk];
          if ((unsigned)hv < (unsigned)H) sel |= 1u << hv;  // other values select no row, as above
        }
#pragma unroll
      for (int h = 0; h < kPackHeads; ++h) {
        if (h < H) {
          const int a = (sel >> h) & 1u;
          const int64_t o = ((int64_t)b * H + h) * T + t;
          mask_out[o] = (uint8_t)a;
          if (row_of != nullptr) row_of[o] = -1;
          cnt[h] += a;
        }
      }
    }
  }
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int h = 0; h < kPackHeads; ++h) {
    if (h < H) {
      int v = cnt[h];
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) atomicAdd(&cnt_s[h], v);
    }
  }
  __syncthreads();
  if (threadIdx.x < H && threadIdx.x < kPackHeads)
    blockcounts[((int64_t)b * H + threadIdx.x) * nblk + blk] = cnt_s[threadIdx.x];
}

__global__ void __launch_bounds__(kPackThreads)
pack_count_mask(const uint8_t* __restrict__ mask, int64_t T, int nblk, int32_t* __restrict__ blockcounts) {
  __shared__ int red[16];
  const int blk = blockIdx.x, bh = blockIdx.y;
  int cnt = 0;
  for (int j = 0; j < kPackTile / kPackThreads; ++j) {
    int64_t t = (int64_t)blk * kPackTile + j * kPackThreads + threadIdx.x;
    if (t < T) cnt += mask[(int64_t)bh * T + t] ? 1 : 0;
  }
  int s = block_sum_int(cnt, red);
  if (threadIdx.x == 0) blockcounts[(int64_t)bh * nblk + blk] = s;
}

// Single workgroup: per-row totals, optional compaction of empty rows,
// row_offsets, and per-(row, tile) base offsets written over blockcounts.
// Launched with kScanThreads (four waves): a 16-wave workgroup has to wait
// for a nearly empty CU while the concurrent GEMM fills them.
constexpr int kScanThreads = 256;
__global__ void __launch_bounds__(1024)
pack_scan_kernel(int32_t* __restrict__ blockcounts, int BH, int nblk, int compact, int32_t* __restrict__ totals,
                 int32_t* __restrict__ compact_id, int32_t* __restrict__ active_heads,
                 int32_t* __restrict__ row_offsets, int32_t* __restrict__ summary) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  __shared__ int wave_tot[16];
  __shared__ int s_carry_p, s_carry_n, s_max;
  if (threadIdx.x == 0) { s_carry_p = 0; s_carry_n = 0; s_max = 0; }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // per-row totals: one wave per row, 64 tile counts per step
  for (int bh = wid; bh < BH; bh += nw) {
    int tot = 0;
    for (int j0 = 0; j0 < nblk; j0 += 64) {
      const int j = j0 + lane;
      int c = j < nblk ? blockcounts[(int64_t)bh * nblk + j] : 0;
      for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
      tot += c;
    }
    if (lane == 0) totals[bh] = tot;
  }
  __syncthreads();
  for (int base = 0; base < BH; base += blockDim.x) {
    int bh = base + threadIdx.x;
    int tot = (bh < BH) ? totals[bh] : 0;
    int act = (bh < BH) && (!compact || tot > 0);
    // scan (act, tot) jointly: two scans
    int va = act, vn = act ? tot : 0;
    for (int off = 1; off < 64; off <<= 1) {
      int na = __shfl_up(va, off, 64), nn = __shfl_up(vn, off, 64);
      if (lane >= off) { va += na; vn += nn; }
    }
    __shared__ int wave_n[16];
    if (lane == 63) { wave_tot[wid] = va; wave_n[wid] = vn; }
    __syncthreads();
    int ba = 0, bn = 0, ta = 0, tn = 0;
    for (int w = 0; w < nw; ++w) {
      if (w < wid) { ba += wave_tot[w]; bn += wave_n[w]; }
      ta += wave_tot[w];
      tn += wave_n[w];
    }
    int cp = s_carry_p, cn = s_carry_n;
    if (bh < BH) {
      if (act) {
        int id = cp + ba + va - 1;
        int off = cn + bn + vn - tot;
        compact_id[bh] = id;
        if (active_heads) active_heads[id] = bh;
        row_offsets[id] = off;
        atomicMax(&s_max, tot);
      } else {
        compact_id[bh] = -1;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) { s_carry_p = cp + ta; s_carry_n = cn + tn; }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    row_offsets[s_carry_p] = s_carry_n;
    summary[0] = s_carry_p;
    summary[1] = s_carry_n;
    summary[2] = s_max;
    summary[3] = 0;
  }
  __syncthreads();
  // per-tile bases: one wave per row, an exclusive scan of 64 tile counts
  // per step
  for (int bh = wid; bh < BH; bh += nw) {
    const int id = compact_id[bh];
    if (id < 0) continue;
    int run = row_offsets[id];
    for (int j0 = 0; j0 < nblk; j0 += 64) {
      const int j = j0 + lane;
      const int c = j < nblk ? blockcounts[(int64_t)bh * nblk + j] : 0;
      int v = c;
      for (int off = 1; off < 64; off <<= 1) {
        const int n = __shfl_up(v, off, 64);
        if (lane >= off) v += n;
      }
      if (j < nblk) blockcounts[(int64_t)bh * nblk + j] = run + v - c;
      run += __shfl(v, 63, 64);
    }
  }
}

__global__ void __launch_bounds__(kPackThreads)
pack_fill_kernel(const uint8_t* __restrict__ mask, int64_t T, int nblk, const int32_t* __restrict__ bases,
                 const int32_t* __restrict__ compact_id, int32_t* __restrict__ token_idx,
                 int32_t* __restrict__ row_head, int32_t* __restrict__ row_of) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  __shared__ int wave_tot[4];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int id = compact_id[bh];
  if (id < 0) return;
  int run = bases[(int64_t)bh * nblk + blk];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int j = 0; j < kPackTile / kPackThreads; ++j) {
    int64_t t = (int64_t)blk * kPackTile + j * kPackThreads + threadIdx.x;
    int act = (t < T && mask[(int64_t)bh * T + t]) ? 1 : 0;
    int v = act;
    for (int off = 1; off < 64; off <<= 1) {
      int n = __shfl_up(v, off, 64);
      if (lane >= off) v += n;
    }
    if (lane == 63) wave_tot[wid] = v;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < kPackThreads / 64; ++w) {
      if (w < wid) before += wave_tot[w];
      total += wave_tot[w];
    }
    if (act) {
      int pos = run + before + v - 1;
      token_idx[pos] = (int32_t)t;
      row_head[pos] = id;
      if (row_of != nullptr) row_of[(int64_t)bh * T + t] = pos;
    }
    run += total;
    __syncthreads();
  }
}

// Fill with the scan folded in, for BH * nblk <= kFusedScanMax: every
// workgroup reads the whole (BH, nblk) count table (a few KB, from L2) and
// derives its own base -- the totals of the heads before its head, the
// compaction of empty heads, the counts of its head's earlier blocks -- so
// no single-workgroup scan launch sits between the count and the fill.
// Workgroup (0, 0) also writes the per-head outputs (active heads, row
// offsets, summary) as pack_scan_kernel does.
constexpr int kFusedScanMax = 4096;

// Workgroup sums of a and b (every thread gets both).
__device__ __forceinline__ void block_sum2(int& a, int& b, int* red) {
  for (int off = 32; off > 0; off >>= 1) {
    a += __shfl_xor(a, off, 64);
    b += __shfl_xor(b, off, 64);
  }
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) {
    red[2 * wid] = a;
    red[2 * wid + 1] = b;
  }
  __syncthreads();
  a = 0;
  b = 0;
  for (int w = 0; w < nw; ++w) {
    a += red[2 * w];
    b += red[2 * w + 1];
  }
}

__global__ void __launch_bounds__(kPackThreads)
pack_fill_scan_kernel(const uint8_t* __restrict__ mask, int BH, int64_t T, int nblk,
                      const int32_t* __restrict__ blockcounts, int compact, int32_t* __restrict__ active_heads,
                      int32_t* __restrict__ row_offsets, int32_t* __restrict__ summary,
                      int32_t* __restrict__ token_idx, int32_t* __restrict__ row_head, int32_t* __restrict__ row_of) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  extern __shared__ int s_tot[];  // per-head totals (BH)
  __shared__ int red[2 * (kPackThreads / 64)];
  __shared__ int wave_tot[kPackThreads / 64];
  const int blk = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  for (int h = tid; h < BH; h += kPackThreads) s_tot[h] = 0;
  __syncthreads();
  // totals per head (LDS atomics: integer sums, any order) and this head's
  // counts of the blocks before this one
  int before_blk = 0;
  const int n = BH * nblk;
  for (int i = tid; i < n; i += kPackThreads) {
    const int c = blockcounts[i];
    const int h = i / nblk;
    if (c != 0) atomicAdd(&s_tot[h], c);
    if (h == bh && i - h * nblk < blk) before_blk += c;
  }
  __syncthreads();
  // rows of the heads before this one, and how many of them are active
  int rows_before = 0, heads_before = 0;
  for (int h = tid; h < bh; h += kPackThreads) {
    const int t = s_tot[h];
    rows_before += t;
    heads_before += (!compact || t > 0) ? 1 : 0;
  }
  block_sum2(rows_before, heads_before, red);
  int unused = 0;
  block_sum2(before_blk, unused, red);
  if (blk == 0 && bh == 0) {
    // per-head outputs: a scan over the BH totals, kPackThreads heads a step
    int carry_p = 0, carry_n = 0, mx = 0;
    for (int base = 0; base < BH; base += kPackThreads) {
      const int h = base + tid;
      const int tot = h < BH ? s_tot[h] : 0;
      const int act = (h < BH) && (!compact || tot > 0);
      int va = act, vn = act ? tot : 0;
      for (int off = 1; off < 64; off <<= 1) {
        const int na = __shfl_up(va, off, 64), nn = __shfl_up(vn, off, 64);
        if (lane >= off) {
          va += na;
          vn += nn;
        }
      }
      __syncthreads();
      if (lane == 63) {
        red[2 * wid] = va;
        red[2 * wid + 1] = vn;
      }
      __syncthreads();
      int ba = 0, bn = 0, ta = 0, tn = 0;
      for (int w = 0; w < kPackThreads / 64; ++w) {
        if (w < wid) {
          ba += red[2 * w];
          bn += red[2 * w + 1];
        }
        ta += red[2 * w];
        tn += red[2 * w + 1];
      }
      if (act) {
        const int id = carry_p + ba + va - 1;
        if (active_heads) active_heads[id] = h;
        row_offsets[id] = carry_n + bn + vn - tot;
        mx = max(mx, tot);
      }
      carry_p += ta;
      carry_n += tn;
    }
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
    __syncthreads();
    if (lane == 0) red[wid] = mx;
    __syncthreads();
    if (tid == 0) {
      for (int w = 0; w < kPackThreads / 64; ++w) mx = max(mx, red[w]);
      row_offsets[carry_p] = carry_n;
      summary[0] = carry_p;
      summary[1] = carry_n;
      summary[2] = mx;
      summary[3] = 0;
    }
  }
  if (compact && s_tot[bh] == 0) return;
  const int id = heads_before;
  int run = rows_before + before_blk;
  for (int j = 0; j < kPackTile / kPackThreads; ++j) {
    const int64_t t = (int64_t)blk * kPackTile + j * kPackThreads + tid;
    const int act = (t < T && mask[(int64_t)bh * T + t]) ? 1 : 0;
    int v = act;
    for (int off = 1; off < 64; off <<= 1) {
      const int nn = __shfl_up(v, off, 64);
      if (lane >= off) v += nn;
    }
    if (lane == 63) wave_tot[wid] = v;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < kPackThreads / 64; ++w) {
      if (w < wid) before += wave_tot[w];
      total += wave_tot[w];
    }
    if (act) {
      const int pos = run + before + v - 1;
      token_idx[pos] = (int32_t)t;
      row_head[pos] = id;
      if (row_of != nullptr) row_of[(int64_t)bh * T + t] = pos;
    }
    run += total;
    __syncthreads();
  }
}

__global__ void head_max_token_kernel(const int32_t* __restrict__ token_idx, const int32_t* __restrict__ row_offsets,
                                      int P, int32_t* __restrict__ out) {
  __shared__ int red;
  const int p = blockIdx.x;
  if (threadIdx.x == 0) red = -1;
  __syncthreads();
  int m = -1;
  for (int r = row_offsets[p] + threadIdx.x; r < row_offsets[p + 1]; r += blockDim.x) m = max(m, token_idx[r]);
  atomicMax(&red, m);
  __syncthreads();
  if (threadIdx.x == 0) out[p] = red;
}

struct PackWs {
  int32_t* blockcounts;
  int32_t* totals;
  int32_t* compact_id;
};

static size_t pack_ws_bytes(int64_t BH, int64_t T, int* nblk_out) {
  int64_t nblk = (T + kPackTile - 1) / kPackTile;
  if (nblk < 1) nblk = 1;
  if (nblk_out) *nblk_out = (int)nblk;
  size_t a = (size_t)BH * nblk * 4;
  a = (a + 255) & ~(size_t)255;
  size_t b = ((size_t)BH * 4 + 255) & ~(size_t)255;
  return a + 2 * b;
}

static PackWs carve(void* ws, int64_t BH, int nblk) {
  PackWs w;
  size_t a = (size_t)BH * nblk * 4;
  a = (a + 255) & ~(size_t)255;
  size_t b = ((size_t)BH * 4 + 255) & ~(size_t)255;
  w.blockcounts = (int32_t*)ws;
  w.totals = (int32_t*)((char*)ws + a);
  w.compact_id = (int32_t*)((char*)ws + a + b);
  return w;
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_token_topk_workspace_size(int B, int64_t T, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && B >= 0 && T >= 0, "pfa_token_topk_workspace_size: bad arguments");
  *bytes = (size_t)(B > 0 ? B : 1) * rsel::segment_bytes(T);
  return PFA_OK;
}

extern "C" int pfa_token_topk(const float* importance, int B, int64_t T, int64_t keep_count, int guard,
                              float threshold, uint8_t* mask_out, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(B >= 0 && T >= 0 && T < INT32_MAX, "pfa_token_topk: bad sizes B=%d T=%lld", B, (long long)T);
  if (B == 0 || T == 0) return PFA_OK;
  PFA_CHECK_ARG(importance && mask_out, "pfa_token_topk: null pointer");
  size_t need_ws = 0;
  pfa_token_topk_workspace_size(B, T, &need_ws);
  PFA_CHECK_ARG(workspace && ws_bytes >= need_ws, "pfa_token_topk: workspace of %zu bytes required", need_ws);
  hipStream_t s = as_stream(stream);
  unsigned char* ws = (unsigned char*)workspace;
  const size_t seg = rsel::segment_bytes(T);
  const int g = guard < 0 ? 0 : guard;
  const bool thr = threshold > 0.f;
  int64_t need = keep_count;
  if (!thr) {
    if (g > need) need = g;
    if (need < 1) need = 1;
    if (need > T) need = T;
  }
  rsel::init_kernel<ImportanceKeys><<<(unsigned)B, rsel::kThreads, 0, s>>>(ws, seg, need);
  PFA_CHECK_LAUNCH("pfa_token_topk/init");
  const dim3 grid((unsigned)rsel::groups_of(T), (unsigned)B);
  if (thr) {
    topk_need_kernel<<<grid, rsel::kThreads, 0, s>>>(importance, T, threshold, keep_count, g, ws, seg);
    PFA_CHECK_LAUNCH("pfa_token_topk/need");
  }
  const ImportanceKeys src{importance, T};
  int rc = rsel::run_passes(src, T, B, ws, seg, s, "pfa_token_topk/select");
  if (rc != PFA_OK) return rc;
  topk_mask_kernel<<<grid, rsel::kThreads, 0, s>>>(src, g, ws, seg, mask_out);
  PFA_CHECK_LAUNCH("pfa_token_topk/mask");
  return PFA_OK;
}

extern "C" int pfa_pack_workspace_size(int B, int H, int64_t T, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && B >= 0 && H > 0 && T >= 0, "pfa_pack_workspace_size: bad arguments");
  *bytes = pack_ws_bytes((int64_t)B * H, T, nullptr);
  return PFA_OK;
}

namespace pfa {

// The three launches of pfa_pack_rows over a carved workspace.
static int pack_rows_launch(const int32_t* head_idx, int topk, const uint8_t* token_mask, int B, int H, int64_t T,
                            int nblk, uint8_t* mask_out, int32_t* active_heads_out, int32_t* row_offsets_out,
                            int32_t* token_idx_out, int32_t* row_head_out, int32_t* row_of_out,
                            int32_t* summary_out, PackWs w, hipStream_t s) {
  const int64_t BH = (int64_t)B * H;
  dim3 grid(nblk, (unsigned)BH);
  if (H <= kPackHeads)
    pack_count_routed_tok<<<dim3(nblk, (unsigned)B), kPackThreads, 0, s>>>(head_idx, topk, token_mask, H, T, nblk,
                                                                          mask_out, w.blockcounts, row_of_out);
  else
    pack_count_routed<<<grid, kPackThreads, 0, s>>>(head_idx, topk, token_mask, H, T, nblk, mask_out, w.blockcounts,
                                                    row_of_out);
  PFA_CHECK_LAUNCH("pfa_pack_rows/count");
  if (BH * nblk <= kFusedScanMax) {
    pack_fill_scan_kernel<<<grid, kPackThreads, (size_t)BH * sizeof(int), s>>>(
        mask_out, (int)BH, T, nblk, w.blockcounts, 1, active_heads_out, row_offsets_out, summary_out, token_idx_out,
        row_head_out, row_of_out);
    PFA_CHECK_LAUNCH("pfa_pack_rows/fill");
    return PFA_OK;
  }
  pack_scan_kernel<<<1, kScanThreads, 0, s>>>(w.blockcounts, (int)BH, nblk, 1, w.totals, w.compact_id, active_heads_out,
                                      row_offsets_out, summary_out);
  PFA_CHECK_LAUNCH("pfa_pack_rows/scan");
  pack_fill_kernel<<<grid, kPackThreads, 0, s>>>(mask_out, T, nblk, w.blockcounts, w.compact_id, token_idx_out,
                                                 row_head_out, row_of_out);
  PFA_CHECK_LAUNCH("pfa_pack_rows/fill");
  return PFA_OK;
}

// Scratch of pfa_pack_rows_static: per-(head, block) counts, per-head totals
// and compact ids (the pfa_pack_rows workspace layout), at most
// kPackStaticBytes.  Every entry is written before it is read, so nothing is
// cleared between calls.
constexpr size_t kPackStaticBytes = PFA_PACK_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kPackStaticBytes];

// Device address of `scratch` per device, looked up once per device with
// that device current (host code never passes the symbol itself).
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("pfa_pack_rows_static: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("pfa_pack_rows_static: device %d beyond the %d supported", dev, kMaxDevices);
    return PFA_E_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("pfa_pack_rows_static: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return e != hipSuccess ? (int)e : PFA_E_UNSUPPORTED;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PFA_OK;
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_pack_rows(const int32_t* head_idx, int topk, const uint8_t* token_mask, int B, int H, int64_t T,
                             uint8_t* mask_out, int32_t* active_heads_out, int32_t* row_offsets_out,
                             int32_t* token_idx_out, int32_t* row_head_out, int32_t* row_of_out,
                             int32_t* summary_out, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(head_idx && mask_out && row_offsets_out && token_idx_out && row_head_out && summary_out && workspace,
                "pfa_pack_rows: null pointer");
  PFA_CHECK_ARG(B > 0 && H > 0 && T > 0 && topk >= 1 && topk <= H, "pfa_pack_rows: bad sizes");
  PFA_CHECK_ARG((int64_t)B * H * T < (int64_t)INT32_MAX, "pfa_pack_rows: B*H*T exceeds int32 row indexing");
  int nblk;
  int64_t BH = (int64_t)B * H;
  size_t need = pack_ws_bytes(BH, T, &nblk);
  if (ws_bytes < need) {
    set_error("pfa_pack_rows: workspace %zu < %zu", ws_bytes, need);
    return PFA_E_WORKSPACE;
  }
  return pack_rows_launch(head_idx, topk, token_mask, B, H, T, nblk, mask_out, active_heads_out, row_offsets_out,
                          token_idx_out, row_head_out, row_of_out, summary_out, carve(workspace, BH, nblk),
                          as_stream(stream));
}

extern "C" int pfa_pack_rows_static(const int32_t* head_idx, int topk, const uint8_t* token_mask, int B, int H,
                                    int64_t T, uint8_t* mask_out, int32_t* active_heads_out,
                                    int32_t* row_offsets_out, int32_t* token_idx_out, int32_t* row_head_out,
                                    int32_t* row_of_out, int32_t* summary_out, void* stream) {
  clear_error();
  PFA_CHECK_ARG(head_idx && mask_out && row_offsets_out && token_idx_out && row_head_out && summary_out,
                "pfa_pack_rows_static: null pointer");
  PFA_CHECK_ARG(B > 0 && H > 0 && T > 0 && topk >= 1 && topk <= H, "pfa_pack_rows_static: bad sizes");
  PFA_CHECK_ARG((int64_t)B * H * T < (int64_t)INT32_MAX, "pfa_pack_rows_static: B*H*T exceeds int32 row indexing");
  int nblk;
  const int64_t BH = (int64_t)B * H;
  const size_t need = pack_ws_bytes(BH, T, &nblk);
  PFA_CHECK_ARG(need <= kPackStaticBytes,
                "pfa_pack_rows_static: B*H=%lld heads x %d token blocks need %zu bytes of scratch, above the "
                "static maximum of %zu (use pfa_pack_rows with a workspace)",
                (long long)BH, nblk, need, kPackStaticBytes);
  void* ptr = nullptr;
  const int rc = scratch_address(&ptr);
  if (rc != PFA_OK) return rc;
  return pack_rows_launch(head_idx, topk, token_mask, B, H, T, nblk, mask_out, active_heads_out, row_offsets_out,
                          token_idx_out, row_head_out, row_of_out, summary_out, carve(ptr, BH, nblk),
                          as_stream(stream));
}

extern "C" int pfa_pack_mask(const uint8_t* mask, int P, int64_t T, int32_t* row_offsets_out, int32_t* token_idx_out,
                             int32_t* row_head_out, int32_t* summary_out, void* workspace, size_t ws_bytes,
                             void* stream) {
  clear_error();
  PFA_CHECK_ARG(mask && row_offsets_out && token_idx_out && row_head_out && summary_out && workspace,
                "pfa_pack_mask: null pointer");
  PFA_CHECK_ARG(P > 0 && T > 0, "pfa_pack_mask: bad sizes");
  PFA_CHECK_ARG((int64_t)P * T < (int64_t)INT32_MAX, "pfa_pack_mask: P*T exceeds int32 row indexing");
  int nblk;
  size_t need = pack_ws_bytes(P, T, &nblk);
  if (ws_bytes < need) {
    set_error("pfa_pack_mask: workspace %zu < %zu", ws_bytes, need);
    return PFA_E_WORKSPACE;
  }
  PackWs w = carve(workspace, P, nblk);
  hipStream_t s = as_stream(stream);
  dim3 grid(nblk, (unsigned)P);
  pack_count_mask<<<grid, kPackThreads, 0, s>>>(mask, T, nblk, w.blockcounts);
  PFA_CHECK_LAUNCH("pfa_pack_mask/count");
  pack_scan_kernel<<<1, kScanThreads, 0, s>>>(w.blockcounts, P, nblk, 0, w.totals, w.compact_id, nullptr, row_offsets_out,
                                      summary_out);
  PFA_CHECK_LAUNCH("pfa_pack_mask/scan");
  pack_fill_kernel<<<grid, kPackThreads, 0, s>>>(mask, T, nblk, w.blockcounts, w.compact_id, token_idx_out,
                                                 row_head_out, nullptr);
  PFA_CHECK_LAUNCH("pfa_pack_mask/fill");
  return PFA_OK;
}

extern "C" int pfa_head_max_token(const int32_t* token_idx, const int32_t* row_offsets, int P, int32_t* out,
                                  void* stream) {
  clear_error();
  PFA_CHECK_ARG(token_idx && row_offsets && out && P >= 0, "pfa_head_max_token: bad arguments");
  if (P == 0) return PFA_OK;
  head_max_token_kernel<<<P, 256, 0, as_stream(stream)>>>(token_idx, row_offsets, P, out);
  PFA_CHECK_LAUNCH("pfa_head_max_token");
  return PFA_OK;
}
