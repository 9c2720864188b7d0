// Per-head symmetric int8 quantisation of the active heads' q, k or v
// (AdaptiveSparseAttention._quantize_per_head_int8, aspa.py:1312-1363), on
// the device and in place of the reference's tensor ops:
//   base  = max |x| over the head's (T, D) elements          ("max" mode)
//         = torch.quantile(|x|, p) with linear interpolation ("percentile")
//           (its absmax when the quantile is 0)
//   "ema_percentile": ema = decay*ema + (1-decay)*base, base = ema
//   scale = max(base / 127, 1e-6)
//   q     = clamp(round_half_even(x / scale), -127, 127)
// Every step is an f32 operation rounded as the reference's tensor op is
// (no contraction).
//
// Launch sequence of pfa_quantize_heads_int8 (grid (chunks, P_cap); compact
// heads p >= P = summary[0] return at once):
//   qh_chunk_max          per (head, chunk) absmax partial (every slot written)
//   [percentile] 3 x (qh_hist -> qh_pick): radix select of the k-th smallest
//       |x| bit pattern (non-negative floats order as their bits), 11/11/9
//       bits, the histogram cleared by the pick that consumed it; then
//       qh_min_above when the (k+1)-th value differs from the k-th
//   qh_finalize           per head: base, EMA, scale
//   qh_quantize           per (head, chunk): the int8 values
#include "pfa_common.h"

#include <algorithm>

namespace pfa {

constexpr int kQhThreads = 256;
constexpr int kQhBins = 2048;
constexpr int kQhStateWords = 8;  // per head: prefix, k_lo, need_hi, eq_lo, min_above, pad...

struct QhArgs {
  pfa_tensor4 x;
  int H;
  int64_t T;
  int D;
  const int32_t* head_map;
  int P_cap;
  const int32_t* summary;
  int64_t rows_per_chunk;
  int nchunk;
};

__device__ __forceinline__ int qh_active(const QhArgs& a, int p) {
  const int P = a.summary ? a.summary[0] : a.P_cap;
  return p < P;
}

template <int DT>
__device__ __forceinline__ const typename Elem<DT>::T* qh_head_base(const QhArgs& a, int bh) {
  const typename Elem<DT>::T* base = (const typename Elem<DT>::T*)a.x.ptr;
  return base + (int64_t)(bh / a.H) * a.x.s_b + (int64_t)(bh % a.H) * a.x.s_h;
}

// |x| bit patterns of this workgroup's chunk, visited by fn(u)
template <int DT, typename F>
__device__ __forceinline__ void qh_visit(const QhArgs& a, int p, F&& fn) {
  const int bh = a.head_map ? a.head_map[p] : p;
  const auto* hb = qh_head_base<DT>(a, bh);
  const int64_t t0 = (int64_t)blockIdx.x * a.rows_per_chunk;
  int64_t t1 = t0 + a.rows_per_chunk;
  if (t1 > a.T) t1 = a.T;
  if (t0 >= t1) return;
  const int64_t ne = (t1 - t0) * a.D;
  for (int64_t e = threadIdx.x; e < ne; e += kQhThreads) {
    const int64_t t = t0 + e / a.D;
    const int d = (int)(e % a.D);
    fn(__float_as_uint(fabsf(load_f<DT>(hb + t * a.x.s_t + d))));
  }
}

__device__ __forceinline__ uint32_t qh_block_max(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < kQhThreads / 64; ++w) v = max(v, red[w]);
  return v;
}

template <int DT>
__global__ void __launch_bounds__(kQhThreads) qh_chunk_max(QhArgs a, uint32_t* __restrict__ part) {
  __shared__ uint32_t red[kQhThreads / 64];
  const int p = blockIdx.y;
  if (!qh_active(a, p)) return;
  uint32_t m = 0;  // |x| bits: +0.0 is the smallest
  qh_visit<DT>(a, p, [&](uint32_t u) { m = max(m, u); });
  m = qh_block_max(m, red);
  if (threadIdx.x == 0) part[(int64_t)p * a.nchunk + blockIdx.x] = m;
}

// Histogram of bits [shift, shift + width) of the values whose bits above
// shift + width equal the head's prefix so far.
template <int DT>
__global__ void __launch_bounds__(kQhThreads) qh_hist(QhArgs a, int shift, int width, const uint32_t* __restrict__ state,
                                                      uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[kQhBins];
  const int p = blockIdx.y;
  if (!qh_active(a, p)) return;
  for (int i = threadIdx.x; i < kQhBins; i += kQhThreads) h[i] = 0;
  __syncthreads();
  const uint32_t prefix = state[p * kQhStateWords + 0];
  const int hs = shift + width;
  qh_visit<DT>(a, p, [&](uint32_t u) {
    const bool match = hs >= 32 || (u >> hs) == (prefix >> hs);
    if (match) atomicAdd(&h[(u >> shift) & ((1u << width) - 1u)], 1u);
  });
  __syncthreads();
  uint32_t* g = hist + (int64_t)p * kQhBins;
  for (int i = threadIdx.x; i < (1 << width); i += kQhThreads)
    if (h[i] != 0) atomicAdd(&g[i], h[i]);
}

// One workgroup per head: the bin that holds rank k (state[1]); the prefix
// gains that bin, k drops by the counts below it; the histogram is cleared
// for the next pass.  After the last pass, state[3] = values equal to the
// selected one that rank above k (its multiplicity beyond k).
__global__ void __launch_bounds__(kQhThreads) qh_pick(int P_cap, const int32_t* summary, int shift, int width, int last,
                                                      uint32_t* __restrict__ state, uint32_t* __restrict__ hist) {
  __shared__ uint32_t wsum[kQhThreads / 64];
  __shared__ uint32_t s_bin, s_below;
  const int p = blockIdx.x;
  if (p >= (summary ? summary[0] : P_cap)) return;
  if (threadIdx.x == 0) {
    s_bin = 0;
    s_below = 0;
  }
  uint32_t* g = hist + (int64_t)p * kQhBins;
  uint32_t* st = state + p * kQhStateWords;
  const uint32_t k = st[1];
  const int nb = 1 << width;
  const int per = (nb + kQhThreads - 1) / kQhThreads;  // contiguous bins per thread
  const int b0 = threadIdx.x * per;
  uint32_t mine = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < nb) mine += g[b0 + i];
  // exclusive scan of the per-thread sums
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t incl = mine;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t n = (uint32_t)__shfl_up((int)incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  uint32_t before = incl - mine;
  for (int w = 0; w < wid; ++w) before += wsum[w];
  if (before <= k && k < before + mine) {
    uint32_t run = before;
    for (int i = 0; i < per && b0 + i < nb; ++i) {
      const uint32_t c = g[b0 + i];
      if (k < run + c) {
        s_bin = (uint32_t)(b0 + i);
        s_below = run;
        if (last) st[3] = run + c - 1 - k;  // equal values ranked after k
        break;
      }
      run += c;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb; i += kQhThreads) g[i] = 0;
  if (threadIdx.x == 0) {
    st[0] |= s_bin << shift;
    st[1] = k - s_below;
  }
}

// The smallest |x| bit pattern above the selected value (heads whose
// (k+1)-th value is not a copy of the k-th); state[4] starts at UINT32_MAX.
template <int DT>
__global__ void __launch_bounds__(kQhThreads) qh_min_above(QhArgs a, uint32_t* __restrict__ state) {
  __shared__ uint32_t red[kQhThreads / 64];
  const int p = blockIdx.y;
  if (!qh_active(a, p)) return;
  uint32_t* st = state + p * kQhStateWords;
  if (st[2] == 0 || st[3] != 0) return;  // no second rank needed, or it equals the first
  const uint32_t v = st[0];
  uint32_t m = 0xffffffffu;
  qh_visit<DT>(a, p, [&](uint32_t u) {
    if (u > v) m = min(m, u);
  });
  for (int o = 32; o > 0; o >>= 1) m = min(m, (uint32_t)__shfl_xor((int)m, o, 64));
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kQhThreads / 64; ++w) m = min(m, red[w]);
    m = min(m, red[0]);
    atomicMin(&st[4], m);
  }
}

// Rank state before the first pass: prefix 0, k = k_lo, need_hi, eq 0,
// min_above = UINT32_MAX.
__global__ void qh_init_state(int P_cap, uint32_t k_lo, uint32_t need_hi, uint32_t* __restrict__ state,
                              uint32_t* __restrict__ hist) {
  const int p = blockIdx.x;
  for (int i = threadIdx.x; i < kQhBins; i += blockDim.x) hist[(int64_t)p * kQhBins + i] = 0;
  if (threadIdx.x == 0) {
    uint32_t* st = state + p * kQhStateWords;
    st[0] = 0;
    st[1] = k_lo;
    st[2] = need_hi;
    st[3] = 0;
    st[4] = 0xffffffffu;
  }
}

// Per head: absmax, base (max / interpolated quantile / its EMA), scale.
// mode 0 max, 1 percentile, 2 ema_percentile; use_q: the quantile state is
// there (percentile > 0).
__global__ void qh_finalize(int P_cap, const int32_t* summary, const int32_t* head_map, int nchunk,
                            const uint32_t* __restrict__ part, const uint32_t* __restrict__ state, int mode,
                            int use_q, float weight, float decay, float one_minus_decay, float* __restrict__ ema,
                            int ema_valid, float* __restrict__ scales) {
#pragma clang fp contract(off)
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= P_cap || p >= (summary ? summary[0] : P_cap)) return;
  uint32_t m = 0;
  for (int c = 0; c < nchunk; ++c) m = max(m, part[(int64_t)p * nchunk + c]);
  const float amax = __uint_as_float(m);
  float base = amax;
  if (mode != 0 && use_q) {
    const uint32_t* st = state + p * kQhStateWords;
    const float lo = __uint_as_float(st[0]);
    const float hi = (st[2] == 0 || st[3] != 0) ? lo : __uint_as_float(st[4]);
    // torch.lerp: weight < 0.5 ? lo + w (hi - lo) : hi - (hi - lo)(1 - w)
    // (plain operators: the pragma above keeps each product rounded; the
    // __f*_rn helpers are ordinary inline functions and would not be)
    const float q = weight < 0.5f ? lo + weight * (hi - lo) : hi - (hi - lo) * (1.0f - weight);
    base = q > 0.f ? q : amax;
  }
  if (mode == 2) {
    const float e = ema_valid ? ema[p] : amax;
    base = decay * e + one_minus_decay * base;
    ema[p] = base;
  }
  const int bh = head_map ? head_map[p] : p;
  scales[bh] = fmaxf(__fdiv_rn(base, 127.0f), 1e-6f);
}

// The int8 values, into dst (addressed like x, by the same global head) as
// int8 or as their exact bf16 values.
template <int DT, int OUT>
__global__ void __launch_bounds__(kQhThreads) qh_quantize(QhArgs a, const float* __restrict__ scales, pfa_tensor4 dst) {
  const int p = blockIdx.y;
  if (!qh_active(a, p)) return;
  const int bh = a.head_map ? a.head_map[p] : p;
  const float sc = scales[bh];
  const auto* hb = qh_head_base<DT>(a, bh);
  auto* ob = (typename Elem<OUT>::T*)dst.ptr + (int64_t)(bh / a.H) * dst.s_b + (int64_t)(bh % a.H) * dst.s_h;
  const int64_t t0 = (int64_t)blockIdx.x * a.rows_per_chunk;
  int64_t t1 = t0 + a.rows_per_chunk;
  if (t1 > a.T) t1 = a.T;
  if (t0 >= t1) return;
  const int64_t ne = (t1 - t0) * a.D;
  for (int64_t e = threadIdx.x; e < ne; e += kQhThreads) {
    const int64_t t = t0 + e / a.D;
    const int d = (int)(e % a.D);
    float q = rintf(__fdiv_rn(load_f<DT>(hb + t * a.x.s_t + d), sc));
    q = fminf(fmaxf(q, -127.f), 127.f);
    auto* o = ob + t * dst.s_t + d;
    if constexpr (OUT == PFA_I8) *o = (int8_t)(int)q;
    else store_f<OUT>(o, q);
  }
}

struct QhWs {
  uint32_t* part;
  uint32_t* state;
  uint32_t* hist;
};

static size_t qh_ws_bytes(int P_cap, int nchunk, int mode, QhWs* w, char* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return base ? (uint32_t*)(base + o) : nullptr;
  };
  uint32_t* part = take((size_t)P_cap * nchunk * 4);
  uint32_t* state = nullptr;
  uint32_t* hist = nullptr;
  if (mode != 0) {
    state = take((size_t)P_cap * kQhStateWords * 4);
    hist = take((size_t)P_cap * kQhBins * 4);
  }
  if (w) *w = QhWs{part, state, hist};
  return off;
}

static int qh_chunks(int64_t T, int D, int64_t* rows_per_chunk) {
  // about 16K elements per workgroup, at most 4096 chunks per head
  int64_t rpc = (16384 + D - 1) / D;
  if (rpc < 1) rpc = 1;
  int64_t n = (T + rpc - 1) / rpc;
  if (n > 4096) {
    rpc = (T + 4095) / 4096;
    n = (T + rpc - 1) / rpc;
  }
  *rows_per_chunk = rpc;
  return (int)(n > 0 ? n : 1);
}

template <int DT>
static int qh_run(const QhArgs& a, int mode, float percentile, double decay, float* ema, int ema_valid,
                  pfa_tensor4 dst, int dst_dtype, float* scales, const QhWs& w, hipStream_t s) {
  const dim3 grid((unsigned)a.nchunk, (unsigned)a.P_cap);
  qh_chunk_max<DT><<<grid, kQhThreads, 0, s>>>(a, w.part);
  PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/max");
  const bool use_q = mode != 0 && percentile > 0.f;
  float weight = 0.f;
  if (use_q) {
    // torch.quantile: rank = q * (n - 1) in f32, k_lo = trunc(rank), k_hi =
    // ceil(rank), weight = rank - k_lo
    const int64_t n = a.T * (int64_t)a.D;
    const float rank = percentile * (float)(n - 1);
    const int64_t k_lo = std::min((int64_t)rank, n - 1);
    const int64_t k_hi = std::min((int64_t)ceilf(rank), n - 1);
    weight = rank - (float)k_lo;
    qh_init_state<<<a.P_cap, 256, 0, s>>>(a.P_cap, (uint32_t)k_lo, k_hi != k_lo ? 1u : 0u, w.state, w.hist);
    PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/init");
    const int shifts[3] = {20, 9, 0}, widths[3] = {11, 11, 9};
    for (int pass = 0; pass < 3; ++pass) {
      qh_hist<DT><<<grid, kQhThreads, 0, s>>>(a, shifts[pass], widths[pass], w.state, w.hist);
      PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/hist");
      qh_pick<<<a.P_cap, kQhThreads, 0, s>>>(a.P_cap, a.summary, shifts[pass], widths[pass], pass == 2 ? 1 : 0,
                                             w.state, w.hist);
      PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/pick");
    }
    if (k_hi != k_lo) {
      qh_min_above<DT><<<grid, kQhThreads, 0, s>>>(a, w.state);
      PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/min_above");
    }
  }
  qh_finalize<<<(a.P_cap + 63) / 64, 64, 0, s>>>(a.P_cap, a.summary, a.head_map, a.nchunk, w.part, w.state, mode,
                                                 use_q ? 1 : 0, weight, (float)decay, (float)(1.0 - decay), ema,
                                                 ema_valid, scales);
  PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/finalize");
  if (dst_dtype == PFA_I8)
    qh_quantize<DT, PFA_I8><<<grid, kQhThreads, 0, s>>>(a, scales, dst);
  else
    qh_quantize<DT, PFA_BF16><<<grid, kQhThreads, 0, s>>>(a, scales, dst);
  PFA_CHECK_LAUNCH("pfa_quantize_heads_int8/quantize");
  return PFA_OK;
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_quantize_heads_workspace_size(int P_cap, int64_t T, int D, int mode, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && P_cap >= 0 && T >= 0 && D > 0 && mode >= 0 && mode <= 2,
                "pfa_quantize_heads_workspace_size: bad arguments");
  int64_t rpc;
  const int nchunk = qh_chunks(T, D, &rpc);
  *bytes = qh_ws_bytes(P_cap > 0 ? P_cap : 1, nchunk, mode, nullptr, nullptr);
  return PFA_OK;
}

extern "C" int pfa_quantize_heads_int8(pfa_tensor4 x, int dtype, int H, int64_t T, int D, const int32_t* head_map,
                                       int P_cap, const int32_t* summary, int mode, float percentile, double ema_decay,
                                       float* ema, int ema_valid, pfa_tensor4 dst, int dst_dtype, float* scales,
                                       void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(H > 0 && T >= 0 && D > 0 && P_cap >= 0, "pfa_quantize_heads_int8: bad sizes");
  PFA_CHECK_ARG(mode >= 0 && mode <= 2, "pfa_quantize_heads_int8: mode must be 0 (max), 1 (percentile) or 2 "
                                        "(ema_percentile), got %d", mode);
  PFA_CHECK_ARG(dst_dtype == PFA_I8 || dst_dtype == PFA_BF16, "pfa_quantize_heads_int8: dst dtype must be int8 or bf16");
  if (P_cap == 0 || T == 0) return PFA_OK;
  PFA_CHECK_ARG(x.ptr && dst.ptr && scales, "pfa_quantize_heads_int8: null pointer");
  PFA_CHECK_ARG(mode != 2 || ema, "pfa_quantize_heads_int8: ema_percentile needs the ema buffer");
  PFA_CHECK_ARG(T * (int64_t)D < (int64_t)INT32_MAX, "pfa_quantize_heads_int8: T*D must be below 2^31 per head");
  PFA_CHECK_ARG(!(percentile > 1.f) && !(percentile < 0.f), "pfa_quantize_heads_int8: percentile outside [0, 1]");
  QhArgs a;
  a.x = x; a.H = H; a.T = T; a.D = D; a.head_map = head_map; a.P_cap = P_cap; a.summary = summary;
  a.nchunk = qh_chunks(T, D, &a.rows_per_chunk);
  const size_t need = qh_ws_bytes(P_cap, a.nchunk, mode, nullptr, nullptr);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("pfa_quantize_heads_int8: workspace %zu < %zu", ws_bytes, need);
    return PFA_E_WORKSPACE;
  }
  QhWs w;
  qh_ws_bytes(P_cap, a.nchunk, mode, &w, (char*)workspace);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case PFA_F32: return qh_run<PFA_F32>(a, mode, percentile, ema_decay, ema, ema_valid, dst, dst_dtype, scales, w, s);
    case PFA_BF16:
      return qh_run<PFA_BF16>(a, mode, percentile, ema_decay, ema, ema_valid, dst, dst_dtype, scales, w, s);
    case PFA_F16: return qh_run<PFA_F16>(a, mode, percentile, ema_decay, ema, ema_valid, dst, dst_dtype, scales, w, s);
    default:
      set_error("pfa_quantize_heads_int8: unsupported dtype %d", dtype);
      return PFA_E_UNSUPPORTED;
  }
}
