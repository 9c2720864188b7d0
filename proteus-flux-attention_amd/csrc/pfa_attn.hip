// Packed sparse attention, one wave per packed row (gather formulation).
//
// A wave owns one query row and streams that row's key set (its candidate
// list, or the causal range 0..t).  The wave is split into KPI = 512/D key
// groups of LPK = D/8 lanes; each lane holds 8 consecutive head dims, so a
// key row (D elements) is fetched by LPK lanes with 16-byte loads and each
// iteration of the inner loop covers KPI keys.  Scores are reduced inside a
// key group with xor-shuffles, the running maximum across groups, and the
// online softmax (base-2, scores pre-scaled by log2 e) keeps the output
// accumulator in f32 registers: no output traffic until the final, already
// normalised, store into the dense [b][h][t][d] position (fused scatter).
//
// XCD-aware launch: workgroups are dispatched round-robin over the 8 XCDs of
// MI355X, so logical block L is taken from physical block P with
// L = (P % 8) * ceil(nblk/8) + P / 8; each XCD then walks one contiguous
// slice of packed rows (rows of one head are adjacent), keeping that
// slice's keys in its own L2.
#include "pfa_common.h"

namespace pfa {

constexpr int kAttnWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;

enum AttnMode { kModeCand = 0, kModeCausal = 1, kModeMasked = 2 };

template <int DT>
__device__ __forceinline__ float load_mask(const void* m, int64_t off, int mdt) {
  if (mdt == PFA_F32) return ((const float*)m)[off];
  if (mdt == PFA_BF16) return bf16_to_f32(((const uint16_t*)m)[off]);
  return f16_to_f32(((const uint16_t*)m)[off]);
}

struct AttnArgs {
  pfa_tensor4 q, k, v, out;
  int H;
  int64_t T;
  const int32_t* token_idx;
  const int32_t* row_head;
  const int32_t* head_map;
  int64_t N;                // rows launched
  const int32_t* n_rows;    // device row count bounding N, or null
  const int32_t* cand;
  int64_t cand_stride;
  const int32_t* cand_len;
  const void* mask;
  int mask_dtype;
  const int32_t* head_max;
  float scale;
  const float* q_scale;
  const float* k_scale;
  const float* v_scale;
  int mode;
};

// Rows to process: the launch size, bounded by the device row count when one
// is given.
__device__ __forceinline__ int64_t attn_rows(const AttnArgs& a) {
  return a.n_rows ? min<int64_t>(a.N, (int64_t)a.n_rows[0]) : a.N;
}

// The grid is launched with a multiple of 8 workgroups, so this is a
// bijection on [0, gridDim.x).
__device__ __forceinline__ int64_t remap_block(int64_t P, int64_t nblk) {
  int64_t per = nblk / 8;
  return (P % 8) * per + P / 8;
}

template <int IDT, int ODT, int D>
__global__ void __launch_bounds__(64 * kAttnWaves)
sparse_attn_row_kernel(AttnArgs a) {
  using IT = typename Elem<IDT>::T;
  using OT = typename Elem<ODT>::T;
  constexpr int LPK = D / 8;       // lanes per key
  constexpr int KPI = 64 / LPK;    // keys per iteration
  constexpr int U = (KPI >= 16) ? 2 : 4;  // iterations per softmax step
  const int lane = threadIdx.x & 63;
  const int grp = lane / LPK;
  const int e = lane % LPK;

  const int64_t nblk = gridDim.x;
  const int64_t lb = remap_block(blockIdx.x, nblk);
  const int64_t r = lb * kAttnWaves + (threadIdx.x >> 6);
  if (r >= attn_rows(a)) return;

  const int64_t t = a.token_idx[r];
  const int hp = a.row_head[r];
  const int bh = a.head_map ? a.head_map[hp] : hp;
  const int64_t bb = bh / a.H, hh = bh % a.H;

  const IT* qp = (const IT*)a.q.ptr + bb * a.q.s_b + hh * a.q.s_h + t * a.q.s_t + 8 * e;
  const IT* kb = (const IT*)a.k.ptr + bb * a.k.s_b + hh * a.k.s_h + 8 * e;
  const IT* vb = (const IT*)a.v.ptr + bb * a.v.s_b + hh * a.v.s_h + 8 * e;

  float qf[8];
  load8<IDT>(qp, qf);
  float qmul = a.scale * kLog2e;
  float kmul = 1.f, vmul = 1.f;
  if constexpr (IDT == PFA_I8) {
    qmul *= a.q_scale[bh];
    kmul = a.k_scale[bh];
    vmul = a.v_scale[bh];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) qf[i] *= qmul;

  int64_t n;
  const int32_t* crow = nullptr;
  if (a.mode == kModeCand) {
    n = min<int64_t>(a.cand_len[r], a.cand_stride);
    crow = a.cand + r * a.cand_stride;
  } else if (a.mode == kModeCausal) {
    n = t + 1;
  } else {
    n = (int64_t)a.head_max[hp] + 1;
  }
  const bool has_mask = a.mask != nullptr;

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  float m = -INFINITY, l = 0.f;

  for (int64_t i0 = 0; i0 < n; i0 += (int64_t)KPI * U) {
    float kf[U][8], vf[U][8], s[U];
    int64_t key[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t i = i0 + u * KPI + grp;
      ok[u] = i < n;
      int64_t kk = 0;
      if (ok[u]) kk = (a.mode == kModeCand) ? (int64_t)crow[i] : i;
      kk = kk < 0 ? 0 : (kk >= a.T ? a.T - 1 : kk);
      key[u] = kk;
      load8<IDT>(kb + kk * a.k.s_t, kf[u]);
      load8<IDT>(vb + kk * a.v.s_t, vf[u]);
    }
    float cmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = __builtin_fmaf(qf[i], kf[u][i], d);
#pragma unroll
      for (int off = 1; off < LPK; off <<= 1) d += __shfl_xor(d, off, 64);
      d *= kmul;
      if (has_mask) d += kLog2e * load_mask<IDT>(a.mask, t * a.T + key[u], a.mask_dtype);
      s[u] = ok[u] ? d : -INFINITY;
      cmax = fmaxf(cmax, s[u]);
    }
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off, 64));
    float mn = fmaxf(m, cmax);
    if (mn == -INFINITY) continue;  // nothing finite yet
    float alpha = exp2f(m - mn);    // m == -inf -> 0
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float p = exp2f(s[u] - mn);
      l += p;
      float pv = p * vmul;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(pv, vf[u][i], acc[i]);
    }
    m = mn;
  }
  // combine key groups
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
    l += __shfl_xor(l, off, 64);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], off, 64);
  }
  if (grp == 0) {
    float inv = 1.f / l;  // l == 0 -> inf, 0 * inf -> NaN as softmax over all -inf
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (l == 0.f) ? __builtin_nanf("") : acc[i] * inv;
    OT* op = (OT*)a.out.ptr + bb * a.out.s_b + hh * a.out.s_h + t * a.out.s_t + 8 * e;
    store8<ODT>(op, o);
  }
}

// Generic head dimension (any D <= 1024): one key per lane for the scores,
// then lanes switch to head dims for P.V; q and the 64 probabilities of a
// step live in LDS.  Used for shapes the vectorised kernel does not cover.
template <int IDT, int ODT>
__global__ void __launch_bounds__(64)
sparse_attn_generic_kernel(AttnArgs a, int D) {
  using IT = typename Elem<IDT>::T;
  using OT = typename Elem<ODT>::T;
  extern __shared__ int64_t sm64[];
  int64_t* ks = sm64;                  // 64 keys (8-byte aligned at offset 0)
  float* ps = (float*)(sm64 + 64);     // 64
  float* qs = ps + 64;                 // D
  float* accs = qs + D;                // D
  const int lane = threadIdx.x;
  const int64_t r = blockIdx.x;
  if (r >= attn_rows(a)) return;
  const int64_t t = a.token_idx[r];
  const int hp = a.row_head[r];
  const int bh = a.head_map ? a.head_map[hp] : hp;
  const int64_t bb = bh / a.H, hh = bh % a.H;
  const IT* qp = (const IT*)a.q.ptr + bb * a.q.s_b + hh * a.q.s_h + t * a.q.s_t;
  const IT* kb = (const IT*)a.k.ptr + bb * a.k.s_b + hh * a.k.s_h;
  const IT* vb = (const IT*)a.v.ptr + bb * a.v.s_b + hh * a.v.s_h;
  float qmul = a.scale * kLog2e, kmul = 1.f, vmul = 1.f;
  if constexpr (IDT == PFA_I8) {
    qmul *= a.q_scale[bh];
    kmul = a.k_scale[bh];
    vmul = a.v_scale[bh];
  }
  for (int d = lane; d < D; d += 64) { qs[d] = load_f<IDT>(qp + d) * qmul; accs[d] = 0.f; }
  __syncthreads();
  int64_t n;
  const int32_t* crow = nullptr;
  if (a.mode == kModeCand) { n = min<int64_t>(a.cand_len[r], a.cand_stride); crow = a.cand + r * a.cand_stride; }
  else if (a.mode == kModeCausal) n = t + 1;
  else n = (int64_t)a.head_max[hp] + 1;
  float m = -INFINITY, l = 0.f;
  for (int64_t i0 = 0; i0 < n; i0 += 64) {
    int64_t i = i0 + lane;
    bool ok = i < n;
    int64_t kk = ok ? ((a.mode == kModeCand) ? (int64_t)crow[i] : i) : 0;
    kk = kk < 0 ? 0 : (kk >= a.T ? a.T - 1 : kk);
    float d = 0.f;
    for (int j = 0; j < D; ++j) d = __builtin_fmaf(qs[j], load_f<IDT>(kb + kk * a.k.s_t + j), d);
    d *= kmul;
    if (a.mask) d += kLog2e * load_mask<IDT>(a.mask, t * a.T + kk, a.mask_dtype);
    float s = ok ? d : -INFINITY;
    float cmax = s;
    for (int off = 1; off < 64; off <<= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off, 64));
    float mn = fmaxf(m, cmax);
    if (mn == -INFINITY) continue;
    float alpha = exp2f(m - mn);
    float p = exp2f(s - mn);
    float ps_sum = p;
    for (int off = 1; off < 64; off <<= 1) ps_sum += __shfl_xor(ps_sum, off, 64);
    l = l * alpha + ps_sum;
    ps[lane] = p * vmul;
    ks[lane] = kk;
    __syncthreads();
    int cnt = (int)min<int64_t>(64, n - i0);
    for (int dd = lane; dd < D; dd += 64) {
      float acc = accs[dd] * alpha;
      for (int j = 0; j < cnt; ++j) acc = __builtin_fmaf(ps[j], load_f<IDT>(vb + ks[j] * a.v.s_t + dd), acc);
      accs[dd] = acc;
    }
    __syncthreads();
    m = mn;
  }
  OT* op = (OT*)a.out.ptr + bb * a.out.s_b + hh * a.out.s_h + t * a.out.s_t;
  for (int dd = lane; dd < D; dd += 64) store_f<ODT>(op + dd, (l == 0.f) ? __builtin_nanf("") : accs[dd] / l);
}

template <int IDT, int ODT>
static int launch_attn(const AttnArgs& a, int D, hipStream_t s) {
  bool vec = (D % 8 == 0) && (D == 16 || D == 32 || D == 64 || D == 128);
  auto al = [](const pfa_tensor4& x, int esz) {
    return ((uintptr_t)x.ptr % (8 * esz)) == 0 && x.s_b % 8 == 0 && x.s_h % 8 == 0 && x.s_t % 8 == 0;
  };
  int ies = (IDT == PFA_F32) ? 4 : (IDT == PFA_I8 ? 1 : 2);
  int oes = (ODT == PFA_F32) ? 4 : 2;
  vec = vec && al(a.q, ies) && al(a.k, ies) && al(a.v, ies) && al(a.out, oes);
  if (vec) {
    int64_t blocks = (a.N + kAttnWaves - 1) / kAttnWaves;
    blocks = (blocks + 7) / 8 * 8;
    PFA_CHECK_ARG(blocks < INT32_MAX, "pfa_sparse_attn_fwd: too many rows");
    switch (D) {
      case 16: sparse_attn_row_kernel<IDT, ODT, 16><<<(unsigned)blocks, 64 * kAttnWaves, 0, s>>>(a); break;
      case 32: sparse_attn_row_kernel<IDT, ODT, 32><<<(unsigned)blocks, 64 * kAttnWaves, 0, s>>>(a); break;
      case 64: sparse_attn_row_kernel<IDT, ODT, 64><<<(unsigned)blocks, 64 * kAttnWaves, 0, s>>>(a); break;
      default: sparse_attn_row_kernel<IDT, ODT, 128><<<(unsigned)blocks, 64 * kAttnWaves, 0, s>>>(a); break;
    }
  } else {
    PFA_CHECK_ARG(D <= 4096, "pfa_sparse_attn_fwd: D=%d too large", D);
    size_t lds = (size_t)(2 * D + 64) * 4 + 64 * 8;
    sparse_attn_generic_kernel<IDT, ODT><<<(unsigned)a.N, 64, lds, s>>>(a, D);
  }
  PFA_CHECK_LAUNCH("pfa_sparse_attn_fwd");
  return PFA_OK;
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_sparse_attn_fwd(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v, int in_dtype, pfa_tensor4 out,
                                   int out_dtype, int H, int64_t T, int D, const int32_t* token_idx,
                                   const int32_t* row_head, const int32_t* head_map, int64_t N,
                                   const int32_t* n_rows_dev, const int32_t* cand,
                                   int64_t cand_stride, const int32_t* cand_len, const void* mask, int mask_dtype,
                                   const int32_t* head_max_token, float scale, const float* q_scale,
                                   const float* k_scale, const float* v_scale, void* stream) {
  clear_error();
  PFA_CHECK_ARG(H > 0 && T > 0 && D > 0 && N >= 0, "pfa_sparse_attn_fwd: bad sizes H=%d T=%lld D=%d N=%lld", H,
                (long long)T, D, (long long)N);
  if (N == 0) return PFA_OK;
  PFA_CHECK_ARG(q.ptr && k.ptr && v.ptr && out.ptr && token_idx && row_head, "pfa_sparse_attn_fwd: null pointer");
  PFA_CHECK_ARG(cand == nullptr || cand_len != nullptr, "pfa_sparse_attn_fwd: cand without lengths");
  PFA_CHECK_ARG(cand != nullptr || mask == nullptr || head_max_token != nullptr,
                "pfa_sparse_attn_fwd: masked dense branch needs head_max_token");
  PFA_CHECK_ARG(mask == nullptr || mask_dtype == PFA_F32 || mask_dtype == PFA_BF16 || mask_dtype == PFA_F16,
                "pfa_sparse_attn_fwd: bad mask dtype");
  PFA_CHECK_ARG(in_dtype != PFA_I8 || (q_scale && k_scale && v_scale), "pfa_sparse_attn_fwd: int8 needs scales");
  AttnArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.H = H; a.T = T; a.token_idx = token_idx; a.row_head = row_head; a.head_map = head_map; a.N = N;
  a.n_rows = n_rows_dev;
  a.cand = cand; a.cand_stride = cand_stride; a.cand_len = cand_len; a.mask = mask; a.mask_dtype = mask_dtype;
  a.head_max = head_max_token; a.scale = scale; a.q_scale = q_scale; a.k_scale = k_scale; a.v_scale = v_scale;
  a.mode = cand ? kModeCand : (mask ? kModeMasked : kModeCausal);
  hipStream_t s = as_stream(stream);
  if (in_dtype == PFA_F32 && out_dtype == PFA_F32) return launch_attn<PFA_F32, PFA_F32>(a, D, s);
  if (in_dtype == PFA_BF16 && out_dtype == PFA_BF16) return launch_attn<PFA_BF16, PFA_BF16>(a, D, s);
  if (in_dtype == PFA_F16 && out_dtype == PFA_F16) return launch_attn<PFA_F16, PFA_F16>(a, D, s);
  if (in_dtype == PFA_BF16 && out_dtype == PFA_F32) return launch_attn<PFA_BF16, PFA_F32>(a, D, s);
  if (in_dtype == PFA_I8 && out_dtype == PFA_F32) return launch_attn<PFA_I8, PFA_F32>(a, D, s);
  if (in_dtype == PFA_I8 && out_dtype == PFA_BF16) return launch_attn<PFA_I8, PFA_BF16>(a, D, s);
  if (in_dtype == PFA_I8 && out_dtype == PFA_F16) return launch_attn<PFA_I8, PFA_F16>(a, D, s);
  set_error("pfa_sparse_attn_fwd: unsupported dtype pair in=%d out=%d", in_dtype, out_dtype);
  return PFA_E_UNSUPPORTED;
}
