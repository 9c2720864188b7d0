// All-query attention over an int8 shortlist: the final pass of the chunked
// shortlist pipeline (config 5).  Every query token t of one sequence
// attends to the S shortlisted keys; with `causal`, only to keys whose
// original position key_pos[j] <= t.  K and V of the shortlist are int8 with
// one symmetric scale per (head, key row).
//
// Every key is read by every 128-query tile of its head (8,192 tiles at
// T = 2^20), so the shortlist is converted once per call into bf16 working
// copies in the workspace; the attention then streams 64-key tiles of them
// by LDS DMA into the swizzled 128-byte-row layout of the bf16 attention
// kernels (the V^T operand from the LDS transpose read), and S = Q K^T and
// O += P V run on v_mfma_f32_16x16x32_bf16 with an online softmax in f32
// registers.  (Dequantising inside every tile spent about 2 ms of VALU time
// at config 5.)
//
// Workgroup: 4 waves, 128 consecutive query tokens of one head (32 per wave
// in two 16-query MFMA column groups).  The shortlist is sorted by
// position, so a query tile's keys are a prefix of it: keys below
// rng.x (position < first token of the tile) are visible to every query and
// run unmasked; the at most few keys in [rng.x, rng.y) are masked per
// (query, key).  Block b handles head b % H, so on 8 XCDs each XCD's L2
// holds one head's K/V; tiles run heaviest first.
//
// Precision.  The working copies hold the int8 values themselves, which
// bf16 represents exactly; the per-key scales stay in f32 and travel with
// each tile (512 bytes beside its 16 KB of K and V).  Scores are in log2
// units: the MFMA gives q . k8 (exact products, f32 sums) and one fma
// takes it to q . k8 * c_j - m, c_j = k_scale[j] * scale * log2(e) and m
// the row's reference maximum.  So a score is as accurate as an f32 dot
// product, with no rounding of the scaled K (a bf16 copy of k8 * c moved
// the scores of rows with 4x the typical norm by tenths).  m moves lazily
// (P <= 2^8 between moves) and the row sum l sums the unrounded P in f32.
// The P.V product takes the weights w_j = P_j * v_scale[j] against the
// exact v8: on a tile where some weight exceeds 1/8 of its row's running
// sum, as two bf16 parts (hi + lo, w to ~2^-17), else rounded once to
// bf16, whose independent errors of <= 2^-9 relative on weights that are
// each a small share of the row largely cancel.  QK^T and P.V are 32 MFMAs
// per 64-key tile and wave, 48 on the tiles that take the lo parts.
#include "pfa_common.h"

namespace pfa {
namespace fin {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
#ifndef PFA_FIN_NG
#define PFA_FIN_NG 2
#endif
constexpr int kNG = PFA_FIN_NG;        // 16-query MFMA column groups per wave
constexpr int kQ = 16 * kNG * kWaves;  // queries per workgroup
constexpr int kTile = kSwzKeys;  // keys per tile
constexpr int kD = 64;
#ifndef PFA_FIN_LAZY_LOG2
#define PFA_FIN_LAZY_LOG2 8.0f
#endif
constexpr float kLazyLog2 = PFA_FIN_LAZY_LOG2;  // P <= 2^kLazyLog2 between rescales
#ifndef PFA_FIN_LO_FRAC
#define PFA_FIN_LO_FRAC 0.125f
#endif
// a tile's P.V weights take their lo parts when one of them exceeds this
// fraction of its lane's running row sum
constexpr float kLoFrac = PFA_FIN_LO_FRAC;

#ifndef PFA_FIN_STAGES
#define PFA_FIN_STAGES 2
#endif
constexpr int kStages = PFA_FIN_STAGES;  // LDS ring of K/V tiles
// a stage: K tile, V tile (64 rows of 128 bytes each), then the tile's 64
// K scales and 64 V scales (f32)
constexpr int kScaleOff = 2 * kSwzTileElems;           // uint16 elements into a stage
constexpr int kStageElems = kScaleOff + 2 * kTile * 2;  // + 512 bytes
constexpr int kDmaPerStage = kDmaPerTile + 1;           // per wave: four tile rows and one scale chunk

struct Args {
  const uint16_t* q;
  int64_t q_sh, q_st;
  uint16_t* out;
  int64_t o_sh, o_st;
  const uint16_t* kb;  // shortlist K and V as bf16 integers (H, S, 64)
  const uint16_t* vb;
  const float* ksc;  // (H, Sp): k_scale * scale * log2(e), zero past S
  const float* vsc;  // (H, Sp): v_scale, zero past S
  const int32_t* kpos;
  const int2* rng;
  int H, S, Sp, causal, nqt;
  int64_t T;
};

struct St {
  float m, l;
  f32x4_t acc[4];
};

__device__ __forceinline__ float i8f(uint32_t w, int e) { return (float)(int)(int8_t)((w >> (8 * e)) & 0xffu); }

// bf16 copies of the int8 K and V rows (exact) and the padded f32 scale
// rows: thread -> row idx/4 of (H, Sp), elements 16*(idx%4) .. +15.  K
// scales carry the factor kmul = scale * log2(e).
__global__ void __launch_bounds__(256) dequant_kernel(const int8_t* __restrict__ k8, const int8_t* __restrict__ v8,
                                                      const float* __restrict__ ks, const float* __restrict__ vs,
                                                      int S, int Sp, int64_t rows, float kmul,
                                                      uint16_t* __restrict__ kh, uint16_t* __restrict__ vh,
                                                      float* __restrict__ kso, float* __restrict__ vso) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * 4) return;
  const int64_t prow = idx >> 2;
  const int qd = (int)(idx & 3);
  const int h = (int)(prow / Sp), j = (int)(prow - (int64_t)h * Sp);
  const int64_t row = (int64_t)h * S + j;
  if (qd == 0) {
    kso[prow] = j < S ? ks[row] * kmul : 0.f;
    vso[prow] = j < S ? vs[row] : 0.f;
  }
  if (j >= S) return;
  const uint4 k = *reinterpret_cast<const uint4*>(k8 + row * kD + 16 * qd);
  const uint4 v = *reinterpret_cast<const uint4*>(v8 + row * kD + 16 * qd);
  const uint32_t kw4[4] = {k.x, k.y, k.z, k.w};
  const uint32_t vw4[4] = {v.x, v.y, v.z, v.w};
  __bf16 kd[16], vd[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    kd[e] = (__bf16)i8f(kw4[e >> 2], e & 3);
    vd[e] = (__bf16)i8f(vw4[e >> 2], e & 3);
  }
  const int64_t off = row * kD + 16 * qd;
  __builtin_memcpy(kh + off, kd, 32);
  __builtin_memcpy(vh + off, vd, 32);
}

// The softmax and P.V half of a tile: P = exp2(s), s the scores relative
// to the row's reference maximum (the row sums take the unrounded P), the weights w = P * v_scale, and O += W V8 with W
// rounded to bf16.  lo (wave-uniform): each weight also enters by its
// rounding residue, bf16(w - bf16(w)), in a second product (hi + lo is w
// to about 2^-17), so a key that dominates its row adds v8 * v_scale at
// f32 accuracy.  With hi alone the weights are rounded once (relative
// error <= 2^-9 each); the caller sets lo on the tiles where some weight
// is a large fraction of its row's sum, and leaves it clear where every
// weight is a small share of the row, whose rounding errors are
// independent and largely cancel.  (One code path with a branch around
// the lo products per 32 keys: two whole paths, with and without them,
// took ~60 more registers.)
__device__ __forceinline__ void softmax_pv(float (&s)[kNG][16], const float* vsc, const SwzTile& t, St (&st)[kNG],
                                           bool lo) {
#pragma clang fp contract(off)
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) {
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 v4 = *reinterpret_cast<const float4*>(vsc + 16 * kb + 4 * g);
      const float vsj[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[gr][4 * kb + i]);  // -inf -> 0
        psum += p;
        s[gr][4 * kb + i] = p * vsj[i];
      }
    }
    st[gr].l += psum;
  }
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    bf16x8_t ph[kNG];
#pragma unroll
    for (int gr = 0; gr < kNG; ++gr) {
      __bf16 hv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) hv[i] = (__bf16)s[gr][8 * kc + i];
      __builtin_memcpy(&ph[gr], hv, 16);
    }
    bf16x8_t va[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      // V^T: lane (dim 16db + lane%16, g) holds keys 32kc + 4g + (0..3) and
      // 32kc + 16 + 4g + (0..3), matching the weights
      const i16x4_t lo4 = ds_tr4(t.vtr(kc, 0, db));
      const i16x4_t hi4 = ds_tr4(t.vtr(kc, 1, db));
      __builtin_memcpy(&va[db], &lo4, 8);
      __builtin_memcpy(reinterpret_cast<char*>(&va[db]) + 8, &hi4, 8);
#pragma unroll
      for (int gr = 0; gr < kNG; ++gr)
        st[gr].acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db], ph[gr], st[gr].acc[db], 0, 0, 0);
    }
    if (lo) {
      bf16x8_t pl[kNG];
#pragma unroll
      for (int gr = 0; gr < kNG; ++gr) {
        __bf16 lv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float w = s[gr][8 * kc + i];
          lv[i] = (__bf16)(w - (float)(__bf16)w);  // exact difference, rounded once
        }
        __builtin_memcpy(&pl[gr], lv, 16);
      }
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int gr = 0; gr < kNG; ++gr)
          st[gr].acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db], pl[gr], st[gr].acc[db], 0, 0, 0);
    }
  }
}

// One 64-key tile: scores q . k8 times the keys' scales, relative to the
// row's reference maximum m, then softmax_pv.  MASKED: keys past S or
// (causal) after the query's position are dropped; kpos is the shortlist's
// positions (global; read only in masked tiles).  sc: the tile's K scales
// (64 floats) followed by its V scales.  The lane's keys are 16kb + 4g + i,
// scores s[.][4kb + i].
//
// The reference moves lazily: only on a row's first visible key, or when
// one of its scores exceeds m by more than kLazyLog2 (then m becomes the
// row's maximum and the accumulators are rescaled).  Between moves P stays
// <= 2^kLazyLog2, and a score is one fma, q.k8 * c - m.
template <bool MASKED>
__device__ __forceinline__ void tile(const bf16x8_t (&qf)[kNG][2], const SwzTile& t, const float* sc,
                                     const int32_t* kpos, int key0, int S, int causal, const int (&tq)[kNG],
                                     St (&st)[kNG]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  float mneg[kNG];
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) mneg[gr] = st[gr].m == -INFINITY ? 0.f : -st[gr].m;
  float s[kNG][16];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(t.kfrag(kb, 0));
    const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(t.kfrag(kb, 1));
    const float4 k4 = *reinterpret_cast<const float4*>(sc + 16 * kb + 4 * g);
    const float ksj[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
    for (int gr = 0; gr < kNG; ++gr) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[gr][0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[gr][1], c, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = __builtin_fmaf(c[i], ksj[i], mneg[gr]);
        if constexpr (MASKED) {
          const int key = key0 + 16 * kb + 4 * g + i;
          const int pos = kpos[key < S ? key : S - 1];
          const bool ok = key < S && (!causal || pos <= tq[gr]);
          s[gr][4 * kb + i] = ok ? v : -INFINITY;
        } else {
          s[gr][4 * kb + i] = v;
        }
      }
    }
  }
  bool lo_needed = false;
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) {
    float tmax = s[gr][0];
#pragma unroll
    for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[gr][i]);
    const bool fresh = st[gr].m == -INFINITY;
    if (__ballot(fresh ? tmax > -INFINITY : tmax > kLazyLog2) != 0) {
      const float tm = max_over_rows4(tmax);  // the row's maximum, relative
      const bool mv = fresh ? tm > -INFINITY : tm > kLazyLog2;
      const float d = mv ? tm : 0.f;
      if (mv && !fresh) {  // a fresh row's accumulators are still zero
        const float alpha = __builtin_amdgcn_exp2f(-d);
        st[gr].l *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[gr].acc[db][i] *= alpha;
      }
      if (mv) st[gr].m = -mneg[gr] + d;
#pragma unroll
      for (int i = 0; i < 16; ++i) s[gr][i] -= d;
      tmax -= d;
    }
    // the lane's largest P against its partial row sum so far: that sum is
    // at most the row's, so a weight below kLoFrac of it is below kLoFrac of
    // the row's final sum (v_scale aside, which every key of the row shares
    // up to its own factor)
    lo_needed |= __builtin_amdgcn_exp2f(tmax) > kLoFrac * st[gr].l;
  }
  softmax_pv(s, sc + kTile, t, st, __ballot(lo_needed) != 0);
}

__global__ void __launch_bounds__(256) key_ranges_kernel(const int32_t* __restrict__ kpos, int S, int64_t T,
                                                         int nqt, int causal, int2* __restrict__ rng) {
  const int qt = blockIdx.x * blockDim.x + threadIdx.x;
  if (qt >= nqt) return;
  if (!causal) {
    rng[qt] = make_int2(S, S);
    return;
  }
  const int64_t t0 = (int64_t)qt * kQ;
  const int64_t t1 = (t0 + kQ < T ? t0 + kQ : T) - 1;
  int lo = 0, hi = S;  // first j with kpos[j] >= t0
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)kpos[mid] < t0) lo = mid + 1;
    else hi = mid;
  }
  const int below = lo;
  hi = S;  // first j with kpos[j] > t1
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)kpos[mid] <= t1) lo = mid + 1;
    else hi = mid;
  }
  rng[qt] = make_int2(below, lo);
}

#ifndef PFA_FIN_WAVES_PER_EU
#define PFA_FIN_WAVES_PER_EU 3
#endif
// a workgroup's ring is kStages x 16.5 KB of LDS
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(PFA_FIN_WAVES_PER_EU, 8)))
final_attn_kernel(Args a) {
  __shared__ __align__(16) uint16_t ring[kStages][kStageElems];

  const int bid = blockIdx.x;
  const int h = bid % a.H;
  const int qt = a.nqt - 1 - bid / a.H;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  SwzLane L;
  L.init();
  const int2 rg = a.rng[qt];
  const int64_t t_base = (int64_t)qt * kQ;
  int tq[kNG];
  bool qv[kNG];
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) {
    const int64_t t = t_base + 16 * kNG * wid + 16 * gr + r16;
    qv[gr] = t < a.T;
    tq[gr] = (int)(qv[gr] ? t : a.T - 1);
  }
  // per-head bases, wave-uniform (scalar registers for the DMA)
  const int hu = __builtin_amdgcn_readfirstlane(h);
  const int64_t hoff = (int64_t)hu * a.S * kD;
  const uint16_t* kbh = a.kb + hoff;
  const uint16_t* vbh = a.vb + hoff;
  // this wave's scale chunk: waves 0, 1 move K scales 0..31, 32..63 of the
  // tile, waves 2, 3 the V scales (lanes 0..7, 16 bytes each)
  const int wu = __builtin_amdgcn_readfirstlane(wid);
  const float* sch = (wu < 2 ? a.ksc : a.vsc) + (int64_t)hu * a.Sp + 32 * (wu & 1);
  const int ntile = (rg.y + kTile - 1) / kTile;
  const int drow = tid >> 3;  // this thread's DMA rows: drow and drow + 32
  const uint32_t ring0 = lds_addr(&ring[0][0]);
  const uint32_t ring_w = __builtin_amdgcn_readfirstlane(ring0 + 1024u * (uint32_t)wid);
  const uint32_t scl_w = __builtin_amdgcn_readfirstlane(ring0 + 2u * kScaleOff + 128u * (uint32_t)wid);
  constexpr uint32_t kStageBytes = kStageElems * 2;
  auto request = [&](int i) {
    const int k0 = kTile * i;
    const int ka = min(k0 + drow, a.S - 1), kz = min(k0 + drow + 32, a.S - 1);
    const uint32_t so = kStageBytes * (uint32_t)(i % kStages);
    dma_tile_rows64(kbh, vbh, ka, kz, ring_w + so);
    // the scale rows are padded to a multiple of 64 keys: always in bounds
    if (lane < 8) lds_dma16_s(sch, (uint32_t)(k0 + 4 * lane) * 4u, scl_w + so);
  };
#pragma unroll
  for (int i = 0; i < kStages - 1; ++i)
    if (i < ntile) request(i);
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  bf16x8_t qf[kNG][2];
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr)
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      const uint4 w = *reinterpret_cast<const uint4*>(qh + (int64_t)tq[gr] * a.q_st + 32 * dc + 8 * g);
      __builtin_memcpy(&qf[gr][dc], &w, 16);
    }
  // settle the q fragments here: the tile loop then holds no load of the
  // compiler's own to wait for (its wait would also drain the tile requests)
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) asm volatile("" : "+v"(qf[gr][0]), "+v"(qf[gr][1]));
  St st[kNG];
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) {
    st[gr].m = -INFINITY;
    st[gr].l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) st[gr].acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // tile i has landed (tiles i+1 .. i+kStages-2 may still be in flight) and
  // every wave is done with tile i-1, whose stage takes tile i+kStages-1
  auto next = [&](int i) {
    if (kStages == 3 && i + 1 < ntile)
      dma_wait_barrier<kDmaPerStage>();
    else
      dma_wait_barrier<0>();
    if (i + kStages - 1 < ntile) request(i + kStages - 1);
  };
  // the tiles whose keys all lie below the tile's first query, then the
  // masked tail (the keys in [rng.x, rng.y))
  const int nfull = min(rg.x / kTile, ntile);
  for (int i = 0; i < nfull; ++i) {
    next(i);
    const uint16_t* stg = ring[i % kStages];
    const SwzTile t{stg, L};
    tile<false>(qf, t, reinterpret_cast<const float*>(stg + kScaleOff), a.kpos, kTile * i, a.S, a.causal, tq, st);
  }
  for (int i = nfull; i < ntile; ++i) {
    next(i);
    const uint16_t* stg = ring[i % kStages];
    const SwzTile t{stg, L};
    tile<true>(qf, t, reinterpret_cast<const float*>(stg + kScaleOff), a.kpos, kTile * i, a.S, a.causal, tq, st);
  }
  uint16_t* oh = a.out + (int64_t)h * a.o_sh;
#pragma unroll
  for (int gr = 0; gr < kNG; ++gr) {
    float l = st[gr].l;
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!qv[gr]) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;  // a query with no visible key writes zeros
    uint16_t* op = oh + (int64_t)tq[gr] * a.o_st;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      uint16_t o4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = f32_to_bf16(st[gr].acc[db][i] * inv);
      *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) =
          make_uint2((uint32_t)o4[0] | ((uint32_t)o4[1] << 16), (uint32_t)o4[2] | ((uint32_t)o4[3] << 16));
    }
  }
}

}  // namespace fin
}  // namespace pfa

using namespace pfa;

// workspace: the query tiles' key ranges, the bf16 K and V copies, then the
// K and V scale rows (H, Sp) with Sp = S rounded up to 64 keys
static size_t fin_rng_bytes(int64_t T) {
  const int64_t nqt = (T + fin::kQ - 1) / fin::kQ;
  return ((size_t)(nqt > 0 ? nqt : 1) * sizeof(int2) + 255) / 256 * 256;
}
static int fin_padded(int S) { return (S + fin::kTile - 1) / fin::kTile * fin::kTile; }
static size_t fin_copy_bytes(int H, int S) { return ((size_t)H * (size_t)S * fin::kD * 2 + 255) / 256 * 256; }
static size_t fin_scale_bytes(int H, int S) { return ((size_t)H * (size_t)fin_padded(S) * 4 + 255) / 256 * 256; }

extern "C" int pfa_int8_kv_attn_workspace_size(int64_t T, int H, int S, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && T >= 0 && H >= 0 && S >= 0, "pfa_int8_kv_attn_workspace_size: bad arguments");
  *bytes = fin_rng_bytes(T) + 2 * fin_copy_bytes(H, S) + 2 * fin_scale_bytes(H, S);
  return PFA_OK;
}

extern "C" int pfa_int8_kv_attn_fwd(pfa_tensor4 q, pfa_tensor4 out, int64_t T, int H, int D, const int8_t* k8,
                                    const int8_t* v8, const float* k_scale, const float* v_scale,
                                    const int32_t* key_pos, int S, int causal, float scale, void* workspace,
                                    size_t ws_bytes, void* stream) {
  clear_error();
  PFA_CHECK_ARG(D == fin::kD, "pfa_int8_kv_attn_fwd: D must be 64 (got %d)", D);
  PFA_CHECK_ARG(T >= 0 && T < INT32_MAX && H > 0 && S >= 0, "pfa_int8_kv_attn_fwd: bad sizes T=%lld H=%d S=%d",
                (long long)T, H, S);
  if (T == 0) return PFA_OK;
  PFA_CHECK_ARG(q.ptr && out.ptr, "pfa_int8_kv_attn_fwd: null q/out");
  auto al = [](const pfa_tensor4& x) { return ((uintptr_t)x.ptr % 16) == 0 && x.s_h % 8 == 0 && x.s_t % 8 == 0; };
  PFA_CHECK_ARG(al(q) && al(out), "pfa_int8_kv_attn_fwd: q/out must be 16-byte aligned with strides of 8 elements");
  hipStream_t s = as_stream(stream);
  PFA_CHECK_ARG(S > 0, "pfa_int8_kv_attn_fwd: empty shortlist (S must be >= 1)");
  PFA_CHECK_ARG(k8 && v8 && k_scale && v_scale && key_pos, "pfa_int8_kv_attn_fwd: null shortlist pointer");
  PFA_CHECK_ARG(((uintptr_t)k8 % 16) == 0 && ((uintptr_t)v8 % 16) == 0, "pfa_int8_kv_attn_fwd: k8/v8 must be 16-byte aligned");
  PFA_CHECK_ARG((int64_t)fin_padded(S) * fin::kD < INT32_MAX, "pfa_int8_kv_attn_fwd: S too large (%d)", S);
  size_t need = 0;
  pfa_int8_kv_attn_workspace_size(T, H, S, &need);
  PFA_CHECK_ARG(workspace && ws_bytes >= need, "pfa_int8_kv_attn_fwd: workspace of %zu bytes required", need);
  const int nqt = (int)((T + fin::kQ - 1) / fin::kQ);
  const int Sp = fin_padded(S);
  int2* rng = (int2*)workspace;
  uint16_t* kbf = (uint16_t*)((char*)workspace + fin_rng_bytes(T));
  uint16_t* vbf = (uint16_t*)((char*)kbf + fin_copy_bytes(H, S));
  float* ksf = (float*)((char*)vbf + fin_copy_bytes(H, S));
  float* vsf = (float*)((char*)ksf + fin_scale_bytes(H, S));
  const int64_t rows = (int64_t)H * Sp;
  fin::dequant_kernel<<<(unsigned)((rows * 4 + 255) / 256), 256, 0, s>>>(
      k8, v8, k_scale, v_scale, S, Sp, rows, scale * 1.4426950408889634f, kbf, vbf, ksf, vsf);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd/dequant");
  fin::key_ranges_kernel<<<(unsigned)((nqt + 255) / 256), 256, 0, s>>>(key_pos, S, T, nqt, causal ? 1 : 0, rng);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd/ranges");
  fin::Args a;
  a.q = (const uint16_t*)q.ptr;
  a.q_sh = q.s_h;
  a.q_st = q.s_t;
  a.out = (uint16_t*)out.ptr;
  a.o_sh = out.s_h;
  a.o_st = out.s_t;
  a.kb = kbf;
  a.vb = vbf;
  a.ksc = ksf;
  a.vsc = vsf;
  a.kpos = key_pos;
  a.rng = rng;
  a.H = H;
  a.S = S;
  a.Sp = Sp;
  a.causal = causal ? 1 : 0;
  a.nqt = nqt;
  a.T = T;
  const int64_t blocks = (int64_t)nqt * H;
  PFA_CHECK_ARG(blocks < INT32_MAX, "pfa_int8_kv_attn_fwd: too many query tiles");
  fin::final_attn_kernel<<<(unsigned)blocks, fin::kThreads, 0, s>>>(a);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd");
  return PFA_OK;
}
