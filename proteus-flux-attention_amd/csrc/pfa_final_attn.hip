// All-query attention over an int8 shortlist: the final pass of the chunked
// shortlist pipeline (config 5).  Every query token t of one sequence
// attends to the S shortlisted keys; with `causal`, only to keys whose
// original position key_pos[j] <= t.  K and V of the shortlist are int8 with
// one symmetric scale per (head, key row).
//
// Every key is read by every 128-query tile of its head (8,192 tiles at
// T = 2^20), so the shortlist is dequantised once per call, into bf16
// working copies in the workspace; the attention then streams 64-key tiles
// of them by LDS DMA into the swizzled 128-byte-row layout of the bf16
// attention kernels (the V^T operand from the LDS transpose read), and
// S = Q K^T and O += P V run on v_mfma_f32_16x16x32_bf16 with an online
// softmax in f32 registers.  (Dequantising inside every tile spent about 2 ms
// of VALU time at config 5.)
//
// Workgroup: 4 waves, 128 consecutive query tokens of one head (32 per wave
// in two 16-query MFMA column groups).  The shortlist is sorted by
// position, so a query tile's keys are a prefix of it: keys below
// rng.x (position < first token of the tile) are visible to every query and
// run unmasked; the at most few keys in [rng.x, rng.y) are masked per
// (query, key).  Block b handles head b % H, so on 8 XCDs each XCD's L2
// holds one head's K/V; tiles run heaviest first.
//
// Precision.  Scores are in log2 units: K carries the factor
// c = k_scale * scale * log2(e).  A single bf16 copy of k8 * c would round
// every key element to 8 bits, and with large scores (rows of 4x the
// typical norm, whose single keys dominate their queries) that moves a
// score by tenths and the output by more than the bf16 tolerance.  So K is
// held as two bf16 parts, hi = bf16(k8 * c) and lo = bf16(k8 * c - hi)
// (their sum is k8 * c to about 2^-17), and every QK^T product is the sum of
// two MFMA products; V likewise (hi/lo of v8 * v_scale).  The softmax takes
// the exact row maximum (the dominant key's P is exactly 1), so what
// remains is the bf16 rounding of P for the P.V product.
#include "pfa_common.h"

namespace pfa {
namespace fin {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQ = 32 * kWaves;  // queries per workgroup
constexpr int kTile = kSwzKeys;  // keys per tile
constexpr int kD = 64;
constexpr float kRescaleLog2 = 0.0f;  // rescale when some row's max rises

#ifndef PFA_FIN_STAGES
#define PFA_FIN_STAGES 2
#endif
constexpr int kStages = PFA_FIN_STAGES;  // LDS ring of K/V tiles

struct Args {
  const uint16_t* q;
  int64_t q_sh, q_st;
  uint16_t* out;
  int64_t o_sh, o_st;
  const uint16_t* kb;  // dequantised shortlist, bf16 (H, S, 64): hi parts
  const uint16_t* vb;
  const uint16_t* kl;  // lo parts
  const uint16_t* vl;
  const int32_t* kpos;
  const int2* rng;
  int H, S, causal, nqt;
  int64_t T;
};

struct St {
  float m, l;
  f32x4_t acc[4];
};

__device__ __forceinline__ float i8f(uint32_t w, int e) { return (float)(int)(int8_t)((w >> (8 * e)) & 0xffu); }

// hi = bf16(x8 * scale) and lo = bf16(x8 * scale - hi) for the (H*S, 64)
// rows of K and V: thread -> row idx/4, elements 16*(idx%4) .. +15.  K rows
// carry the factor kmul = scale * log2(e): x8 * (k_scale * kmul).
__global__ void __launch_bounds__(256) dequant_kernel(const int8_t* __restrict__ k8, const int8_t* __restrict__ v8,
                                                      const float* __restrict__ ks, const float* __restrict__ vs,
                                                      int64_t rows, float kmul, uint16_t* __restrict__ kh,
                                                      uint16_t* __restrict__ vh, uint16_t* __restrict__ kl,
                                                      uint16_t* __restrict__ vl) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * 4) return;
  const int64_t row = idx >> 2;
  const int qd = (int)(idx & 3);
  const uint4 k = *reinterpret_cast<const uint4*>(k8 + row * kD + 16 * qd);
  const uint4 v = *reinterpret_cast<const uint4*>(v8 + row * kD + 16 * qd);
  const float kscale = ks[row] * kmul, vscale = vs[row];
  const uint32_t kw4[4] = {k.x, k.y, k.z, k.w};
  const uint32_t vw4[4] = {v.x, v.y, v.z, v.w};
  __bf16 kd[16], vd[16], kr[16], vr[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float kf = i8f(kw4[e >> 2], e & 3) * kscale;
    const float vf = i8f(vw4[e >> 2], e & 3) * vscale;
    kd[e] = (__bf16)kf;
    vd[e] = (__bf16)vf;
    kr[e] = (__bf16)(kf - (float)kd[e]);  // exact difference, rounded once
    vr[e] = (__bf16)(vf - (float)vd[e]);
  }
  const int64_t off = row * kD + 16 * qd;
  __builtin_memcpy(kh + off, kd, 32);
  __builtin_memcpy(vh + off, vd, 32);
  __builtin_memcpy(kl + off, kr, 32);
  __builtin_memcpy(vl + off, vr, 32);
}

// O += P V for the tile (P rounded to bf16), V as the sum of its hi part
// (tile th) and lo part (tile tl).
__device__ __forceinline__ void pv_accumulate(const float (&s)[2][16], const SwzTile& th, const SwzTile& tl,
                                              St (&st)[2]) {
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    bf16x8_t pb[2];
#pragma unroll
    for (int gr = 0; gr < 2; ++gr) {
      __bf16 pv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = (__bf16)s[gr][8 * kc + i];
        pv[4 + i] = (__bf16)s[gr][8 * kc + 4 + i];
      }
      __builtin_memcpy(&pb[gr], pv, 16);
    }
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const SwzTile& t = part ? tl : th;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        // V^T: lane (dim 16db + lane%16, g) holds keys 32kc + 4g + (0..3) and
        // 32kc + 16 + 4g + (0..3), matching pb
        const i16x4_t lo = ds_tr4(t.vtr(kc, 0, db));
        const i16x4_t hi = ds_tr4(t.vtr(kc, 1, db));
        bf16x8_t va;
        __builtin_memcpy(&va, &lo, 8);
        __builtin_memcpy(reinterpret_cast<char*>(&va) + 8, &hi, 8);
#pragma unroll
        for (int gr = 0; gr < 2; ++gr)
          st[gr].acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[gr], st[gr].acc[db], 0, 0, 0);
      }
    }
  }
}

// One 64-key tile: scores from the hi and lo parts of K, the tile's row
// maxima (rescaling when one rises), P, and the P.V products.  MASKED:
// keys past S or (causal) after the query's position are dropped; kpos is
// the shortlist's positions (global; read only in masked tiles).
template <bool MASKED>
__device__ __forceinline__ void tile(const bf16x8_t (&qf)[2][2], const SwzTile& th, const SwzTile& tl,
                                     const int32_t* kpos, int key0, int S, int causal, const int (&tq)[2],
                                     St (&st)[2]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  float s[2][16];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(th.kfrag(kb, 0));
    const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(th.kfrag(kb, 1));
    const bf16x8_t b0 = *reinterpret_cast<const bf16x8_t*>(tl.kfrag(kb, 0));
    const bf16x8_t b1 = *reinterpret_cast<const bf16x8_t*>(tl.kfrag(kb, 1));
#pragma unroll
    for (int gr = 0; gr < 2; ++gr) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b0, qf[gr][0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b1, qf[gr][1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[gr][0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[gr][1], c, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (MASKED) {
          const int key = key0 + 16 * kb + 4 * g + i;
          const int pos = kpos[key < S ? key : S - 1];
          const bool ok = key < S && (!causal || pos <= tq[gr]);
          s[gr][4 * kb + i] = ok ? c[i] : -INFINITY;
        } else {
          s[gr][4 * kb + i] = c[i];
        }
      }
    }
  }
  // lazy rescaling: the accumulators are rescaled only on tiles where some
  // row of the wave sees a new maximum; m stays the exact running max
#pragma unroll
  for (int gr = 0; gr < 2; ++gr) {
    float tmax = s[gr][0];
#pragma unroll
    for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[gr][i]);
    const float tm = max_over_rows4(tmax);
    if (__ballot(tm > st[gr].m + kRescaleLog2) != 0) {
      const float mn = fmaxf(st[gr].m, tm);
      const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(st[gr].m - mn);  // m == -inf -> 0
      st[gr].l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[gr].acc[db][i] *= alpha;
      st[gr].m = mn;
    }
    const float moff = st[gr].m == -INFINITY ? 0.f : st[gr].m;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[gr][i] = __builtin_amdgcn_exp2f(s[gr][i] - moff);  // -inf -> 0
      psum += s[gr][i];
    }
    st[gr].l += psum;
  }
  pv_accumulate(s, th, tl, st);
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

// two 4-wave workgroups per CU: each holds two 32 KB stages of hi and lo
// K/V tiles (64 KB of LDS), so two fit a CU
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8)))
final_attn_kernel(Args a) {
  // a stage: K hi, V hi, K lo, V lo (64 rows of 128 bytes each)
  __shared__ __align__(16) uint16_t ring[kStages][4 * kSwzTileElems];

  const int bid = blockIdx.x;
  const int h = bid % a.H;
  const int qt = a.nqt - 1 - bid / a.H;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  SwzLane L;
  L.init();
  const int2 rg = a.rng[qt];
  const int64_t t_base = (int64_t)qt * kQ;
  int tq[2];
  bool qv[2];
#pragma unroll
  for (int gr = 0; gr < 2; ++gr) {
    const int64_t t = t_base + 32 * wid + 16 * gr + r16;
    qv[gr] = t < a.T;
    tq[gr] = (int)(qv[gr] ? t : a.T - 1);
  }
  // per-head bases, wave-uniform (scalar registers for the DMA)
  const int64_t hoff = (int64_t)__builtin_amdgcn_readfirstlane(h) * a.S * kD;
  const uint16_t* kbh = a.kb + hoff;
  const uint16_t* vbh = a.vb + hoff;
  const uint16_t* klh = a.kl + hoff;
  const uint16_t* vlh = a.vl + hoff;
  const int ntile = (rg.y + kTile - 1) / kTile;
  const int drow = tid >> 3;  // this thread's DMA rows: drow and drow + 32
  const uint32_t ring_w = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]) + 1024u * (uint32_t)wid);
  constexpr uint32_t kStageBytes = 4 * kSwzTileElems * 2;
  auto request = [&](int i) {
    const int k0 = kTile * i;
    const int ka = min(k0 + drow, a.S - 1), kz = min(k0 + drow + 32, a.S - 1);
    const uint32_t st0 = ring_w + kStageBytes * (uint32_t)(i % kStages);
    dma_tile_rows64(kbh, vbh, ka, kz, st0);
    dma_tile_rows64(klh, vlh, ka, kz, st0 + 4 * kSwzTileElems);
  };
#pragma unroll
  for (int i = 0; i < kStages - 1; ++i)
    if (i < ntile) request(i);
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  bf16x8_t qf[2][2];
#pragma unroll
  for (int gr = 0; gr < 2; ++gr)
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      const uint4 w = *reinterpret_cast<const uint4*>(qh + (int64_t)tq[gr] * a.q_st + 32 * dc + 8 * g);
      __builtin_memcpy(&qf[gr][dc], &w, 16);
    }
  // settle the q fragments here: the tile loop then holds no load of the
  // compiler's own to wait for (its wait would also drain the tile requests)
  asm volatile("" : "+v"(qf[0][0]), "+v"(qf[0][1]), "+v"(qf[1][0]), "+v"(qf[1][1]));
  St st[2];
#pragma unroll
  for (int gr = 0; gr < 2; ++gr) {
    st[gr].m = -INFINITY;
    st[gr].l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) st[gr].acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // tile i has landed (tiles i+1 .. i+kStages-2 may still be in flight) and
  // every wave is done with tile i-1, whose stage takes tile i+kStages-1
  auto next = [&](int i) {
    if (kStages == 3 && i + 1 < ntile)
      dma_wait_barrier<2 * kDmaPerTile>();
    else
      dma_wait_barrier<0>();
    if (i + kStages - 1 < ntile) request(i + kStages - 1);
  };
  // the tiles whose keys all lie below the tile's first query, then the
  // masked tail (the keys in [rng.x, rng.y))
  const int nfull = min(rg.x / kTile, ntile);
  for (int i = 0; i < nfull; ++i) {
    next(i);
    const SwzTile th{ring[i % kStages], L}, tl{ring[i % kStages] + 2 * kSwzTileElems, L};
    tile<false>(qf, th, tl, a.kpos, kTile * i, a.S, a.causal, tq, st);
  }
  for (int i = nfull; i < ntile; ++i) {
    next(i);
    const SwzTile th{ring[i % kStages], L}, tl{ring[i % kStages] + 2 * kSwzTileElems, L};
    tile<true>(qf, th, tl, a.kpos, kTile * i, a.S, a.causal, tq, st);
  }
  uint16_t* oh = a.out + (int64_t)h * a.o_sh;
#pragma unroll
  for (int gr = 0; gr < 2; ++gr) {
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

// workspace: the query tiles' key ranges, then the bf16 K and V copies
// (hi parts, then lo parts)
static size_t fin_rng_bytes(int64_t T) {
  const int64_t nqt = (T + fin::kQ - 1) / fin::kQ;
  return ((size_t)(nqt > 0 ? nqt : 1) * sizeof(int2) + 255) / 256 * 256;
}
static size_t fin_copy_bytes(int H, int S) { return ((size_t)H * (size_t)S * fin::kD * 2 + 255) / 256 * 256; }

extern "C" int pfa_int8_kv_attn_workspace_size(int64_t T, int H, int S, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && T >= 0 && H >= 0 && S >= 0, "pfa_int8_kv_attn_workspace_size: bad arguments");
  *bytes = fin_rng_bytes(T) + 4 * fin_copy_bytes(H, S);
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
  PFA_CHECK_ARG((int64_t)S * fin::kD < INT32_MAX, "pfa_int8_kv_attn_fwd: S too large (%d)", S);
  size_t need = 0;
  pfa_int8_kv_attn_workspace_size(T, H, S, &need);
  PFA_CHECK_ARG(workspace && ws_bytes >= need, "pfa_int8_kv_attn_fwd: workspace of %zu bytes required", need);
  const int nqt = (int)((T + fin::kQ - 1) / fin::kQ);
  int2* rng = (int2*)workspace;
  uint16_t* kbf = (uint16_t*)((char*)workspace + fin_rng_bytes(T));
  uint16_t* vbf = (uint16_t*)((char*)kbf + fin_copy_bytes(H, S));
  uint16_t* klf = (uint16_t*)((char*)vbf + fin_copy_bytes(H, S));
  uint16_t* vlf = (uint16_t*)((char*)klf + fin_copy_bytes(H, S));
  const int64_t rows = (int64_t)H * S;
  fin::dequant_kernel<<<(unsigned)((rows * 4 + 255) / 256), 256, 0, s>>>(
      k8, v8, k_scale, v_scale, rows, scale * 1.4426950408889634f, kbf, vbf, klf, vlf);
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
  a.kl = klf;
  a.vl = vlf;
  a.kpos = key_pos;
  a.rng = rng;
  a.H = H;
  a.S = S;
  a.causal = causal ? 1 : 0;
  a.nqt = nqt;
  a.T = T;
  const int64_t blocks = (int64_t)nqt * H;
  PFA_CHECK_ARG(blocks < INT32_MAX, "pfa_int8_kv_attn_fwd: too many query tiles");
  fin::final_attn_kernel<<<(unsigned)blocks, fin::kThreads, 0, s>>>(a);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd");
  return PFA_OK;
}
