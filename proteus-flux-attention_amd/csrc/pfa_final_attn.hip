// All-query attention over an int8 shortlist: the final pass of the chunked
// shortlist pipeline (config 5).  Every query token t of one sequence
// attends to the S shortlisted keys; with `causal`, only to keys whose
// original position key_pos[j] <= t.  K and V of the shortlist are int8 with
// one symmetric scale per (head, key row); they are dequantised inside the
// tile: each staged 64-key tile is converted k8 * k_scale -> bf16 (and
// likewise V) into the swizzled 128-byte-row layout of the bf16 attention
// kernels (each thread writes two 16-byte chunks of K and two of V; the V^T
// operand comes from the LDS transpose read), then S = Q K^T and O += P V run
// on v_mfma_f32_16x16x32_bf16 with an online softmax in f32 registers.
//
// Workgroup: 4 waves, 128 consecutive query tokens of one head (32 per wave
// in two 16-query MFMA column groups).  The shortlist is sorted by
// position, so a query tile's keys are a prefix of it: keys below
// rng.x (position < first token of the tile) are visible to every query and
// run unmasked; the at most few keys in [rng.x, rng.y) are masked per
// (query, key).  Block b handles head b % H, so on 8 XCDs each XCD's L2
// holds one head's int8 K/V; tiles run heaviest first.
#include "pfa_common.h"

namespace pfa {
namespace fin {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQ = 32 * kWaves;  // queries per workgroup
constexpr int kTile = kSwzKeys;  // keys per tile
constexpr int kD = 64;
constexpr float kRescaleLog2 = 0.0f;  // rescale only when some row's max rises

struct Args {
  const uint16_t* q;
  int64_t q_sh, q_st;
  uint16_t* out;
  int64_t o_sh, o_st;
  const int8_t* k8;
  const int8_t* v8;
  const float* ks;
  const float* vs;
  const int32_t* kpos;
  const int2* rng;
  int H, S, causal, nqt;
  int64_t T;
  float scale_log2;
};

struct St {
  float m, l;
  f32x4_t acc[4];
};

// one 64-key tile staged by 256 threads: thread -> key tid/4, elements
// 16*(tid%4) .. +15 of that key's K and V rows
struct Fetch {
  uint4 k, v;
  float kscale, vscale;
  int pos;
};

__device__ __forceinline__ Fetch fetch(const int8_t* kb, const int8_t* vb, const float* ksb, const float* vsb,
                                       const int32_t* kpos, int key) {
  const int qd = threadIdx.x & 3;
  Fetch f;
  f.k = *reinterpret_cast<const uint4*>(kb + (int64_t)key * kD + 16 * qd);
  f.v = *reinterpret_cast<const uint4*>(vb + (int64_t)key * kD + 16 * qd);
  f.kscale = ksb[key];
  f.vscale = vsb[key];
  f.pos = kpos[key];
  return f;
}

__device__ __forceinline__ float i8f(uint32_t w, int e) { return (float)(int)(int8_t)((w >> (8 * e)) & 0xffu); }

// the thread's 16 K and 16 V elements (key tid/4, dims 16*(tid%4) ..+15) are
// chunks 2*(tid%4) and 2*(tid%4)+1 of the key's row
__device__ __forceinline__ void store(const Fetch& f, uint16_t* tile_base, int32_t* kp) {
  const int j = threadIdx.x >> 2, qd = threadIdx.x & 3;
  const int sw = tile_swz(j);
  const uint32_t kw4[4] = {f.k.x, f.k.y, f.k.z, f.k.w};
  const uint32_t vw4[4] = {f.v.x, f.v.y, f.v.z, f.v.w};
  __bf16 kd[16], vd[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    kd[e] = (__bf16)(i8f(kw4[e >> 2], e & 3) * f.kscale);
    vd[e] = (__bf16)(i8f(vw4[e >> 2], e & 3) * f.vscale);
  }
  uint4 kw[2], vw[2];
  __builtin_memcpy(kw, kd, 32);
  __builtin_memcpy(vw, vd, 32);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int slot = 8 * j + ((2 * qd + h) ^ sw);
    *reinterpret_cast<uint4*>(tile_base + 8 * slot) = kw[h];
    *reinterpret_cast<uint4*>(tile_base + kSwzTileElems + 8 * slot) = vw[h];
  }
  if (qd == 0) kp[j] = f.pos;
}

template <bool MASKED>
__device__ __forceinline__ void tile(const bf16x8_t (&qf)[2][2], const SwzTile& tl, const int32_t* kp, int key0,
                                     int S, int causal, const int (&tq)[2], float sl2, St (&st)[2]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  float s[2][16];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(tl.kfrag(kb, 0));
    const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(tl.kfrag(kb, 1));
#pragma unroll
    for (int gr = 0; gr < 2; ++gr) {
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[gr][0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[gr][1], c, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (MASKED) {
          const int kl = 16 * kb + 4 * g + i;
          const bool ok = key0 + kl < S && (!causal || kp[kl] <= tq[gr]);
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
    tmax = max_over_rows4(tmax);
    const float tm = tmax * sl2;
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
      s[gr][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[gr][i], sl2, -moff));  // -inf -> 0
      psum += s[gr][i];
    }
    st[gr].l += psum;
  }
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
    for (int db = 0; db < 4; ++db) {
      // V^T: lane (dim 16db + lane%16, g) holds keys 32kc + 4g + (0..3) and
      // 32kc + 16 + 4g + (0..3), matching pb
      const i16x4_t lo = ds_tr4(tl.vtr(kc, 0, db));
      const i16x4_t hi = ds_tr4(tl.vtr(kc, 1, db));
      bf16x8_t va;
      __builtin_memcpy(&va, &lo, 8);
      __builtin_memcpy(reinterpret_cast<char*>(&va) + 8, &hi, 8);
#pragma unroll
      for (int gr = 0; gr < 2; ++gr)
        st[gr].acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[gr], st[gr].acc[db], 0, 0, 0);
    }
  }
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

// at most 168 VGPRs: three 4-wave workgroups per CU
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 8))) final_attn_kernel(Args a) {
  __shared__ __align__(16) uint16_t ring[2][2 * kSwzTileElems];
  __shared__ int32_t kp[2][kTile];

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
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  bf16x8_t qf[2][2];
#pragma unroll
  for (int gr = 0; gr < 2; ++gr)
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      const uint4 w = *reinterpret_cast<const uint4*>(qh + (int64_t)tq[gr] * a.q_st + 32 * dc + 8 * g);
      __builtin_memcpy(&qf[gr][dc], &w, 16);
    }
  St st[2];
#pragma unroll
  for (int gr = 0; gr < 2; ++gr) {
    st[gr].m = -INFINITY;
    st[gr].l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) st[gr].acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int8_t* kb = a.k8 + (int64_t)h * a.S * kD;
  const int8_t* vb = a.v8 + (int64_t)h * a.S * kD;
  const float* ksb = a.ks + (int64_t)h * a.S;
  const float* vsb = a.vs + (int64_t)h * a.S;
  const int ntile = (rg.y + kTile - 1) / kTile;
  const int jrow = tid >> 2;
  if (ntile > 0) store(fetch(kb, vb, ksb, vsb, a.kpos, min(jrow, a.S - 1)), ring[0], kp[0]);
  __syncthreads();
  for (int i = 0; i < ntile; ++i) {
    const int cur = i & 1;
    const bool more = i + 1 < ntile;
    Fetch nxt;
    if (more) nxt = fetch(kb, vb, ksb, vsb, a.kpos, min(kTile * (i + 1) + jrow, a.S - 1));
    const int key0 = kTile * i;
    const SwzTile tl{ring[cur], L};
    if (key0 + kTile <= rg.x) tile<false>(qf, tl, kp[cur], key0, a.S, a.causal, tq, a.scale_log2, st);
    else tile<true>(qf, tl, kp[cur], key0, a.S, a.causal, tq, a.scale_log2, st);
    if (more) store(nxt, ring[cur ^ 1], kp[cur ^ 1]);
    __syncthreads();
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

extern "C" int pfa_int8_kv_attn_workspace_size(int64_t T, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes && T >= 0, "pfa_int8_kv_attn_workspace_size: bad arguments");
  const int64_t nqt = (T + fin::kQ - 1) / fin::kQ;
  *bytes = (size_t)(nqt > 0 ? nqt : 1) * sizeof(int2);
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
  PFA_CHECK_ARG(((uintptr_t)k8 % 8) == 0 && ((uintptr_t)v8 % 8) == 0, "pfa_int8_kv_attn_fwd: k8/v8 must be 8-byte aligned");
  size_t need = 0;
  pfa_int8_kv_attn_workspace_size(T, &need);
  PFA_CHECK_ARG(workspace && ws_bytes >= need, "pfa_int8_kv_attn_fwd: workspace of %zu bytes required", need);
  const int nqt = (int)((T + fin::kQ - 1) / fin::kQ);
  int2* rng = (int2*)workspace;
  fin::key_ranges_kernel<<<(unsigned)((nqt + 255) / 256), 256, 0, s>>>(key_pos, S, T, nqt, causal ? 1 : 0, rng);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd/ranges");
  fin::Args a;
  a.q = (const uint16_t*)q.ptr;
  a.q_sh = q.s_h;
  a.q_st = q.s_t;
  a.out = (uint16_t*)out.ptr;
  a.o_sh = out.s_h;
  a.o_st = out.s_t;
  a.k8 = k8;
  a.v8 = v8;
  a.ks = k_scale;
  a.vs = v_scale;
  a.kpos = key_pos;
  a.rng = rng;
  a.H = H;
  a.S = S;
  a.causal = causal ? 1 : 0;
  a.nqt = nqt;
  a.T = T;
  a.scale_log2 = scale * 1.4426950408889634f;
  const int64_t blocks = (int64_t)nqt * H;
  PFA_CHECK_ARG(blocks < INT32_MAX, "pfa_int8_kv_attn_fwd: too many query tiles");
  fin::final_attn_kernel<<<(unsigned)blocks, fin::kThreads, 0, s>>>(a);
  PFA_CHECK_LAUNCH("pfa_int8_kv_attn_fwd");
  return PFA_OK;
}
