// Shortlist attention on bf16 MFMA, driven by the structure of the
// candidate sets instead of materialised candidate lists.
//
// For packed row r (compact head p, token t) the reference's candidate set
// (sparse_attn.py:376-596, no truncation) is the disjoint union of
//   W(t) = [lo, t]                       local window, lo = t - min(t+1, w) + 1
//   A(t) = { t - s*j : j0 <= j <= min(slots, t/s) }   strided anchors below lo
//   X(t) = proto positions below lo that are not strided anchors, plus the
//          clamped anchor 0 when max(t - s*slots, 0) == 0 is not itself a
//          strided anchor ("zero anchor")
// and a position p belongs to the prototype prefix set of t exactly when
// p <= t < evict[p]; the set of t is drawn from the set table row of t's
// 64-token block plus the block's own tokens (pfa_proto_prefix_blocks).
//
// Pass 1, short_anchor_kernel: one workgroup per (compact head, residue class
// c = t mod s).  The anchors of every row of the class lie on the strided
// key sequence c, c+s, c+2s, ...; row M = (t-c)/s uses keys
// m in [max(0, M-slots), M-j0], so the class is a banded attention over one
// shared key sequence.  Writes unnormalised online-softmax partials
// (max, sum, acc[64]) per row.
//
// Pass 2, short_main_kernel: one workgroup per 64 consecutive packed rows.
// Rows of one head whose tokens span less than w share the window union
// [lo_first, t_last] and all their prototype keys lie in the prefix set of
// the first row (anything newer than t_first is inside every window), so a
// "segment" of rows streams those keys once, masks per (row, key), merges the
// anchor partial and writes the normalised bf16 row into [b][h][t][:].
//
// Tiles: 4 waves x 16 query rows, 64 keys per tile.  Key tiles reach LDS by
// DMA (global_load_lds, no register staging) into a ring of stages, so the
// next tiles are in flight while one is computed; rows are 128 bytes with
// XOR-swizzled 16-byte chunks (conflict-free K fragment reads; the V^T
// operand comes from the LDS transpose read).  Each wave computes
// S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_16x16x32_bf16, so a lane
// owns one query row throughout: the softmax max needs two cross-lane
// permutes per tile.
#include "pfa_common.h"

namespace pfa {


constexpr int kRows = 64;   // query rows per workgroup
constexpr int kTile = 64;   // keys per tile
// floats per partial row: m, l, pad, pad, acc[64 * NH] (NH 64-dim halves)
__host__ __device__ constexpr int part_w(int NH) { return 4 + 64 * NH; }
constexpr int kPartW = part_w(1);
constexpr int kMaxProto = 1024;
constexpr int kClassChunk = 2048;  // anchor pass: class rows compacted per round
constexpr float kRescaleLog2 = 0.0f;  // rescale only when some row's max rises
// Anchor-pass fusions.  Workgroup (c, p) owns the tokens t = c (mod stride)
// of global head head_map[p]: every (head, token) pair of the active heads
// belongs to exactly one workgroup, and the P_cap - P workgroups past the
// active heads take the inactive ones.
//   kFuseKRope: rotate the k rows of the active heads in place with the q
//     RoPE tables (the arithmetic of the RoPE kernels), before the class's
//     anchor tiles are read;
//   kFuseZero: write zeros to out for every (head, token) pair without a
//     packed row (the rows the main pass does not write).
constexpr int kFuseKRope = 1;
constexpr int kFuseZero = 2;

struct ShortArgs {
  pfa_tensor4 q, k, v, out;
  int H;
  int64_t T;
  const int32_t* token_idx;
  const int32_t* row_head;
  const int32_t* head_map;
  int64_t N;
  int local_w, stride, slots;
  const int32_t* blk;    // (B, nblk, K) prefix set table rows, or null
  int K;
  int64_t nblk;
  const int32_t* evict;  // (B, T) or null
  const int32_t* row_of; // (B*H, T)
  const int32_t* summary;
  float* part;           // (N, part_w(NH))
  int32_t* lengths;      // (N) or null
  const uint16_t* rcos;  // (T, 64) RoPE tables applied to q rows on load, or null
  const uint16_t* rsin;
  float scale_log2;
  int off32;  // every K/V byte offset of the sequence fits in 32 bits
  // per global head (b*H + h) int8 scales of q, k, v, or null: q, k, v then
  // hold the integer values (exact in bf16) of the per-head int8
  // quantisation, scores are scaled by q_scale*k_scale and outputs by v_scale
  const float* qsc;
  const float* ksc;
  const float* vsc;
  // work the anchor pass takes over from separate passes (kFuse* bits)
  int fuse;
  // head dim D (16, 32 or 64) and cmask = D/8 - 1: rows narrower than 64
  // are attended as 64-wide rows whose q dims past D are zero (their K/V
  // tile chunks hold copies of the row's own chunks, see dma_tile)
  int dh;
  uint32_t cmask;
  __device__ __forceinline__ float head_scale_log2(int bh) const {
    return qsc ? scale_log2 * (qsc[bh] * ksc[bh]) : scale_log2;
  }
  __device__ __forceinline__ float head_out_scale(int bh) const { return vsc ? vsc[bh] : 1.f; }
};

// NH: 64-dim halves of the head (1, or 2 for D = 128); acc[4 * NH] holds
// the lane's output dims 16db + 4g .. +3.
template <int NH>
struct QState {
  float m, l;
  f32x4_t acc[4 * NH];
  int cnt;
};

// K/V tile of 64 keys and NH 64-dim halves in LDS: the K halves at base +
// h * kSwzTileElems, then the V halves, each a swizzled 64 x 64 tile
// (SwzTile's layout); kfrag / vtr as SwzTile's, with dc < 2 * NH and
// db < 4 * NH.
template <int NH>
struct SwzTileH {
  const uint16_t* base;
  const SwzLane& L;
  __device__ __forceinline__ const uint16_t* kfrag(int kb, int dc) const {
    return base + (dc >> 1) * kSwzTileElems + 1024 * kb + L.ko[dc & 1];
  }
  __device__ __forceinline__ const uint16_t* vtr(int kc, int h, int db) const {
    return base + (NH + (db >> 2)) * kSwzTileElems + 64 * (32 * kc + 16 * h) + L.vo[db & 3];
  }
};

__device__ __forceinline__ int64_t win_lo(int64_t t, int w) {
  int64_t wl = t + 1 < w ? t + 1 : w;
  return t - wl + 1;
}

__device__ __forceinline__ bool strided_anchor(int64_t t, int64_t p, int s, int slots) {
  if (s <= 0 || slots <= 0 || p >= t) return false;
  int64_t d = t - p;
  return (d % s) == 0 && d / s <= slots;
}

__device__ __forceinline__ bool zero_anchor(int64_t t, int s, int slots) {
  if (s <= 0 || slots <= 0) return false;
  int64_t q = t / s;
  return slots > q && !((t % s) == 0 && q >= 1);
}

__device__ __forceinline__ uint16_t bf16_bits(float f) { return f32_to_bf16(f); }

constexpr int kTileElems = kSwzTileElems;  // one unpadded K or V tile, bf16 elements

// Waves raise their issue priority (s_setprio, arbitration only) while
// they issue a tile's QK^T and P.V products, so that a wave with matrix
// work ready issues it ahead of the softmax arithmetic of the other waves
// on its SIMD (the matrix unit would otherwise idle behind it).
//
// One 64-key tile for the 16 query rows of this wave, in two stages that
// every tile kind shares: the scores (qk_tile, or qk_tile_b with the mask
// -- -inf for keys of the tile that are not candidates of the lane's row --
// as the MFMA's initial accumulator) and softmax_pv (online softmax and
// the P.V product).  One accumulation path for all tile kinds keeps the
// running state in the same registers across tiles.
//
// S^T = K Q^T: s[kb][i] is the raw score of tile key 16kb + 4g + i against
// the lane's query row (the scale is applied in the exp argument).
template <int NQ, typename Tile>
__device__ __forceinline__ void qk_tile(const bf16x8_t (&qf)[NQ], const Tile& t, float (&s)[4][4]) {
  // all the fragment reads first, then four independent MFMA chains
  bf16x8_t a[NQ][4];
#pragma unroll
  for (int dc = 0; dc < NQ; ++dc)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) a[dc][kb] = *reinterpret_cast<const bf16x8_t*>(t.kfrag(kb, dc));
  f32x4_t c[4];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    c[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0][kb], qf[0], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
  for (int dc = 1; dc < NQ; ++dc)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) c[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[dc][kb], qf[dc], c[kb], 0, 0, 0);
  __builtin_amdgcn_s_setprio(0);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kb][i] = c[kb][i];
}

// The same product with the accumulator started at bias[kb] (0 for a
// candidate, -inf for a key the row does not take): the mask rides on the
// MFMA's C operand, so a masked tile needs no select after the product.
// For finite q and k the scores are those of qk_tile with -inf in the
// masked places.
template <int NQ, typename Tile>
__device__ __forceinline__ void qk_tile_b(const bf16x8_t (&qf)[NQ], const Tile& t, const f32x4_t (&bias)[4],
                                          float (&s)[4][4]) {
  bf16x8_t a[NQ][4];
#pragma unroll
  for (int dc = 0; dc < NQ; ++dc)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) a[dc][kb] = *reinterpret_cast<const bf16x8_t*>(t.kfrag(kb, dc));
  f32x4_t c[4];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) c[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0][kb], qf[0], bias[kb], 0, 0, 0);
#pragma unroll
  for (int dc = 1; dc < NQ; ++dc)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) c[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[dc][kb], qf[dc], c[kb], 0, 0, 0);
  __builtin_amdgcn_s_setprio(0);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kb][i] = c[kb][i];
}

// Window bias: keys kl of the tile in [lo, hi] (tile-local) get 0, the
// others -inf; lo4 = lo - 4g and hi4 = hi - 4g, so each element is one
// compare against a constant (16kb + i).  LO / HI pick which bounds can cut
// this tile (a wave-uniform choice).
template <bool LO, bool HI>
__device__ __forceinline__ void bias_range(f32x4_t (&b)[4], int lo4, int hi4) {
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 16 * kb + i;
      bool ok = true;
      if constexpr (LO) ok = ok & (c >= lo4);
      if constexpr (HI) ok = ok & (c <= hi4);
      b[kb][i] = ok ? 0.f : -INFINITY;
    }
}

// Candidates counted from a masked tile's scores: the masked places are
// -inf, every other score is finite (finite q and k).
__device__ __forceinline__ int count_finite(const float (&s)[4][4]) {
  int n = 0;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) n += s[kb][i] != -INFINITY ? 1 : 0;
  return n;
}

// Scores of a window tile whose lane's candidates are the keys kl in
// [lo, hi] (tile-local, lo > hi for none); need_lo / need_hi say whether
// some row of the wave is cut by that bound in this tile.  Uncut tiles take
// the plain product.
template <bool COUNT, int NQ, typename Tile>
__device__ __forceinline__ void window_qk(const bf16x8_t (&qf)[NQ], const Tile& t, bool need_lo, bool need_hi, int lo,
                                          int hi, int& cnt, float (&s)[4][4]) {
  const int g4 = 4 * ((threadIdx.x & 63) >> 4);
  // the conditions are wave-uniform: scalar branches
  need_lo = __builtin_amdgcn_readfirstlane(need_lo ? 1 : 0) != 0;
  need_hi = __builtin_amdgcn_readfirstlane(need_hi ? 1 : 0) != 0;
  if (!need_lo && !need_hi) {
    if constexpr (COUNT) cnt += 16;
    qk_tile(qf, t, s);
    return;
  }
  f32x4_t bias[4];
  if (need_lo && need_hi) bias_range<true, true>(bias, lo - g4, hi - g4);
  else if (need_lo) bias_range<true, false>(bias, lo - g4, 0);
  else bias_range<false, true>(bias, 0, hi - g4);
  qk_tile_b(qf, t, bias, s);
  if constexpr (COUNT) cnt += count_finite(s);
}

// Online softmax (exp2 on v_exp_f32 directly: arguments are <= 0, -inf
// gives 0): updates the running max / sum (rescaling the accumulator when
// the max rises) and returns P rounded to bf16 (v_cvt_pk_bf16_f32, round to
// nearest even) as the two B operands of the P.V product, pb[kc] holding
// keys 32kc + 4g + (0..3) and 32kc + 16 + 4g + (0..3).
template <int NH>
__device__ __forceinline__ void softmax_p(float (&s)[4][4], float scale_log2, QState<NH>& st, bf16x8_t (&pb)[2]) {
  float tmax = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[kb][i]);
  tmax = max_over_rows4(tmax);
  // Lazy rescaling: the accumulator is rescaled only on tiles where some row
  // of the wave sees a new maximum (a wave-uniform branch); st.m stays the
  // exact running max (log2 units), so every P <= 1 and the arithmetic is
  // that of the plain online softmax.
  const float tm = tmax * scale_log2;
  if (__ballot(tm > st.m + kRescaleLog2) != 0) {
    const float mn = fmaxf(st.m, tm);
    const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(st.m - mn);  // st.m == -inf -> 0
    st.l *= alpha;
#pragma unroll
    for (int db = 0; db < 4 * NH; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) st.acc[db][i] *= alpha;
    st.m = mn;
  }
  // a row whose reference is still -inf has seen only masked keys: its
  // scores are -inf and its P is 0 with any finite offset
  const float moff = st.m == -INFINITY ? 0.f : st.m;
  float psum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[kb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], scale_log2, -moff));  // -inf -> 0
      psum += s[kb][i];
    }
  st.l += psum;
  // P is rounded to bf16 for the P.V MFMA (the reference's bf16 path rounds
  // its probabilities to bf16 too); the accumulator stays f32.
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    __bf16 pv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = (__bf16)s[2 * kc][i];
      pv[4 + i] = (__bf16)s[2 * kc + 1][i];
    }
    __builtin_memcpy(&pb[kc], pv, 16);
  }
}

// A operand V^T of the P.V product: lane (dim 16db + r16, g) holds keys
// 32kc + 4g + (0..3) and 32kc + 16 + 4g + (0..3), matching pb[kc].
template <typename Tile>
__device__ __forceinline__ bf16x8_t v_frag(const Tile& t, int kc, int db) {
  const i16x4_t lo = ds_tr4(t.vtr(kc, 0, db));
  const i16x4_t hi = ds_tr4(t.vtr(kc, 1, db));
  bf16x8_t va;
  __builtin_memcpy(&va, &lo, 8);
  __builtin_memcpy(reinterpret_cast<char*>(&va) + 8, &hi, 8);
  return va;
}

// Softmax and O^T += V^T P^T for one 16-row group.
// The sixteen transpose reads of V^T are issued before the softmax, so
// their latency overlaps the exponentials instead of sitting between the
// P.V products.
// With two 64-dim halves the second half's V^T reads follow the first
// half's products (the registers of one half's operands at a time).
template <int NH, typename Tile>
__device__ __forceinline__ void softmax_pv(float (&s)[4][4], const Tile& t, float scale_log2, QState<NH>& st) {
  bf16x8_t va[2][4];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int db = 0; db < 4; ++db) va[kc][db] = v_frag(t, kc, db);
  bf16x8_t pb[2];
  softmax_p(s, scale_log2, st, pb);
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    if (h > 0) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 4; ++db) va[kc][db] = v_frag(t, kc, 4 * h + db);
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < 4; ++db)
        st.acc[4 * h + db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[kc][db], pb[kc], st.acc[4 * h + db], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  }
}

// The lane's q chunks 4dc + g (dims 32dc + 8g ..+7); with NARROW the
// chunks past cmask (a row of 16 or 32 dims) are zero.
template <int NQ, bool NARROW>
__device__ __forceinline__ void load_q(const uint16_t* qrow, bf16x8_t (&qf)[NQ], uint32_t cmask) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int dc = 0; dc < NQ; ++dc) {
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (!NARROW || (uint32_t)(4 * dc + g) <= cmask) w = *reinterpret_cast<const uint4*>(qrow + 32 * dc + 8 * g);
    __builtin_memcpy(&qf[dc], &w, 16);
  }
}

// q row with RoPE applied on load: the lane's two 8-dim chunks are whole
// (even, odd) pairs, rotated with the same arithmetic as the RoPE kernels
// (rope_rotate8), so the fragments hold exactly the bits a rotated q tensor
// would hold.
// NARROW: chunks past cmask (a row of 16 or 32 dims, tables of that width)
// are zero.
template <bool NARROW>
__device__ __forceinline__ void load_q_rope(const uint16_t* qrow, const uint16_t* crow, const uint16_t* srow,
                                            bf16x8_t (&qf)[2], uint32_t cmask) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int dc = 0; dc < 2; ++dc) {
    if (NARROW && (uint32_t)(4 * dc + g) > cmask) {
      qf[dc] = bf16x8_t{};
      continue;
    }
    const int d0 = 32 * dc + 8 * g;
    float xv[8], cv[8], sv[8], o[8];
    load8<PFA_BF16>(qrow + d0, xv);
    load8<PFA_BF16>(crow + d0, cv);
    load8<PFA_BF16>(srow + d0, sv);
    rope_rotate8<PFA_BF16>(xv, cv, sv, o);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f32_to_bf16(o[2 * i]) | ((uint32_t)f32_to_bf16(o[2 * i + 1]) << 16);
    __builtin_memcpy(&qf[dc], w, 16);
  }
}

// NARROW: a row of 16 or 32 dims (a.cmask); otherwise 32 * NQ dims.  The
// RoPE tables on load are (T, D) for rows of at most 64 dims (NQ = 2,
// checked by the host).
template <int NQ, bool NARROW>
__device__ __forceinline__ void load_q_row(const ShortArgs& a, const uint16_t* qb, int64_t t, bf16x8_t (&qf)[NQ]) {
  if constexpr (NQ == 2) {
    if (a.rcos != nullptr) {
      const int64_t tw = NARROW ? (int64_t)a.dh : 64;  // table row width
      load_q_rope<NARROW>(qb + t * a.q.s_t, a.rcos + t * tw, a.rsin + t * tw, qf, NARROW ? a.cmask : 7u);
      return;
    }
  }
  load_q<NQ, NARROW>(qb + t * a.q.s_t, qf, NARROW ? a.cmask : 0u);
}

// dma_tile from wave-uniform K/V bases with 32-bit byte offsets per lane
// (the caller checks that every offset of the sequence fits in 32 bits):
// no 64-bit address arithmetic per tile.
// NH = 2: the second 64-dim half of each row (source + 128 bytes) fills
// the second K and V tiles of the stage (SwzTileH's layout).
template <int NH>
__device__ __forceinline__ void dma_tile32(const uint16_t* kb, const uint16_t* vb, uint32_t ks_t, uint32_t vs_t,
                                           int key0, int key1, uint32_t lds_w, uint32_t cmask) {
  const int tid = threadIdx.x;
  const uint32_t c = 2u * 8u * ((uint32_t)((tid & 7) ^ tile_swz(tid >> 3)) & cmask);
  const uint32_t k2 = 2u * ks_t, v2 = 2u * vs_t;
  constexpr uint32_t kT = 2 * kSwzTileElems;  // bytes of one 64 x 64 tile
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    lds_dma16_s(kb, (uint32_t)key0 * k2 + c + 128u * h, lds_w + kT * h);
    lds_dma16_s(kb, (uint32_t)key1 * k2 + c + 128u * h, lds_w + kT * h + 4096);
  }
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    lds_dma16_s(vb, (uint32_t)key0 * v2 + c + 128u * h, lds_w + kT * (NH + h));
    lds_dma16_s(vb, (uint32_t)key1 * v2 + c + 128u * h, lds_w + kT * (NH + h) + 4096);
  }
}
// dma_tile (64-bit addresses) for NH halves.
template <int NH>
__device__ __forceinline__ void dma_tile_h(const uint16_t* kb, const uint16_t* vb, uint32_t ks_t, uint32_t vs_t,
                                           int key0, int key1, uint32_t lds_w, uint32_t cmask) {
  constexpr uint32_t kT = 2 * kSwzTileElems;
  if constexpr (NH == 1) {
    dma_tile(kb, vb, ks_t, vs_t, key0, key1, lds_w, cmask);
  } else {
    const int tid = threadIdx.x;
    const int c = 8 * (int)((uint32_t)((tid & 7) ^ tile_swz(tid >> 3)) & cmask);
    const uint64_t k0 = (uint64_t)(uint32_t)key0 * ks_t, k1 = (uint64_t)(uint32_t)key1 * ks_t;
    const uint64_t v0 = (uint64_t)(uint32_t)key0 * vs_t, v1 = (uint64_t)(uint32_t)key1 * vs_t;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      lds_dma16(kb + c + 64 * h + k0, lds_w + kT * h);
      lds_dma16(kb + c + 64 * h + k1, lds_w + kT * h + 4096);
    }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      lds_dma16(vb + c + 64 * h + v0, lds_w + kT * (NH + h));
      lds_dma16(vb + c + 64 * h + v1, lds_w + kT * (NH + h) + 4096);
    }
  }
}

template <int NH>
__device__ __forceinline__ void init_state(QState<NH>& st) {
  st.m = -INFINITY;
  st.l = 0.f;
  st.cnt = 0;
#pragma unroll
  for (int db = 0; db < 4 * NH; ++db) st.acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ int64_t xcd_block(int64_t P, int64_t nblk) {
  int64_t per = nblk / 8;
  return (P % 8) * per + P / 8;
}

// The fused per-class work of the anchor pass, eight lanes per token (lane
// group j of a pass takes token c + s*(M0 + j), each lane one 16-byte chunk
// of the 64-element row, so a wave's accesses are whole 128-byte rows).
// ROPE: rotate the k row of the token in place (rope_rotate8 on the lane's
// four (even, odd) pairs: the bits of pfa_rope_k_inplace).  ZERO: write
// zeros to the out row of the token (a head without rows).  The loads of
// kFusedBatch passes are issued together before any of them is used (one
// memory latency per batch).
constexpr int kFusedBatch = 4;
__device__ __forceinline__ void unpack8(const uint4& w, float (&o)[8]) {
  const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(v[i] << 16);
    o[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

template <bool ROPE, bool ZERO>
__device__ __forceinline__ void class_rows_fused(const ShortArgs& a, int64_t bb, int64_t hh, int c, int64_t Mmax) {
  const int tid = threadIdx.x;
  const int ch = tid & 7;
  const int s = a.stride;
  uint16_t* kb = (uint16_t*)a.k.ptr + bb * a.k.s_b + hh * a.k.s_h + 8 * ch;
  uint16_t* ob = (uint16_t*)a.out.ptr + bb * a.out.s_b + hh * a.out.s_h + 8 * ch;
  for (int64_t M0 = 0; M0 <= Mmax; M0 += 32 * kFusedBatch) {
    uint4 kx[kFusedBatch], kc[kFusedBatch], ks[kFusedBatch];
    int64_t tt[kFusedBatch];
    bool ok[kFusedBatch];
#pragma unroll
    for (int j = 0; j < kFusedBatch; ++j) {
      const int64_t M = M0 + 32 * j + (tid >> 3);
      ok[j] = M <= Mmax;
      // past the class's last token the lane reloads token c (in range,
      // unused): the loads stay unconditional, so none waits on another
      tt[j] = c + (int64_t)s * (ok[j] ? M : 0);
      if constexpr (ROPE) {
        kx[j] = *reinterpret_cast<const uint4*>(kb + tt[j] * a.k.s_t);
        kc[j] = *reinterpret_cast<const uint4*>(a.rcos + tt[j] * 64 + 8 * ch);
        ks[j] = *reinterpret_cast<const uint4*>(a.rsin + tt[j] * 64 + 8 * ch);
      }
    }
#pragma unroll
    for (int j = 0; j < kFusedBatch; ++j) {
      if (!ok[j]) continue;
      if constexpr (ROPE) {
        float xv[8], cv[8], sv[8], o[8];
        unpack8(kx[j], xv);
        unpack8(kc[j], cv);
        unpack8(ks[j], sv);
        rope_rotate8<PFA_BF16>(xv, cv, sv, o);
        uint4 w;
        w.x = (uint32_t)f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
        w.y = (uint32_t)f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
        w.z = (uint32_t)f32_to_bf16(o[4]) | ((uint32_t)f32_to_bf16(o[5]) << 16);
        w.w = (uint32_t)f32_to_bf16(o[6]) | ((uint32_t)f32_to_bf16(o[7]) << 16);
        *reinterpret_cast<uint4*>(kb + tt[j] * a.k.s_t) = w;
      }
      if constexpr (ZERO) *reinterpret_cast<uint4*>(ob + tt[j] * a.out.s_t) = make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// ---------------------------------------------------------------------
// Pass 1: anchors per (residue class, compact head)
// ---------------------------------------------------------------------
// Occupancy: at most 168 VGPRs so that three 4-wave workgroups share a CU.
// The pass runs beside the prototype-table kernels on another stream; three
// workgroups (about 100 KB of LDS with a two-stage ring) leave LDS and wave
// slots for them.
constexpr int kAnchorStages = 2;
// Row groups per wave: NG = 2 (32 rows per wave, 128 per chunk) for long
// residue classes, whose chunks each stream long key bands: the tile
// transfers and barriers are then shared by twice the rows.
constexpr int kAnchorNG2Positions = 256;  // class positions from which NG = 2 is launched
// NARROW: rows of D = 16 or 32 elements (a.cmask); otherwise D = 64 * NH.
// cm masks the tile DMA's chunk within a 64-dim half.
template <int NG, bool NARROW, int NH>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NH == 1 ? 3 : 2, 8)))
short_anchor_kernel(ShortArgs a, int ccap) {
  const uint32_t cm = NARROW ? a.cmask : 7u;
  constexpr int PW = part_w(NH);
  constexpr int S = kAnchorStages;
  __shared__ __align__(16) uint16_t ring[S][2 * NH * kTileElems];
  // active rows of the class, compacted ccap at a time (a multiple of 256,
  // at most kClassChunk; dynamic LDS): row index and class position M
  extern __shared__ int32_t cls_dyn[];
  int32_t* cls_r = cls_dyn;
  int32_t* cls_m = cls_dyn + ccap;
  __shared__ int s_count;
  __shared__ int wave_cnt[4];

  const int c = blockIdx.x;
  const int p = blockIdx.y;
  const int P = a.summary[0];
  const int s = a.stride;
  if (c >= s || (int64_t)c >= a.T) return;
  const int64_t Mmax = (a.T - 1 - c) / s;
  if (p >= P) {
    // inactive heads: workgroup p takes the (p - P)-th global head missing
    // from the ascending active list head_map[0..P)
    if ((a.fuse & kFuseZero) == 0) return;
    int g = p - P;
    for (int j = 0; j < P; ++j) g += a.head_map[j] <= g ? 1 : 0;
    if (g >= (int)gridDim.y) return;
    class_rows_fused<false, true>(a, g / a.H, g % a.H, c, Mmax);
    return;
  }
  const int bh = a.head_map ? a.head_map[p] : p;
  const int64_t bb = bh / a.H, hh = bh % a.H;
  const float sl2 = a.head_scale_log2(bh);
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // The rotated k rows are read back below by this workgroup's own tile
  // transfers (the class's keys are this workgroup's alone): the barrier of
  // the row compaction (a workgroup-scope release/acquire, one CU and one
  // L1) orders every wave's stores before them.  A device-scope fence here
  // would write back the whole L2 from every wave.
  // (the zeros of kFuseZero are written by the row compaction below, which
  // reads every row_of entry of the class anyway)
  if (a.fuse & kFuseKRope) class_rows_fused<true, false>(a, bb, hh, c, Mmax);
  SwzLane L;
  L.init();
  const int drow = tid >> 3;  // this thread's DMA rows: drow and drow + 32
  const uint32_t ring_w = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]) + 1024u * (uint32_t)wid);
  constexpr uint32_t kStageBytes = 2 * NH * kTileElems * 2;

  const uint16_t* kb = (const uint16_t*)a.k.ptr + bb * a.k.s_b + hh * a.k.s_h;
  const uint16_t* vb = (const uint16_t*)a.v.ptr + bb * a.v.s_b + hh * a.v.s_h;
  const uint16_t* qb = (const uint16_t*)a.q.ptr + bb * a.q.s_b + hh * a.q.s_h;

  // The class's active rows in rounds: compact the rows of the next class
  // positions (ascending M) until the list holds ccap - 256 or more, then
  // attend them.  A row's keys depend on its own M only, so the rounds
  // compute what one list of every row would.
  int64_t scan = 0;  // the next class position to compact (uniform)
  for (;;) {
  if (tid == 0) s_count = 0;
  __syncthreads();
  for (; scan <= Mmax && s_count + 256 <= ccap; scan += 256) {
    const int64_t M = scan + tid;
    int r = -1;
    if (M <= Mmax) r = a.row_of[(int64_t)bh * a.T + c + (int64_t)s * M];
    const bool act = r >= 0;
    if ((a.fuse & kFuseZero) && M <= Mmax && !act) {
      // the token has no row of this head: its out row is zero (stores only,
      // nothing in this workgroup waits for them)
      uint4* orow = reinterpret_cast<uint4*>((uint16_t*)a.out.ptr + bb * a.out.s_b + hh * a.out.s_h +
                                             (c + (int64_t)s * M) * a.out.s_t);
#pragma unroll
      for (int j = 0; j < 8; ++j) orow[j] = make_uint4(0u, 0u, 0u, 0u);
    }
    const uint64_t bal = __ballot(act);
    if (lane == 0) wave_cnt[wid] = __popcll(bal);
    __syncthreads();
    int before = s_count;
    for (int w = 0; w < wid; ++w) before += wave_cnt[w];
    if (act) {
      const int pos = before + __popcll(bal & ((1ull << lane) - 1ull));
      cls_m[pos] = (int32_t)M;
      cls_r[pos] = r;
    }
    __syncthreads();
    if (tid == 0) s_count += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
  const int nrows = s_count;
  __syncthreads();  // every wave has read the count before the next round clears it

  // chunks of 64 * NG rows: wave w takes rows 16 * (NG * w + g) + r16 of
  // the chunk in its row groups g < NG, every group against the same tiles
  constexpr int kChunk = kRows * NG;
  for (int c0 = 0; c0 < nrows; c0 += kChunk) {
    bool qv[NG], wave_rows[NG], wave_full[NG];
    int Mq[NG], rq[NG], hi_q[NG], lo_q[NG], w_lolo[NG], w_lohi[NG], w_hilo[NG], w_hihi[NG];
    int64_t tq[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int base = 16 * (NG * wid + g);
      const int qs = base + (lane & 15);
      qv[g] = c0 + qs < nrows;
      Mq[g] = qv[g] ? cls_m[c0 + qs] : 0;
      rq[g] = qv[g] ? cls_r[c0 + qs] : 0;
      tq[g] = c + (int64_t)s * Mq[g];
      const int j0 = (int)((tq[g] - win_lo(tq[g], a.local_w)) / s) + 1;
      hi_q[g] = qv[g] ? Mq[g] - j0 : -1;
      lo_q[g] = Mq[g] - a.slots > 0 ? Mq[g] - a.slots : 0;
      // group rows ascending in M: lo_q and hi_q are non-decreasing
      const int fr = base, lr = min(nrows - c0, base + 16) - 1;
      wave_rows[g] = fr <= lr;
      wave_full[g] = lr == base + 15;
      w_lolo[g] = 0, w_lohi[g] = 0, w_hilo[g] = -1, w_hihi[g] = -1;
      if (wave_rows[g]) {
        const int Ma = cls_m[c0 + fr], Mb = cls_m[c0 + lr];
        const int64_t ta = c + (int64_t)s * Ma, tb = c + (int64_t)s * Mb;
        w_lolo[g] = Ma - a.slots > 0 ? Ma - a.slots : 0;
        w_lohi[g] = Mb - a.slots > 0 ? Mb - a.slots : 0;
        w_hilo[g] = Ma - ((int)((ta - win_lo(ta, a.local_w)) / s) + 1);
        w_hihi[g] = Mb - ((int)((tb - win_lo(tb, a.local_w)) / s) + 1);
      }
    }
    // key range of the chunk (lo/hi are non-decreasing in M)
    const int last = min(nrows, c0 + kChunk) - 1;
    const int64_t Mf = cls_m[c0], Ml = cls_m[last];
    const int64_t mlo = Mf - a.slots > 0 ? Mf - a.slots : 0;
    const int64_t tl = c + (int64_t)s * Ml;
    const int64_t mhi = Ml - ((tl - win_lo(tl, a.local_w)) / s + 1);
    // pipelined over the class's key tiles (strided keys c + s*m) through
    // the LDS ring; the first tile is requested before the q row's loads
    const int ntile = mhi >= mlo ? (int)((mhi - mlo) / kTile + 1) : 0;
    auto request = [&](int i) {
      const int m0 = (int)mlo + kTile * i;
      const int ka = c + s * min(m0 + drow, (int)mhi), kz = c + s * min(m0 + drow + 32, (int)mhi);
      if (a.off32)
        dma_tile32<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz,
                       ring_w + kStageBytes * (uint32_t)(i % S), cm);
      else
        dma_tile_h<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz,
                       ring_w + kStageBytes * (uint32_t)(i % S), cm);
    };
#pragma unroll
    for (int i = 0; i < S - 1; ++i)
      if (i < ntile) request(i);
    bf16x8_t qf[NG][2 * NH];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      load_q_row<2 * NH, NARROW>(a, qb, tq[g], qf[g]);
#pragma unroll
      for (int dc = 0; dc < 2 * NH; ++dc)
        asm volatile("" : "+v"(qf[g][dc]));  // no load left for the tile loop to wait on
    }
    QState<NH> st[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) init_state(st[g]);
    for (int i = 0; i < ntile; ++i) {
      if (S == 3 && i + 1 < ntile)
        dma_wait_barrier<kDmaPerTile * NH>();
      else
        dma_wait_barrier<0>();
      if (i + S - 1 < ntile) request(i + S - 1);
      const int m0 = (int)mlo + kTile * i;
      const SwzTileH<NH> tl{ring[i % S], L};
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const bool empty = !wave_rows[g] || m0 > w_hihi[g] || m0 + kTile - 1 < w_lolo[g];
        if (!empty) {
          // the row's keys m in [lo_q, min(hi_q, mhi)], tile-local
          const bool need_lo = !wave_full[g] || m0 < w_lohi[g];
          const bool need_hi = !wave_full[g] || m0 + kTile - 1 > min(w_hilo[g], (int)mhi);
          const int lo = qv[g] ? lo_q[g] - m0 : kTile;
          const int hi = min(hi_q[g], (int)mhi) - m0;
          float sc[4][4];
          int unused = 0;
          window_qk<false>(qf[g], tl, need_lo, need_hi, lo, hi, unused, sc);
          softmax_pv(sc, tl, sl2, st[g]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float lt = st[g].l;
      lt += __shfl_xor(lt, 16, 64);
      lt += __shfl_xor(lt, 32, 64);
      if (qv[g]) {
        float* pr = a.part + (int64_t)rq[g] * PW;
        const int gq = lane >> 4;
        if (gq == 0) { pr[0] = st[g].m; pr[1] = lt; }
#pragma unroll
        for (int db = 0; db < 4 * NH; ++db)
          *reinterpret_cast<f32x4_t*>(pr + 4 + 16 * db + 4 * gq) = st[g].acc[db];
      }
    }
    // every wave is done with the ring before the next chunk's requests
    __syncthreads();
  }
  if (scan > Mmax) break;
  }
}

// ---------------------------------------------------------------------
// Pass 2: window + prototype keys per segment of consecutive rows
// ---------------------------------------------------------------------
// Key tiles reach LDS by DMA into a ring of S stages: tile i + S - 1 is
// requested when tile i starts, so S - 1 tiles are in flight while one is
// computed, and no registers hold tiles in transit.
// Occupancy: S = 2 stages (32 KB) allow four workgroups per CU and 128
// VGPRs; S = 3 (48 KB) three workgroups and 168 VGPRs.  Measured at
// config 3, four workgroups of two stages beat three of three: the pass is
// bound by instruction latency more than by the tile transfers.  Two stages
// at three waves per SIMD (161 VGPRs, no spills; four waves spill 44-56
// bytes per lane) were slower too, at configs 3 and 4 (the spill traffic
// costs less than the fourth wave gains).
#ifndef PFA_MAIN_STAGES
#define PFA_MAIN_STAGES 2
#endif
constexpr int kMainStages = PFA_MAIN_STAGES;
template <int S>
struct MainOcc;
template <>
struct MainOcc<2> {
  static constexpr int kWaves = 4;
};
template <>
struct MainOcc<3> {
  static constexpr int kWaves = 3;
};

// NARROW: rows of D = 16 or 32 elements; otherwise D = 64 * NH (cm as in
// the anchor pass).
template <bool COUNT, int S, bool NARROW, int NH>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NH == 1 ? MainOcc<S>::kWaves : 2, 8)))
short_main_kernel(ShortArgs a, int use_part, int pcap) {
  const uint32_t cm = NARROW ? a.cmask : 7u;
  constexpr int PW = part_w(NH);
  constexpr int kSlots = 16;  // tile slots of the shared window-tile schedule
  __shared__ __align__(16) uint16_t ring[S][2 * NH * kTileElems];
  __shared__ int32_t r_t[kRows];
  __shared__ int32_t r_p[kRows];
  __shared__ int32_t seg_begin[kRows + 1];
  __shared__ int s_nseg;
  __shared__ int s_cnt[2][4];
  __shared__ int s_pe0;
  // prototype key list of the current segment: position, evict, position mod
  // stride (-1 without anchors); pcap is a multiple of the tile size
  extern __shared__ __align__(16) int32_t pdyn[];
  int32_t* pk = pdyn;
  int32_t* pe = pk + pcap;
  int32_t* pm = pe + pcap;
  int32_t* ord = pm + pcap;  // tile order of the segment (ordcap entries)

  const int64_t lb = xcd_block(blockIdx.x, gridDim.x);
  const int64_t r0 = lb * kRows;
  if (r0 >= a.N) return;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int w = a.local_w;
  const int sa = a.stride, sl = a.slots;
  SwzLane L;
  L.init();
  // segments, found by the first wave: rows are ordered by (head, token)
  // with absent rows last, so "row j ends the segment begun at row i"
  // (absent, another head, or t_j - t_i >= w) is monotone in j > i; each
  // lane binary-searches its successor and lane 0 follows the chain from
  // row 0.
  if (wid == 0) {
    const int64_t r = r0 + lane;
    const int t = r < a.N ? a.token_idx[r] : -1;
    const int pp = r < a.N ? a.row_head[r] : -1;
    r_t[lane] = t;
    r_p[lane] = pp;
    int lo = lane + 1, hi = kRows;
#pragma unroll
    for (int step = 0; step < 6; ++step) {
      const int mid = (lo + hi) >> 1;
      const int tj = __shfl(t, mid & 63, 64), pj = __shfl(pp, mid & 63, 64);
      const bool ends = mid >= kRows || tj < 0 || pj != pp || tj - t >= w;
      if (lo < hi) {
        if (ends) hi = mid;
        else lo = mid + 1;
      }
    }
    int n = 0, i = 0;
    while (i < kRows && __shfl(t, i, 64) >= 0) {
      if (lane == 0) seg_begin[n] = i;
      ++n;
      i = __shfl(lo, i, 64);
    }
    if (lane == 0) {
      seg_begin[n] = i;
      s_nseg = n;
      s_pe0 = -1;
    }
  }
  __syncthreads();
  const int nseg = s_nseg;
  const int qs = 16 * wid + (lane & 15);
  const int g = lane >> 4;
  const int drow = tid >> 3;  // this thread's DMA rows: drow and drow + 32
  // LDS byte address of stage 0 plus this wave's 1 KB run (wave-uniform)
  const uint32_t ring_w = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]) + 1024u * (uint32_t)wid);
  constexpr uint32_t kStageBytes = 2 * NH * kTileElems * 2;

  for (int sg = 0; sg < nseg; ++sg) {
    const int s0 = seg_begin[sg], s1 = seg_begin[sg + 1];
    const int p = r_p[s0];
    const int bh = a.head_map ? a.head_map[p] : p;
    const int64_t bb = bh / a.H, hh = bh % a.H;
    const float sl2 = a.head_scale_log2(bh);
    const int t_first = r_t[s0], t_last = r_t[s1 - 1];
    const int lo_first = (int)win_lo(t_first, w), lo_last = (int)win_lo(t_last, w);
    const uint16_t* kb = (const uint16_t*)a.k.ptr + bb * a.k.s_b + hh * a.k.s_h;
    const uint16_t* vb = (const uint16_t*)a.v.ptr + bb * a.v.s_b + hh * a.v.s_h;
    const uint16_t* qb = (const uint16_t*)a.q.ptr + bb * a.q.s_b + hh * a.q.s_h;
    // Window tiles lie on the global 64-key grid (tile k: keys 64k .. 64k+63,
    // the keys outside [lo_first, t_last] masked).  Every workgroup takes
    // window tile k in slot k mod kSlots of its tile sequence and fills the
    // free slots with its prototype tiles: neighbouring workgroups of one
    // head share most of their window tiles, and taking a shared tile in the
    // same slot, at about the same time, the later requests find it in L2.
    const int wA = lo_first >> 6, wB = t_last >> 6;
    const int nw = wB - wA + 1;
    // the tile of slot 0, requested now (its transfer overlaps the prototype
    // list) when it is a window tile
    const int k_slot0 = wA + ((0 - wA) & (kSlots - 1));
    const bool early = k_slot0 <= wB;
    if (early)
    {
      const int ka = min(kTile * k_slot0 + drow, t_last), kz = min(kTile * k_slot0 + drow + 32, t_last);
      if (a.off32)
        dma_tile32<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz, ring_w, cm);
      else
        dma_tile_h<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz, ring_w, cm);
    }
    const bool qv = qs >= s0 && qs < s1;
    const int tq = qv ? r_t[qs] : t_first;

    // prototype key list: the prefix set of t_first below lo_last (set table
    // row of t_first's block -- any order, INT32_MAX-padded -- then the
    // block's tokens up to t_first, keeping p with evict[p] > t_first).
    // Each thread takes two candidates per pass (their set-table and evict
    // loads are one round each); kept keys are compacted in a fixed order
    // (candidate half, then wave, then lane) from per-wave counts, so the
    // list, and the summation order, is the same on every run.  Slot 0 is
    // kept for key 0 (the zero-anchor rule may need it whether or not it is
    // in the set; pe = -1 when it is not), so the mask tests the
    // zero-anchor rule on that one slot only.
    const bool anch_on = sa > 0 && sl > 0;
    const bool rsv = a.blk != nullptr || (lo_last > 0 && anch_on);
    int plen = rsv ? 1 : 0;
    if (a.blk != nullptr) {
      const int64_t jb = t_first >> 6;
      const int32_t* P = a.blk + (bb * a.nblk + jb) * a.K;
      const int32_t* ev = a.evict + bb * a.T;
      const int ncand = a.K + 64;
      const uint64_t below = (1ull << lane) - 1ull;
      for (int base = 0; base < ncand; base += 512) {
        int32_t v[2], evv[2];
        bool keep[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int e = base + 256 * h + tid;
          v[h] = INT32_MAX;
          if (e < a.K) {
            v[h] = P[e];
          } else if (e < ncand) {
            const int q = (int)(jb << 6) + (e - a.K);
            if (q <= t_first) v[h] = q;
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) evv[h] = v[h] < lo_last ? ev[v[h]] : 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          keep[h] = v[h] < lo_last && evv[h] > t_first;
          if (keep[h] && v[h] == 0) {
            s_pe0 = evv[h];  // key 0 is in the set: its slot carries the evict
            keep[h] = false;
          }
        }
        const uint64_t b0 = __ballot(keep[0]), b1 = __ballot(keep[1]);
        if (lane == 0) {
          s_cnt[0][wid] = __popcll(b0);
          s_cnt[1][wid] = __popcll(b1);
        }
        __syncthreads();
        int off[2] = {plen, plen};
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          off[0] += w2 < wid ? s_cnt[0][w2] : 0;
          off[1] += s_cnt[0][w2] + (w2 < wid ? s_cnt[1][w2] : 0);
          plen += s_cnt[0][w2] + s_cnt[1][w2];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (keep[h]) {
            const int pos = off[h] + __popcll((h ? b1 : b0) & below);
            pk[pos] = v[h];
            pe[pos] = evv[h];
            pm[pos] = anch_on ? v[h] % sa : -1;
          }
        if (tid == 0 && rsv && base + 512 >= ncand) {
          pk[0] = 0;
          pe[0] = s_pe0;
          pm[0] = anch_on ? 0 : -1;
          s_pe0 = -1;
        }
        __syncthreads();
      }
    } else if (rsv) {
      if (tid == 0) {
        pk[0] = 0;
        pe[0] = -1;
        pm[0] = anch_on ? 0 : -1;
      }
      __syncthreads();
    }
    // pad the last prototype tile: pk = INT32_MAX fails every row's test
    // (the tile loop's first barrier orders these writes before any read)
    {
      const int pend = (plen + kTile - 1) / kTile * kTile;
      if (plen + tid < pend) pk[plen + tid] = INT32_MAX;
    }

    // this lane's query row
    const int loq = (int)win_lo(tq, w);
    // prototype test of key p for this row (t = tq): p < win_lo(t), i.e.
    // p <= t - w; evict[p] > t; not a strided anchor of t (p = t mod s and
    // p >= t - s*slots); or key 0 under the zero-anchor rule (slot 0)
    const int p_tw = qv ? tq - w : -1 - w;  // a row that is not there takes no key
    const int p_tmod = sa > 0 ? tq % sa : 0;
    const int p_ts = anch_on ? (int)max((int64_t)tq - (int64_t)sa * sl, (int64_t)INT32_MIN + 1) : INT32_MAX;
    const bool p_zero = qv && zero_anchor(tq, sa, sl);
    // one pipelined pass over the tiles in slot order: ord[i] >= 0 is window
    // tile ord[i], ord[i] < 0 prototype tile -1 - ord[i]
    const int np = (plen + kTile - 1) / kTile;
    const int ntile = nw + np;
    // built by the first wave, one lane per slot: slot i takes window tiles
    // k = i (mod kSlots) in [wA, wB], or else, if it has none, the next
    // prototype tile; prototype tiles left over go last
    if (wid == 0) {
      const int sl_i = lane & (kSlots - 1);
      const int k0 = wA + ((sl_i - wA) & (kSlots - 1));
      const bool win = k0 <= wB;
      const uint64_t empty = __ballot(lane < kSlots && !win);
      const int e = __popcll(empty & ((1ull << lane) - 1ull));  // empty slots before this one
      const int cnt = lane < kSlots ? (win ? (wB - k0) / kSlots + 1 : (e < np ? 1 : 0)) : 0;
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < kSlots; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      const int pos = incl - cnt;
      if (lane < kSlots) {
        if (win)
          for (int j = 0; j < cnt; ++j) ord[pos + j] = k0 + kSlots * j;
        else if (cnt)
          ord[pos] = -1 - e;
      }
      const int n_empty = __popcll(empty);
      const int placed = __shfl(incl, kSlots - 1, 64);
      for (int j = n_empty + lane; j < np; j += 64) ord[placed + (j - n_empty)] = -1 - j;
    }
    __syncthreads();
    auto key_of = [&](int i, int r) -> int {
      const int d = ord[i];
      if (d >= 0) return min(kTile * d + r, t_last);
      return pk[min((-1 - d) * kTile + r, plen - 1)];
    };
    auto request = [&](int i) {
      const int ka = key_of(i, drow), kz = key_of(i, drow + 32);
      if (a.off32)
        dma_tile32<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz,
                       ring_w + kStageBytes * (uint32_t)(i % S), cm);
      else
        dma_tile_h<NH>(kb, vb, (uint32_t)a.k.s_t, (uint32_t)a.v.s_t, ka, kz,
                       ring_w + kStageBytes * (uint32_t)(i % S), cm);
    };
    if (!early) request(0);
#pragma unroll
    for (int i = 1; i < S - 1; ++i)
      if (i < ntile) request(i);
    bf16x8_t qf[2 * NH];
    load_q_row<2 * NH, NARROW>(a, qb, tq, qf);
    // settle the q fragments here: the tile loop then holds no load the
    // compiler would wait for (its wait would also drain the tile requests)
#pragma unroll
    for (int dc = 0; dc < 2 * NH; ++dc) asm volatile("" : "+v"(qf[dc]));
    QState<NH> st;
    init_state(st);

    // the rows of this wave are ascending in token: their key ranges lie in
    // [win_lo(first), last] and all contain [win_lo(last), first]
    const int fr = max(s0, 16 * wid), lr = min(s1, 16 * wid + 16) - 1;
    const bool wave_rows = fr <= lr;
    const bool wave_full = fr == 16 * wid && lr == 16 * wid + 15;
    const int w_tlo = wave_rows ? r_t[fr] : 0, w_thi = wave_rows ? r_t[lr] : -1;
    const int w_llo = (int)win_lo(w_tlo, w), w_lhi = (int)win_lo(w_thi < 0 ? 0 : w_thi, w);

    for (int i = 0; i < ntile; ++i) {
      // tile i has landed (tiles i+1 .. i+S-2 may still be in flight) and
      // every wave is done with tile i-1, whose stage takes tile i+S-1
      if (S == 3 && i + 1 < ntile)
        dma_wait_barrier<kDmaPerTile * NH>();
      else
        dma_wait_barrier<0>();
      if (i + S - 1 < ntile) request(i + S - 1);
      const SwzTileH<NH> tl{ring[i % S], L};
      const int d = ord[i];
      const bool is_win = d >= 0;
      const int k0 = kTile * d;
      const bool active = is_win ? (wave_rows && k0 <= w_thi && k0 + kTile - 1 >= w_llo) : wave_rows;
      if (active) {
        float sc[4][4];
        f32x4_t bias[4];
        bool plain = false;
        if (is_win) {
          // the row's window keys in the tile: [loq - k0, tq - k0]; which
          // bounds cut the tile is wave-uniform
          const bool need_lo = __builtin_amdgcn_readfirstlane((!wave_full || k0 < w_lhi) ? 1 : 0) != 0;
          const bool need_hi = __builtin_amdgcn_readfirstlane((!wave_full || k0 + kTile - 1 > w_tlo) ? 1 : 0) != 0;
          const int lo4 = (qv ? loq - k0 : kTile) - 4 * g, hi4 = tq - k0 - 4 * g;
          if (need_lo && need_hi) bias_range<true, true>(bias, lo4, hi4);
          else if (need_lo) bias_range<true, false>(bias, lo4, 0);
          else if (need_hi) bias_range<false, true>(bias, 0, hi4);
          else plain = true;
        } else {
          // the prototype test of each key (bitwise, no short-circuit
          // branches around the LDS reads)
          const int j0 = (-1 - d) * kTile + 4 * g;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const int4 kp = *reinterpret_cast<const int4*>(pk + j0 + 16 * kb);
            const int4 ke = *reinterpret_cast<const int4*>(pe + j0 + 16 * kb);
            const int4 km = *reinterpret_cast<const int4*>(pm + j0 + 16 * kb);
            const int kpv[4] = {kp.x, kp.y, kp.z, kp.w}, kev[4] = {ke.x, ke.y, ke.z, ke.w},
                      kmv[4] = {km.x, km.y, km.z, km.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              bool ok = (kpv[e] <= p_tw) & (kev[e] > tq) & !((kmv[e] == p_tmod) & (kpv[e] >= p_ts));
              if (kb == 0 && e == 0) ok = ok | (p_zero & (j0 == 0) & (p_tw >= 0));
              bias[kb][e] = ok ? 0.f : -INFINITY;
            }
          }
        }
        if (plain) {
          qk_tile(qf, tl, sc);
          if constexpr (COUNT) st.cnt += 16;
        } else {
          qk_tile_b(qf, tl, bias, sc);
          if constexpr (COUNT) st.cnt += count_finite(sc);
        }
        softmax_pv(sc, tl, sl2, st);
      }
    }

    // merge the anchor partial, normalise, write
    float lt = st.l;
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    int ct = COUNT ? st.cnt : 0;
    if constexpr (COUNT) {
      ct += __shfl_xor(ct, 16, 64);
      ct += __shfl_xor(ct, 32, 64);
    }
    if (qv) {
      const int64_t r = r0 + qs;
      float m = st.m;
      float fa = 1.f, fb = 0.f, lp = 0.f;
      f32x4_t pacc[4 * NH];
#pragma unroll
      for (int db = 0; db < 4 * NH; ++db) pacc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (use_part) {
        const float* pr = a.part + r * PW;
        const float ma = pr[0];
        lp = pr[1];
#pragma unroll
        for (int db = 0; db < 4 * NH; ++db) pacc[db] = *reinterpret_cast<const f32x4_t*>(pr + 4 + 16 * db + 4 * g);
        const float mm = fmaxf(m, ma);
        fa = (m == -INFINITY) ? 0.f : exp2f(m - mm);
        fb = (ma == -INFINITY) ? 0.f : exp2f(ma - mm);
      }
      const float den = lt * fa + lp * fb;
      const float inv = a.head_out_scale(bh) / den;
      uint16_t* op = (uint16_t*)a.out.ptr + bb * a.out.s_b + hh * a.out.s_h + (int64_t)tq * a.out.s_t;
#pragma unroll
      for (int db = 0; db < 4 * NH; ++db) {
        if (NARROW && 16 * db + 4 * g >= a.dh) break;  // dims past D
        uint16_t o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = f32_to_bf16((st.acc[db][i] * fa + pacc[db][i] * fb) * inv);
        *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) =
            make_uint2((uint32_t)o4[0] | ((uint32_t)o4[1] << 16), (uint32_t)o4[2] | ((uint32_t)o4[3] << 16));
      }
      if (COUNT && g == 0) {
        int64_t na = 0;
        if (a.stride > 0 && a.slots > 0) {
          const int64_t M = tq / a.stride;
          const int64_t j0 = (tq - loq) / a.stride + 1;
          const int64_t hi = M - j0, lo = M - a.slots > 0 ? M - a.slots : 0;
          na = hi >= lo ? hi - lo + 1 : 0;
        }
        a.lengths[r] = (int32_t)(ct + na);
      }
    }
    __syncthreads();
  }
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_shortlist_attn_part_floats(void) { return kPartW; }
extern "C" int pfa_shortlist_attn_part_floats_for(int head_dim) { return part_w(head_dim > 64 ? 2 : 1); }

static int shortlist_attn_run(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v, pfa_tensor4 out, int dtype, int H,
                              int64_t T, int D, const int32_t* token_idx, const int32_t* row_head,
                              const int32_t* head_map, int64_t N, int P_cap, const int32_t* summary,
                              const int32_t* row_of, int local_w, int anchor_stride, int anchor_slots,
                              const int32_t* proto_blocks, int proto_k, const int32_t* proto_evict, float scale,
                              float* partials, int32_t* lengths, const void* q_rope_cos, const void* q_rope_sin,
                              const float* q_scale, const float* k_scale, const float* v_scale, int passes,
                              int fuse, void* stream) {
  PFA_CHECK_ARG(dtype == PFA_BF16 && (D == 16 || D == 32 || D == 64 || D == 128),
                "pfa_shortlist_attn_fwd: bf16 with D = 16, 32, 64 or 128 only (got dtype %d D %d)", dtype, D);
  // q RoPE on load takes rows of at most 64 dims, the anchor-pass fusions 64
  PFA_CHECK_ARG((D <= 64 || q_rope_cos == nullptr) && (D == 64 || fuse == 0),
                "pfa_shortlist_attn_fwd: q RoPE on load needs D <= 64 and the anchor-pass fusions D = 64 (got D %d)",
                D);
  PFA_CHECK_ARG(H > 0 && T > 0 && T < INT32_MAX && N >= 0 && P_cap > 0 && local_w >= 1,
                "pfa_shortlist_attn_fwd: bad sizes");
  PFA_CHECK_ARG(passes >= 1 && passes <= 3, "pfa_shortlist_attn_fwd: passes must be 1, 2 or 3 (got %d)", passes);
  PFA_CHECK_ARG((fuse & ~(kFuseKRope | kFuseZero)) == 0, "pfa_shortlist_attn_fwd_fused: unknown fuse bits %d", fuse);
  if (fuse != 0) {
    // the fused work rides on the anchor pass: it must run in this call,
    // even when there are no rows (the zero fill still applies)
    PFA_CHECK_ARG(anchor_stride > 0 && anchor_slots > 0 && (passes & 1),
                  "pfa_shortlist_attn_fwd_fused: fusions need the anchor pass (anchors on, passes 1 or 3)");
    PFA_CHECK_ARG(head_map && summary && row_of && out.ptr && k.ptr,
                  "pfa_shortlist_attn_fwd_fused: head_map, summary, row_of, k and out are required");
    PFA_CHECK_ARG(P_cap % H == 0, "pfa_shortlist_attn_fwd_fused: P_cap (%d) must be B*H (a multiple of H=%d)", P_cap,
                  H);
    PFA_CHECK_ARG(!(fuse & kFuseKRope) || (q_rope_cos && q_rope_sin && !q_scale),
                  "pfa_shortlist_attn_fwd_fused: the k rotation needs the RoPE tables and no int8 scales");
  }
  if (N == 0 && fuse == 0) return PFA_OK;
  PFA_CHECK_ARG(q.ptr && k.ptr && v.ptr && out.ptr && (N == 0 || (token_idx && row_head)) && summary,
                "pfa_shortlist_attn_fwd: null pointer");
  PFA_CHECK_ARG(proto_blocks == nullptr || (proto_k > 0 && proto_k <= kMaxProto && proto_evict),
                "pfa_shortlist_attn_fwd: prototype table (K <= %d with evict) required", kMaxProto);
  const bool anchors = anchor_stride > 0 && anchor_slots > 0;
  PFA_CHECK_ARG(!anchors || (row_of && partials), "pfa_shortlist_attn_fwd: anchors need row_of and partials");
  auto al = [](const pfa_tensor4& x) {
    return ((uintptr_t)x.ptr % 16) == 0 && x.s_b % 8 == 0 && x.s_h % 8 == 0 && x.s_t % 8 == 0;
  };
  PFA_CHECK_ARG(al(q) && al(k) && al(v) && al(out), "pfa_shortlist_attn_fwd: tensors must be 16-byte aligned");
  PFA_CHECK_ARG(k.s_t > 0 && v.s_t > 0 && k.s_t < INT32_MAX && v.s_t < INT32_MAX,
                "pfa_shortlist_attn_fwd: k/v token strides must be positive and below 2^31");
  PFA_CHECK_ARG((q_rope_cos == nullptr) == (q_rope_sin == nullptr),
                "pfa_shortlist_attn_fwd: q_rope_cos and q_rope_sin go together");
  PFA_CHECK_ARG(q_rope_cos == nullptr || (((uintptr_t)q_rope_cos | (uintptr_t)q_rope_sin) & 15) == 0,
                "pfa_shortlist_attn_fwd: RoPE tables must be 16-byte aligned");
  PFA_CHECK_ARG((q_scale == nullptr) == (k_scale == nullptr) && (q_scale == nullptr) == (v_scale == nullptr),
                "pfa_shortlist_attn_fwd: q_scale, k_scale and v_scale go together");
  ShortArgs a;
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.H = H; a.T = T; a.token_idx = token_idx; a.row_head = row_head; a.head_map = head_map; a.N = N;
  a.local_w = local_w; a.stride = anchor_stride; a.slots = anchor_slots;
  a.blk = proto_blocks; a.K = proto_k; a.nblk = (T + 63) / 64; a.evict = proto_evict;
  a.row_of = row_of; a.summary = summary; a.part = partials; a.lengths = lengths;
  a.rcos = (const uint16_t*)q_rope_cos; a.rsin = (const uint16_t*)q_rope_sin;
  a.scale_log2 = scale * 1.4426950408889634f;
  {
    // byte offsets key * s_t * 2 + 240 of every key below T, K and V (the
    // last chunk of a 128-dim row)
    const uint64_t mx = (uint64_t)(T - 1) * (uint64_t)(k.s_t > v.s_t ? k.s_t : v.s_t) * 2u + 256u;
    a.off32 = mx < 0xFFFFFFFFull ? 1 : 0;
  }
  a.qsc = q_scale; a.ksc = k_scale; a.vsc = v_scale;
  a.fuse = fuse;
  a.dh = D;
  a.cmask = (uint32_t)(D / 8 - 1);
  hipStream_t s = as_stream(stream);
  if (anchors && (passes & 1)) {
    dim3 grid((unsigned)((int64_t)anchor_stride < T ? (int64_t)anchor_stride : T), (unsigned)P_cap);
    // class positions rounded up to the 256 of one compaction step, at most
    // kClassChunk (longer classes are attended in rounds)
    const int64_t npos = ((T - 1) / anchor_stride + 1 + 255) / 256 * 256;
    const int ccap = (int)(npos < kClassChunk ? npos : kClassChunk);
    const size_t lds = (size_t)ccap * 8 + 16;
    const bool ng2 = npos >= kAnchorNG2Positions;
    if (D == 128) {
      // one row group per wave: two groups of 128-dim rows exceed the registers
      short_anchor_kernel<1, false, 2><<<grid, 256, lds, s>>>(a, ccap);
    } else if (D == 64) {
      if (ng2) short_anchor_kernel<2, false, 1><<<grid, 256, lds, s>>>(a, ccap);
      else short_anchor_kernel<1, false, 1><<<grid, 256, lds, s>>>(a, ccap);
    } else {
      if (ng2) short_anchor_kernel<2, true, 1><<<grid, 256, lds, s>>>(a, ccap);
      else short_anchor_kernel<1, true, 1><<<grid, 256, lds, s>>>(a, ccap);
    }
    PFA_CHECK_LAUNCH("pfa_shortlist_attn_fwd/anchors");
  }
  if (!(passes & 2) || N == 0) return PFA_OK;
  // prototype slots: key 0's slot, the set table row, the block's 64 tokens;
  // rounded up to whole tiles
  const int pcap = ((proto_blocks ? proto_k : 0) + 64 + 1 + kTile - 1) / kTile * kTile;
  int64_t blocks = (N + kRows - 1) / kRows;
  blocks = (blocks + 7) / 8 * 8;
  PFA_CHECK_ARG(blocks < INT32_MAX, "pfa_shortlist_attn_fwd: too many rows");
  constexpr int S = kMainStages;
  // tile order: the window tiles of a segment (its rows span less than w)
  // plus the prototype tiles
  // (a segment's window tiles lie in [0, T): at most T/64 + 1 of them)
  const int64_t wspan = (int64_t)2 * local_w < T ? (int64_t)2 * local_w : T;
  const int ordcap = (int)((wspan + kTile - 1) / kTile) + 2 + pcap / kTile;
  const size_t dyn = (size_t)pcap * 12 + (size_t)ordcap * 4;
  const int up = anchors ? 1 : 0;
  if (D == 128) {
    if (lengths != nullptr) short_main_kernel<true, S, false, 2><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
    else short_main_kernel<false, S, false, 2><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
  } else if (D == 64) {
    if (lengths != nullptr) short_main_kernel<true, S, false, 1><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
    else short_main_kernel<false, S, false, 1><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
  } else {
    if (lengths != nullptr) short_main_kernel<true, S, true, 1><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
    else short_main_kernel<false, S, true, 1><<<(unsigned)blocks, 256, dyn, s>>>(a, up, pcap);
  }
  PFA_CHECK_LAUNCH("pfa_shortlist_attn_fwd/main");
  return PFA_OK;
}

extern "C" int pfa_shortlist_attn_fwd(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v, pfa_tensor4 out, int dtype, int H,
                                      int64_t T, int D, const int32_t* token_idx, const int32_t* row_head,
                                      const int32_t* head_map, int64_t N, int P_cap, const int32_t* summary,
                                      const int32_t* row_of, int local_w, int anchor_stride, int anchor_slots,
                                      const int32_t* proto_blocks, int proto_k, const int32_t* proto_evict,
                                      float scale, float* partials, int32_t* lengths, const void* q_rope_cos,
                                      const void* q_rope_sin, const float* q_scale, const float* k_scale,
                                      const float* v_scale, int passes, void* stream) {
  clear_error();
  return shortlist_attn_run(q, k, v, out, dtype, H, T, D, token_idx, row_head, head_map, N, P_cap, summary, row_of,
                            local_w, anchor_stride, anchor_slots, proto_blocks, proto_k, proto_evict, scale, partials,
                            lengths, q_rope_cos, q_rope_sin, q_scale, k_scale, v_scale, passes, 0, stream);
}

extern "C" int pfa_shortlist_attn_fwd_fused(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v, pfa_tensor4 out, int dtype,
                                            int H, int64_t T, int D, const int32_t* token_idx,
                                            const int32_t* row_head, const int32_t* head_map, int64_t N, int P_cap,
                                            const int32_t* summary, const int32_t* row_of, int local_w,
                                            int anchor_stride, int anchor_slots, const int32_t* proto_blocks,
                                            int proto_k, const int32_t* proto_evict, float scale, float* partials,
                                            int32_t* lengths, const void* q_rope_cos, const void* q_rope_sin,
                                            int passes, int fuse, void* stream) {
  clear_error();
  return shortlist_attn_run(q, k, v, out, dtype, H, T, D, token_idx, row_head, head_map, N, P_cap, summary, row_of,
                            local_w, anchor_stride, anchor_slots, proto_blocks, proto_k, proto_evict, scale, partials,
                            lengths, q_rope_cos, q_rope_sin, nullptr, nullptr, nullptr, passes, fuse, stream);
}
