// Router: per-token gate probabilities, prototype prior, importance and
// head top-k; the prototype EMA statistics and update.
//
// Mapping: one lane per token, one wave per workgroup (see router_kernel).
//
// Arithmetic follows the reference op by op (aspa.py:135-157, 628-690,
// 1521-1530, 1540-1542): logits are rounded to the input dtype, the router
// softmax is evaluated in f32 and rounded to the input dtype, everything
// after that is f32.  Floating-point contraction is disabled for the
// elementwise epilogue so that each product and sum rounds as the
// reference's separate tensor ops do; dot products use explicit fma.
#include "pfa_common.h"

#pragma clang fp contract(off)

namespace pfa {

constexpr int kRouterTok = 64;  // tokens per workgroup (one per lane)

// Two channels of one token as floats (one 4-byte load when aligned).
template <int DT>
__device__ __forceinline__ void load2(const typename Elem<DT>::T* p, bool two, float& a, float& b) {
  if constexpr (DT == PFA_F32) {
    a = p[0];
    b = two ? p[1] : 0.f;
  } else {
    if (two && (((uintptr_t)p & 3) == 0)) {
      uint32_t w = *reinterpret_cast<const uint32_t*>(p);
      if constexpr (DT == PFA_BF16) { a = __uint_as_float(w << 16); b = __uint_as_float(w & 0xffff0000u); }
      else { a = f16_to_f32((uint16_t)(w & 0xffffu)); b = f16_to_f32((uint16_t)(w >> 16)); }
    } else {
      a = load_f<DT>(p);
      b = two ? load_f<DT>(p + 1) : 0.f;
    }
  }
}

// Prototype EMA statistics of one router workgroup, fused into the router
// pass: gl holds the final gate probabilities of the workgroup's 64 tokens
// (zero for tokens past the end); each lane sums gate[t, g] * x[t, c] over
// the tokens, in token order, for a pair of channels c of this wave's range.
// The x rows were just streamed by the same workgroup, so they come from L2.
template <int DT, int GP>
__device__ __forceinline__ void router_ema_accum(const typename Elem<DT>::T* __restrict__ x, int64_t tok0,
                                                 int64_t n_tok, int C, int G, int cbeg, int cw,
                                                 const float* gl, float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int nt = (int)min<int64_t>(64, n_tok - tok0);
  const typename Elem<DT>::T* xb = x + tok0 * C;
  for (int c0 = cbeg + 2 * lane; c0 < cbeg + cw; c0 += 128) {
    const bool two = c0 + 1 < cbeg + cw;
    float a0[GP], a1[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) { a0[g] = 0.f; a1[g] = 0.f; }
    int u = 0;
    for (; u + 8 <= nt; u += 8) {
      float x0[8], x1[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) load2<DT>(xb + (int64_t)(u + k) * C + c0, two, x0[k], x1[k]);
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          const float pr = gl[(u + k) * GP + g];
          a0[g] = __builtin_fmaf(pr, x0[k], a0[g]);
          a1[g] = __builtin_fmaf(pr, x1[k], a1[g]);
        }
    }
    for (; u < nt; ++u) {
      float x0, x1;
      load2<DT>(xb + (int64_t)u * C + c0, two, x0, x1);
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const float pr = gl[u * GP + g];
        a0[g] = __builtin_fmaf(pr, x0, a0[g]);
        a1[g] = __builtin_fmaf(pr, x1, a1[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) {
        part[(int64_t)g * (C + 1) + c0] = a0[g];
        if (two) part[(int64_t)g * (C + 1) + c0 + 1] = a1[g];
      }
  }
}

// Per-token epilogue shared by the router kernels (one lane per token):
// acc holds the GP gate logits, the GP prototype dot products and the sum of
// squares of the token row.  Writes the token's outputs and the workgroup's
// telemetry partials (row `group` of stats) and returns the final gate
// probabilities in gate.
// hp_lds (HPLDS): the wave's (GP, 64) f32 LDS region, lane l's head
// probabilities in column l: the per-head sums then take one LDS add per
// gate instead of a register array indexed by every (gate, head) pair, in
// the same order (the same bits); the per-gate inputs are read where used.
// For 32 or 64 gates, where the register form spills.
template <int DT, int GP, bool PROTO, bool HPLDS = false>
__device__ __forceinline__ void router_epilogue(float (&acc)[2 * GP + 1], int64_t tok, bool live, int64_t group, int G,
                                                const float* __restrict__ conf_weight,
                                                const float* __restrict__ usage_bias,
                                                const int32_t* __restrict__ gate_to_head, int H, int topk,
                                                float proto_temp, float proto_threshold, float proto_blend,
                                                float usage_boost, float* __restrict__ gate_probs,
                                                float* __restrict__ sim_out, float* __restrict__ blend_out,
                                                float* __restrict__ importance, int32_t* __restrict__ head_idx,
                                                float* __restrict__ head_score, float* __restrict__ stats,
                                                float (&gate)[GP], float* hp_lds = nullptr) {
  constexpr int NV = 2 * GP + 1;
  const int lane = threadIdx.x & 63;
  // per-gate inputs loaded unconditionally (padding gates re-read gate G-1
  // and are never used) so that the loads are issued together
  constexpr int NP = HPLDS ? 1 : GP;
  float cwv[NP], ubv[NP];
  int hgv[NP];
  if constexpr (!HPLDS) {
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      const int gc = g < G ? g : G - 1;
      cwv[g] = conf_weight != nullptr ? conf_weight[gc] : 1.f;
      ubv[g] = usage_bias != nullptr ? usage_bias[gc] : 0.f;
      hgv[g] = gate_to_head[gc];
    }
  }
  auto cw_of = [&](int g) -> float {
    if constexpr (HPLDS) return conf_weight != nullptr ? conf_weight[g] : 1.f;
    else return cwv[g];
  };
  auto ub_of = [&](int g) -> float {
    if constexpr (HPLDS) return usage_bias != nullptr ? usage_bias[g] : 0.f;
    else return ubv[g];
  };
  float* logit = acc;
  float* dotp = acc + GP;
  const float sq = acc[NV - 1];

  // --- SwitchRouter: logits in x dtype, softmax in f32 rounded to x dtype.
  float lmax = -INFINITY;
#pragma unroll
  for (int g = 0; g < GP; ++g)
    if (g < G) { logit[g] = round_to<DT>(logit[g]); lmax = fmaxf(lmax, logit[g]); }
  float lsum = 0.f;
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    gate[g] = 0.f;
    if (g < G) { gate[g] = expf(logit[g] - lmax); lsum = lsum + gate[g]; }
  }
#pragma unroll
  for (int g = 0; g < GP; ++g)
    if (g < G) gate[g] = round_to<DT>(gate[g] / lsum);

  float sim_max = 0.f, blend_scalar = 0.f;
  if constexpr (PROTO) {
    float inv_den = fmaxf(sqrtf(sq), 1e-6f);
    float sims[GP];
    sim_max = -INFINITY;
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) { sims[g] = dotp[g] / inv_den; sim_max = fmaxf(sim_max, sims[g]); }
    float pp[GP];
    float smax = -INFINITY;
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) { pp[g] = sims[g] / proto_temp; smax = fmaxf(smax, pp[g]); }
    float ssum = 0.f;
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) { pp[g] = expf(pp[g] - smax); ssum = ssum + pp[g]; }
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) pp[g] = pp[g] / ssum;
    float den = fmaxf(1e-6f, 1.0f - proto_threshold);
    blend_scalar = fminf(fmaxf((sim_max - proto_threshold) / den, 0.f), 1.f);
    if (conf_weight != nullptr) {
      float cs = 0.f;
#pragma unroll
      for (int g = 0; g < GP; ++g)
        if (g < G) { pp[g] = pp[g] * cw_of(g); cs = cs + pp[g]; }
      cs = fmaxf(cs, 1e-6f);
#pragma unroll
      for (int g = 0; g < GP; ++g)
        if (g < G) pp[g] = pp[g] / cs;
    }
    float blend = proto_blend * blend_scalar;
    float one_m = 1.0f - blend;
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) gate[g] = gate[g] * one_m + pp[g] * blend;
    if (usage_bias != nullptr && usage_boost > 0.f) {
      float scale_u = (1.0f - blend_scalar) * usage_boost;
#pragma unroll
      for (int g = 0; g < GP; ++g)
        if (g < G) gate[g] = gate[g] + ub_of(g) * scale_u;
    }
    float gs = 0.f;
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) { gate[g] = fmaxf(gate[g], 0.f); gs = gs + gate[g]; }
    gs = fmaxf(gs, 1e-6f);
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G) gate[g] = gate[g] / gs;
  }

  float gmax = -INFINITY, ent = 0.f;
#pragma unroll
  for (int g = 0; g < GP; ++g)
    if (g < G) { gmax = fmaxf(gmax, gate[g]); ent = ent + logf(fmaxf(gate[g], 1e-9f)) * gate[g]; }
  float imp = PROTO ? (gmax * (1.0f - blend_scalar) + sim_max * blend_scalar) : gmax;

  float score_sum = 0.f;
  if (live) {
    if (gate_probs) {
#pragma unroll
      for (int g = 0; g < GP; ++g)
        if (g < G) gate_probs[tok * G + g] = gate[g];
    }
    if (sim_out) sim_out[tok] = sim_max;
    if (blend_out) blend_out[tok] = blend_scalar;
    importance[tok] = imp;

    // head_probs = gate_probs @ onehot(gate_to_head); top-k (ties -> lower head).
    float hp[HPLDS ? 1 : GP];
    if constexpr (HPLDS) {
      for (int h = 0; h < H; ++h) hp_lds[h * 64 + lane] = 0.f;
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const int hg = g < G ? gate_to_head[g] : -1;
        if ((unsigned)hg < (unsigned)H) hp_lds[hg * 64 + lane] += gate[g];  // heads outside [0, H) take nothing
      }
    } else {
#pragma unroll
      for (int h = 0; h < GP; ++h) hp[h] = 0.f;
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        if (g < G) {
          const int hg = hgv[g];
#pragma unroll
          for (int h = 0; h < GP; ++h)
            if (h == hg) hp[h] = hp[h] + gate[g];
        }
      }
    }
    auto hp_of = [&](int h) -> float {
      if constexpr (HPLDS) return hp_lds[h * 64 + lane];
      else return hp[h];
    };
    uint64_t taken = 0;
    for (int j = 0; j < topk; ++j) {
      float bv = 0.f;
      int bi = -1;
#pragma unroll
      for (int h = 0; h < GP; ++h) {
        if (h < H && !((taken >> h) & 1ull)) {
          const float v = hp_of(h);
          if (bi < 0 || better(v, h, bv, bi)) { bv = v; bi = h; }
        }
      }
      taken |= 1ull << bi;
      head_idx[tok * topk + j] = bi;
      if (head_score) head_score[tok * topk + j] = bv;
      score_sum += bv;
    }
  }
  if (stats) {
    // per-workgroup telemetry partials: entropy, sim, blend, #blend>0, top-k score sum
    float v[5] = {live ? -ent : 0.f, live ? sim_max : 0.f, live ? blend_scalar : 0.f,
                  (live && blend_scalar > 0.f) ? 1.f : 0.f, score_sum};
#pragma unroll
    for (int i = 0; i < 5; ++i)
      for (int off = 32; off > 0; off >>= 1) v[i] += __shfl_xor(v[i], off, 64);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 5; ++i) stats[group * 8 + i] = v[i];
    }
  }
}

// Router weights come pre-packed per channel as f32, wpk[c][0..GP) = W[:, c]
// and wpk[c][GP..2GP) = P[:, c] (GP = gates padded to 8/16/32/64, padding
// zero).  All lanes of a wave walk the channels in lock step, so the weight
// addresses are wave-uniform and 4-byte aligned: they are read with scalar
// loads and feed the FMAs as SGPR operands.  Each lane streams its own token
// row with 16-byte loads.  NW waves split the channels of the same 64 tokens
// and combine their partial dot products through LDS; wave 0 runs the
// epilogue.
template <int DT, int GP, bool PROTO, int NW>
__global__ void __launch_bounds__(64 * NW)
router_kernel(const typename Elem<DT>::T* __restrict__ x, int64_t n_tok, int C, int G,
              const float* __restrict__ wpk, const float* __restrict__ conf_weight,
              const float* __restrict__ usage_bias, const int32_t* __restrict__ gate_to_head, int H, int topk,
              float proto_temp, float proto_threshold, float proto_blend, float usage_boost,
              float* __restrict__ gate_probs, float* __restrict__ sim_out, float* __restrict__ blend_out,
              float* __restrict__ importance, int32_t* __restrict__ head_idx, float* __restrict__ head_score,
              float* __restrict__ stats, float* __restrict__ ema_part) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  constexpr int NV = 2 * GP + 1;  // logits, proto dots, sum of squares
  constexpr int WS = 2 * GP;  // row stride of the packed table (prototype columns unread without PROTO)
  __shared__ float red[(NW > 1) ? (NW - 1) * 64 * NV : 1];
  __shared__ float gl[64 * GP];  // final gate probabilities for the fused EMA statistics
  const int lane = threadIdx.x & 63;
  // wave index made explicitly wave-uniform so the channel loop (and with it
  // every weight address) lives in scalar registers
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t tok = (int64_t)blockIdx.x * kRouterTok + lane;
  const bool live = tok < n_tok;
  const typename Elem<DT>::T* xr = x + (live ? tok : 0) * C;
  float acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.f;

  const int cw = C / NW;  // channels of this wave (host guarantees C % (32*NW) == 0 when NW > 1)
  const int cbeg = wid * cw;
  if ((cw % 32) == 0) {
    float xa[4][8], xb[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) load8<DT>(xr + cbeg + 8 * u, xa[u]);
    for (int c0 = cbeg; c0 < cbeg + cw; c0 += 32) {
      const bool more = c0 + 32 < cbeg + cw;
      if (more) {
#pragma unroll
        for (int u = 0; u < 4; ++u) load8<DT>(xr + c0 + 32 + 8 * u, xb[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xv = xa[u][j];
          const float* w = wpk + (int64_t)(c0 + 8 * u + j) * WS;
          acc[NV - 1] = __builtin_fmaf(xv, xv, acc[NV - 1]);
#pragma unroll
          for (int g = 0; g < GP; ++g) acc[g] = __builtin_fmaf(xv, w[g], acc[g]);
          if constexpr (PROTO) {
#pragma unroll
            for (int g = 0; g < GP; ++g) acc[GP + g] = __builtin_fmaf(xv, w[GP + g], acc[GP + g]);
          }
        }
      }
      if (more) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < 8; ++j) xa[u][j] = xb[u][j];
      }
    }
  } else {
    for (int c = cbeg; c < cbeg + cw; ++c) {
      const float xv = load_f<DT>(xr + c);
      const float* w = wpk + (int64_t)c * WS;
      acc[NV - 1] = __builtin_fmaf(xv, xv, acc[NV - 1]);
#pragma unroll
      for (int g = 0; g < GP; ++g) acc[g] = __builtin_fmaf(xv, w[g], acc[g]);
      if constexpr (PROTO) {
#pragma unroll
        for (int g = 0; g < GP; ++g) acc[GP + g] = __builtin_fmaf(xv, w[GP + g], acc[GP + g]);
      }
    }
  }
  if constexpr (NW > 1) {
    if (wid > 0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) red[((wid - 1) * NV + i) * 64 + lane] = acc[i];
    }
    __syncthreads();
    if (wid > 0) {
      if (ema_part != nullptr) {
        __syncthreads();  // wave 0 has staged the gate probabilities
        router_ema_accum<DT, GP>(x, (int64_t)blockIdx.x * kRouterTok, n_tok, C, G, cbeg, cw, gl,
                                 ema_part + (int64_t)blockIdx.x * G * (C + 1));
      }
      return;
    }
#pragma unroll
    for (int w = 1; w < NW; ++w)
#pragma unroll
      for (int i = 0; i < NV; ++i) acc[i] = acc[i] + red[((w - 1) * NV + i) * 64 + lane];
  }
  float gate[GP];
  router_epilogue<DT, GP, PROTO>(acc, tok, live, blockIdx.x, G, conf_weight, usage_bias, gate_to_head, H, topk,
                                 proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim_out,
                                 blend_out, importance, head_idx, head_score, stats, gate);
  if (ema_part != nullptr) {
#pragma unroll
    for (int g = 0; g < GP; ++g) gl[lane * GP + g] = (live && g < G) ? gate[g] : 0.f;
    __syncthreads();
    float* part = ema_part + (int64_t)blockIdx.x * G * (C + 1);
    if (lane < G) {
      float cs = 0.f;  // column C: sum of gate g over the workgroup's tokens, in token order
      for (int u = 0; u < 64; ++u) cs += gl[u * GP + lane];
      part[(int64_t)lane * (C + 1) + C] = cs;
    }
    router_ema_accum<DT, GP>(x, (int64_t)blockIdx.x * kRouterTok, n_tok, C, G, cbeg, cw, gl, part);
  }
}

// ---------------------------------------------------------------------
// bf16 router on MFMA (8 or 16 gates)
// ---------------------------------------------------------------------
// Each wave owns one group of 64 tokens (4 tiles of 16) and computes, with
// v_mfma_f32_16x16x32_bf16, the product of 16-row operand tables with the
// tokens' rows.  The operand rows are, in this order, the GP gate weights
// (already rounded to bf16) and three bf16 parts of each normalised
// prototype: an f32 entry p is split as p = hi + mid + lo (hi = bf16(p),
// mid = bf16(p - hi), lo = bf16(p - hi - mid); every difference is exact in
// f32 and the three parts carry p's 24-bit significand), so with bf16 token
// values every product is exact in f32 and the prototype dots are f32 dots
// accumulated in a different order.  Operand row v (kind v / GP: weight, hi,
// mid, lo; gate v % GP) is row v % 16 of table v / 16: with 8 gates the
// tables are [W | hi] and [mid | lo], with 16 gates W, hi, mid and lo each
// fill a table.  Each table has its own accumulator.  Without prototypes
// only the weight table is multiplied.
//
// Channel order: lane (c16, g) of tile n holds the 32 consecutive channels
// 128q + 32g .. +31 of token 16n + c16 (four 16-byte loads, a whole 128-byte
// line per four lanes); half h of them feeds k-step s = 4q + h, so the table
// fragment of lane (r, g) for k-step s holds channels
// ch(s, g, j) = 128*(s/4) + 32g + 8*(s%4) + j.  The sum over channels does
// not depend on the order, only the two operands must agree.
constexpr int kRmWaves = 4;
constexpr int kPrepThreads = 256;  // router_prepare_kernel's workgroup
// Raw router inputs (bf16) for router_mfma_kernel<..., RAWIN = true>, which
// builds the pfa_router_prepare outputs itself: the (G, C) gate weights, the
// (G, C) prototypes (null without them), the confidence and usage (G) (null
// when unused).
struct RouterRaw {
  const uint16_t* w;
  const uint16_t* p;
  const uint16_t* conf;
  const uint16_t* usage;
};
constexpr int kRmEpW = 33;  // staged floats per token: GP logits, GP prototype dot parts, sum of squares

__host__ __device__ constexpr int rm_tables(int GP, bool proto) { return proto ? GP / 4 : 1; }

// Prototype EMA statistics of one 64-token group, one wave, on MFMA:
// part[g][c] = sum_t gate[t][g] * x[t][c].  D = A.B with v_mfma_f32_16x16x32_bf16,
// A = gates (rows) x tokens (k), B = tokens (k) x 16 channels.  A gate
// g = hi + mid + lo is split into three bf16 parts (as the router's
// prototype table: every difference exact, the parts carry g's whole
// significand), so every product with a bf16 x is exact in f32.  With 8
// gates A1 holds hi in rows 0-7 and mid in rows 8-15, A2 lo in rows 0-7;
// with 16 gates A1, A2 and A3 hold hi, mid and lo.  Each gate's sum is
// (hi + mid) + lo.  The x rows are staged in LDS 64 channels at a time (rows
// padded to kXsLd elements: the four rows of a transpose read fall in
// disjoint banks) and read as B by the LDS transpose read; gl holds the
// wave's gates [token][GP].
constexpr int kXsLd = 80;                          // staged x row, bf16 elements
constexpr int kXsWave = 64 * kXsLd * 2;            // bytes per wave

// LDS of the MFMA router: the operand tables (main loop), then the staged
// epilogue rows, then the gate rows and x staging of the EMA statistics, all
// in the same bytes.
__host__ __device__ constexpr int rm_lds_bytes(int C, int GP, bool proto) {
  const int table = 32 * C * rm_tables(GP, proto);
  const int stage = kRmWaves * 64 * kRmEpW * 4;
  const int ema = kRmWaves * 64 * GP * 4 + kRmWaves * kXsWave;
  const int m = table > stage ? table : stage;
  return m > ema ? m : ema;
}

static_assert(rm_lds_bytes(768, 8, true) <= 65536 && rm_lds_bytes(512, 16, true) <= 65536,
              "MFMA router LDS within 64 KiB at the widest rows it is launched for");

template <int GP>
__device__ __forceinline__ void ema_accum_mfma(const uint16_t* __restrict__ x, int64_t tok0, int nt, int C, int G,
                                               const float* gl, float* __restrict__ part, uint16_t* xs) {
  typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
  typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
  typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
  constexpr int NA = GP == 8 ? 2 : 3;
  constexpr int NB = GP <= 16 ? 1 : GP / 16;  // 16-gate blocks (32 or 64 gates: A rows 16b .. 16b + 15)
  const int lane = threadIdx.x & 63, m = lane & 15, kg = lane >> 4;
  // A operands for the two 32-token k-steps
  bf16x8 a[NB][NA][2];
#pragma unroll
  for (int bk = 0; bk < 2 * NB; ++bk) {
    const int b = bk >> 1, ks = bk & 1;
    uint16_t h[NA][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gv = gl[(32 * ks + 8 * kg + j) * GP + (GP == 8 ? (m & 7) : 16 * b + m)];
      const uint16_t hi = f32_to_bf16(gv);
      const float r1 = gv - bf16_to_f32(hi);
      const uint16_t mid = f32_to_bf16(r1);
      const uint16_t lo = f32_to_bf16(r1 - bf16_to_f32(mid));
      if constexpr (GP == 8) {
        h[0][j] = m < 8 ? hi : mid;
        h[1][j] = m < 8 ? lo : (uint16_t)0;
      } else {
        h[0][j] = hi;
        h[1][j] = mid;
        h[NA - 1][j] = lo;
      }
    }
#pragma unroll
    for (int t = 0; t < NA; ++t) __builtin_memcpy(&a[b][t][ks], h[t], 16);
  }
  // staging: lane l moves 16 bytes (channels 8*(l%8) ..+7) of tokens 8i + l/8
  const int srow = lane >> 3, scol = 8 * (lane & 7);
  auto fetch = [&](int cc, uint4 (&r)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = 8 * i + srow;
      r[i] = t < nt ? *reinterpret_cast<const uint4*>(x + (tok0 + t) * C + 64 * cc + scol) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  uint4 cur[8], nxt[8];
  fetch(0, cur);
  const int nc = C / 64;
  for (int cc = 0; cc < nc; ++cc) {
    wave_sync();  // the previous chunk's transpose reads are done
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(xs + (8 * i + srow) * kXsLd + scol) = cur[i];
    if (cc + 1 < nc) fetch(cc + 1, nxt);
    wave_sync();
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      bf16x8 bx[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // lane (n, kg) gets x[32ks + 8kg + 0..7][16ct + n]
        const uint16_t* p0 = xs + (32 * ks + 8 * kg + (m >> 2)) * kXsLd + 16 * ct + 4 * (m & 3);
        const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p0));
        const s16x4 hi4 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p0 + 4 * kXsLd));
        __builtin_memcpy(&bx[ks], &lo4, 8);
        __builtin_memcpy(reinterpret_cast<char*>(&bx[ks]) + 8, &hi4, 8);
      }
      const int c = 64 * cc + 16 * ct + m;
#pragma unroll
      for (int gbk = 0; gbk < NB; ++gbk) {
        f32x4 d[NA];
#pragma unroll
        for (int t = 0; t < NA; ++t) d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int t = 0; t < NA; ++t)
            d[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[gbk][t][ks], bx[ks], d[t], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 16 * gbk + 4 * kg + i;
          if constexpr (GP == 8) {
            // lanes 0-31 hold rows 4*(lane/16) + i: hi (d[0]) and lo (d[1]) of
            // gates 0-7; the mid of the same gates is in d[0] of lane + 32
            const auto sw =
                __builtin_amdgcn_permlane32_swap(__float_as_uint(d[0][i]), __float_as_uint(d[0][i]), false, false);
            if (lane < 32 && g < G) part[(int64_t)g * (C + 1) + c] = (d[0][i] + __uint_as_float(sw[1])) + d[1][i];
          } else {
            if (g < G) part[(int64_t)g * (C + 1) + c] = (d[0][i] + d[1][i]) + d[NA - 1][i];
          }
        }
      }
    }
    if (cc + 1 < nc) {
#pragma unroll
      for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
    }
  }
}

// Confidence weights and usage bias of pfa_router_prepare (G <= 64 gates,
// one lane each, one wave): r_cw[g] = bf16(conf[g] + 1e-6) and r_ub =
// bf16(softmax(-bf16(usage + 1e-6))), for g < GP (padding gates 1 and 0).
template <int GP>
__device__ __forceinline__ void rm_conf_usage(const RouterRaw& raw, int G, float* r_cw, float* r_ub) {
  const int lane = threadIdx.x & 63;
  const bool has = lane < G;
  if (raw.conf != nullptr) {
    const float v = has ? round_to<PFA_BF16>(bf16_to_f32(raw.conf[lane]) + 1e-6f) : 1.f;
    if (lane < GP) r_cw[lane] = v;
  }
  if (raw.usage != nullptr) {
    const float v = has ? -round_to<PFA_BF16>(bf16_to_f32(raw.usage[lane]) + 1e-6f) : -INFINITY;
    float m = v;
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float e = has ? expf(v - m) : 0.f;
    float sum = e;
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane < GP) r_ub[lane] = has ? round_to<PFA_BF16>(e / sum) : 0.f;
  }
}

// DOTS: one 16-gate block of a router with up to 64 gates (RAWIN, GP =
// 16): the block's gate logits, prototype dots and (block 0) the tokens'
// sums of squares go to rl, (2G + 1, n_tok) f32 (rows g, G + g and 2G), for
// router_epi_kernel; no epilogue.  The grid is 1-D, XCD-aware: workgroup L
// runs on XCD L mod 8, and the gate blocks of one token group take
// consecutive slots of one XCD, so x is read once into that XCD's L2.
template <int GP, bool PROTO, bool RAWIN, bool DOTS = false>
__global__ void __launch_bounds__(64 * kRmWaves)
router_mfma_kernel(const uint16_t* __restrict__ x, int64_t n_tok, int C, int G, const float* __restrict__ wpk,
                   const float* __restrict__ conf_weight, const float* __restrict__ usage_bias,
                   const int32_t* __restrict__ gate_to_head, int H, int topk, float proto_temp,
                   float proto_threshold, float proto_blend, float usage_boost, float* __restrict__ gate_probs,
                   float* __restrict__ sim_out, float* __restrict__ blend_out, float* __restrict__ importance,
                   int32_t* __restrict__ head_idx, float* __restrict__ head_score, float* __restrict__ stats,
                   float* __restrict__ ema_part, RouterRaw raw, float* __restrict__ rl = nullptr) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  static_assert(GP == 8 || GP == 16, "MFMA router tables hold 8 or 16 gates");
  static_assert(!DOTS || (GP == 16 && RAWIN), "gate blocks take the 16-gate tables from the raw weights");
  // DOTS: token group bx, gates gb .. gb + G - 1 of Gall
  int64_t bx = blockIdx.x;
  int gbk = 0;
  if constexpr (DOTS) {
    const int ngb = (G + 15) / 16;
    const int64_t slot = (int64_t)(blockIdx.x >> 3);
    gbk = (int)(slot % ngb);
    bx = (slot / ngb) * 8 + (blockIdx.x & 7);
    const int64_t n_wg = ((n_tok + kRouterTok - 1) / kRouterTok + kRmWaves - 1) / kRmWaves;
    if (bx >= n_wg) return;  // the grid is rounded up to whole slots of the eight XCDs
  }
  const int gb = 16 * gbk;
  const int Gall = G;
  if constexpr (DOTS) {
    G = min(16, Gall - gb);
    raw.w += (int64_t)gb * C;
    if (raw.p != nullptr) raw.p += (int64_t)gb * C;
  }
  constexpr int NT = rm_tables(GP, PROTO);
  typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
  typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
  extern __shared__ __align__(16) unsigned char rm_lds[];
  uint16_t* tab = reinterpret_cast<uint16_t*>(rm_lds);  // [C/32][NT][64 lanes][8]
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  // RAWIN: the router inputs of pfa_router_prepare built here from the bf16
  // weights, prototypes, confidence and usage (router_prepare_kernel's
  // arithmetic, thread-to-channel map and reduction order: the same bits)
  __shared__ float r_wsum[kRmWaves][RAWIN ? GP : 1];
  __shared__ float r_den[RAWIN ? GP : 1];
  __shared__ float r_cw[RAWIN ? GP : 1];
  __shared__ float r_ub[RAWIN ? GP : 1];
  if constexpr (RAWIN) {
    static_assert(64 * kRmWaves == kPrepThreads, "router_prepare_kernel's thread map");
    if (!DOTS && wid == kRmWaves - 1) rm_conf_usage<GP>(raw, G, r_cw, r_ub);
    if constexpr (PROTO) {
      float acc[GP];
#pragma unroll
      for (int g = 0; g < GP; ++g) acc[g] = 0.f;
      for (int ch = tid; ch < C; ch += 64 * kRmWaves) {
        // unconditional loads (padding gates re-read gate G-1 and are masked)
        float v[GP];
#pragma unroll
        for (int g = 0; g < GP; ++g) v[g] = bf16_to_f32(raw.p[(int64_t)(g < G ? g : G - 1) * C + ch]);
#pragma unroll
        for (int g = 0; g < GP; ++g) acc[g] = g < G ? __builtin_fmaf(v[g], v[g], acc[g]) : 0.f;
      }
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        float a = acc[g];
        for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
        if (lane == 0) r_wsum[wid][g] = a;
      }
      __syncthreads();
      if (tid < GP) {
        float t = 0.f;
        for (int k = 0; k < kRmWaves; ++k) t += r_wsum[k][tid];
        r_den[tid] = fmaxf(sqrtf(t), 1e-6f);
      }
    }
    __syncthreads();
  }

  // operand tables from the packed f32 rows (wpk[c][0..GP) = W, wpk[c][GP..2GP) = P)
  for (int ch = tid; ch < C; ch += 64 * kRmWaves) {
    float wv[GP], pv[GP];
    if constexpr (RAWIN) {
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const int64_t gi = (int64_t)(g < G ? g : G - 1) * C + ch;
        wv[g] = g < G ? bf16_to_f32(raw.w[gi]) : 0.f;  // bf16 weights: already rounded to the x dtype
        if constexpr (PROTO) pv[g] = g < G ? bf16_to_f32(raw.p[gi]) / r_den[g] : 0.f;
      }
    } else {
      const float4* src = reinterpret_cast<const float4*>(wpk + (int64_t)ch * 2 * GP);
#pragma unroll
      for (int k = 0; k < GP / 4; ++k) {
        const float4 w4 = src[k];
        wv[4 * k] = w4.x; wv[4 * k + 1] = w4.y; wv[4 * k + 2] = w4.z; wv[4 * k + 3] = w4.w;
        if constexpr (PROTO) {
          const float4 p4 = src[GP / 4 + k];
          pv[4 * k] = p4.x; pv[4 * k + 1] = p4.y; pv[4 * k + 2] = p4.z; pv[4 * k + 3] = p4.w;
        }
      }
    }
    const int st = 4 * (ch >> 7) + ((ch >> 3) & 3), g = (ch >> 5) & 3, j = ch & 7;
    uint16_t* base = tab + ((int64_t)st * NT * 64 + 16 * g) * 8 + j;
    auto put = [&](int v, uint16_t val) { base[(v >> 4) * 64 * 8 + (v & 15) * 8] = val; };
#pragma unroll
    for (int r = 0; r < GP; ++r) {
      put(r, f32_to_bf16(wv[r]));
      if constexpr (PROTO) {
        const uint16_t hi = f32_to_bf16(pv[r]);
        const float r1 = pv[r] - bf16_to_f32(hi);
        const uint16_t mid = f32_to_bf16(r1);
        const uint16_t lo = f32_to_bf16(r1 - bf16_to_f32(mid));
        put(GP + r, hi);
        put(2 * GP + r, mid);
        put(3 * GP + r, lo);
      } else if constexpr (GP == 8) {
        put(GP + r, 0);  // unused rows 8-15 of the weight table
      }
    }
  }
  __syncthreads();

  const int64_t group = bx * kRmWaves + wid;
  const int64_t n_groups = (n_tok + kRouterTok - 1) / kRouterTok;
  const int64_t tok0 = group * kRouterTok;
  const uint16_t* xr[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    int64_t t = tok0 + 16 * n + c16;
    t = t < n_tok ? t : n_tok - 1;
    xr[n] = x + t * C + 32 * g4;
  }
  f32x4 acc[NT][4];
  float ss[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    ss[n] = 0.f;
  }
  const int nq = C / 128;
  uint4 cur[4][4], nxt[4][4];
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int h = 0; h < 4; ++h) cur[n][h] = reinterpret_cast<const uint4*>(xr[n])[h];
  for (int q = 0; q < nq; ++q) {
    const bool more = q + 1 < nq;
    if (more) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int h = 0; h < 4; ++h) nxt[n][h] = reinterpret_cast<const uint4*>(xr[n] + 128 * (q + 1))[h];
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const uint16_t* tf = tab + ((int64_t)(4 * q + h) * NT * 64 + lane) * 8;
      bf16x8 a[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) a[t] = *reinterpret_cast<const bf16x8*>(tf + t * 64 * 8);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        bf16x8 b;
        __builtin_memcpy(&b, &cur[n][h], 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[t], b, acc[t][n], 0, 0, 0);
        const uint32_t w[4] = {cur[n][h].x, cur[n][h].y, cur[n][h].z, cur[n][h].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x0 = __uint_as_float(w[i] << 16), x1 = __uint_as_float(w[i] & 0xffff0000u);
          ss[n] = __builtin_fmaf(x0, x0, ss[n]);
          ss[n] = __builtin_fmaf(x1, x1, ss[n]);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int h = 0; h < 4; ++h) cur[n][h] = nxt[n][h];
    }
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    ss[n] += __shfl_xor(ss[n], 16, 64);
    ss[n] += __shfl_xor(ss[n], 32, 64);
  }
  // token-per-lane staging (reuses the table space once every wave is done).
  // Row layout: [0, 16) table-0 rows (the logits, and with 8 gates the hi
  // parts in 8-15), [16, 32) with 8 gates table 1 (mid, lo), with 16 gates
  // the prototype dots (lo + mid) + hi, [32] the sum of squares.
  __syncthreads();
  float* ep = reinterpret_cast<float*>(rm_lds) + wid * 64 * kRmEpW;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    float* e = ep + (16 * n + c16) * kRmEpW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[4 * g4 + i] = acc[0][n][i];
      float pd = 0.f;
      if constexpr (PROTO) {
        if constexpr (GP == 8) pd = acc[NT - 1][n][i];
        else pd = (acc[NT - 1][n][i] + acc[NT - 2][n][i]) + acc[1][n][i];
      }
      e[16 + 4 * g4 + i] = pd;
    }
    if (g4 == 0) e[32] = ss[n];
  }
  __syncthreads();
  float acc_t[2 * GP + 1];
  {
    const float* e = ep + lane * kRmEpW;
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      acc_t[g] = e[g];
      if constexpr (GP == 8) acc_t[GP + g] = (e[24 + g] + e[16 + g]) + e[8 + g];
      else acc_t[GP + g] = e[16 + g];
    }
    acc_t[2 * GP] = e[32];
  }
  const int64_t tok = tok0 + lane;
  const bool live = tok < n_tok;
  if constexpr (DOTS) {
    if (live) {
#pragma unroll
      for (int g = 0; g < GP; ++g)
        if (g < G) {
          rl[(int64_t)(gb + g) * n_tok + tok] = acc_t[g];
          if constexpr (PROTO) rl[(int64_t)(Gall + gb + g) * n_tok + tok] = acc_t[GP + g];
        }
      if (gbk == 0) rl[(int64_t)2 * Gall * n_tok + tok] = acc_t[2 * GP];
    }
    return;
  }
  float gate[GP];
  const float* cw_in = conf_weight;
  const float* ub_in = usage_bias;
  if constexpr (RAWIN) {
    cw_in = raw.conf != nullptr ? r_cw : nullptr;
    ub_in = raw.usage != nullptr ? r_ub : nullptr;
  }
  router_epilogue<PFA_BF16, GP, PROTO>(acc_t, tok, live, group, G, cw_in, ub_in, gate_to_head, H, topk,
                                       proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim_out,
                                       blend_out, importance, head_idx, head_score,
                                       group < n_groups ? stats : nullptr, gate);
  if (ema_part != nullptr) {
    __syncthreads();  // every wave has read its staged rows: the gate rows and x staging reuse those bytes
    float* gl = reinterpret_cast<float*>(rm_lds) + wid * 64 * GP;
#pragma unroll
    for (int g = 0; g < GP; ++g) gl[lane * GP + g] = (live && g < G) ? gate[g] : 0.f;
    __syncthreads();
    if (group < n_groups) {
      float* part = ema_part + group * G * (C + 1);
      if (lane < G) {
        float cs = 0.f;  // column C: sum of gate g over the group's tokens, in token order
        for (int u = 0; u < 64; ++u) cs += gl[u * GP + lane];
        part[(int64_t)lane * (C + 1) + C] = cs;
      }
      ema_accum_mfma<GP>(x, tok0, (int)min<int64_t>(64, n_tok - tok0), C, G, gl, part,
                         reinterpret_cast<uint16_t*>(rm_lds + kRmWaves * 64 * GP * 4 + wid * kXsWave));
    }
  }
}

// Epilogue of the router with 17-64 gates: a token per lane, 64 tokens per
// wave (router_mfma_kernel's groups), from the logits, prototype dots and
// sums of squares that router_mfma_kernel<16, PROTO, true, true> wrote to rl
// ((2G + 1, n_tok) f32); then the prototype EMA statistics of the wave's
// tokens on MFMA (ema_accum_mfma over 16-gate blocks).  The arithmetic of
// the 16-gate router: the same epilogue on the same f32 inputs.
// LDS of router_epi_kernel per wave: (GP, 64) f32 head probabilities /
// (64, GP) gate rows, or the x staging of the EMA statistics if larger.
__host__ __device__ constexpr int rm_epi_wave_bytes(int GP) { return 64 * GP * 4 > kXsWave ? 64 * GP * 4 : kXsWave; }
__host__ __device__ constexpr int rm_epi_lds_bytes(int GP) { return kRmWaves * rm_epi_wave_bytes(GP); }

template <int GP, bool PROTO>
__global__ void __launch_bounds__(64 * kRmWaves)
router_epi_kernel(const uint16_t* __restrict__ x, int64_t n_tok, int C, int G, const float* __restrict__ rl,
                  const int32_t* __restrict__ gate_to_head, int H, int topk, float proto_temp, float proto_threshold,
                  float proto_blend, float usage_boost, float* __restrict__ gate_probs, float* __restrict__ sim_out,
                  float* __restrict__ blend_out, float* __restrict__ importance, int32_t* __restrict__ head_idx,
                  float* __restrict__ head_score, float* __restrict__ stats, float* __restrict__ ema_part,
                  RouterRaw raw) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  static_assert(GP == 32 || GP == 64, "the gate-block epilogue takes 32 or 64 padded gates");
  extern __shared__ __align__(16) unsigned char rm_lds[];
  __shared__ float r_cw[GP];
  __shared__ float r_ub[GP];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (wid == 0) rm_conf_usage<GP>(raw, G, r_cw, r_ub);
  __syncthreads();
  const int64_t group = (int64_t)blockIdx.x * kRmWaves + wid;
  const int64_t n_groups = (n_tok + kRouterTok - 1) / kRouterTok;
  const int64_t tok0 = group * kRouterTok;
  const int64_t tok = tok0 + lane;
  const bool live = tok < n_tok;
  float acc_t[2 * GP + 1];
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    acc_t[g] = (live && g < G) ? rl[(int64_t)g * n_tok + tok] : 0.f;
    acc_t[GP + g] = (PROTO && live && g < G) ? rl[(int64_t)(G + g) * n_tok + tok] : 0.f;
  }
  acc_t[2 * GP] = live ? rl[(int64_t)2 * G * n_tok + tok] : 0.f;
  // the wave's LDS region: the head probabilities of the epilogue, then the
  // gate rows of the EMA statistics, then (once the MFMA operands are built
  // from them) its x staging
  float* gl = reinterpret_cast<float*>(rm_lds + wid * rm_epi_wave_bytes(GP));
  float gate[GP];
  // gate_probs is written below from the gate rows in LDS, a whole row per
  // store instruction
  router_epilogue<PFA_BF16, GP, PROTO, true>(acc_t, tok, live, group, G, raw.conf != nullptr ? r_cw : nullptr,
                                             raw.usage != nullptr ? r_ub : nullptr, gate_to_head, H, topk,
                                             proto_temp, proto_threshold, proto_blend, usage_boost, nullptr,
                                             sim_out, blend_out, importance, head_idx, head_score,
                                             group < n_groups ? stats : nullptr, gate, gl);
  if (gate_probs == nullptr && ema_part == nullptr) return;
  wave_sync();  // the epilogue's reads of the region are done
#pragma unroll
  for (int g = 0; g < GP; ++g) gl[lane * GP + g] = (live && g < G) ? gate[g] : 0.f;
  wave_sync();
  if (gate_probs != nullptr && group < n_groups) {
    const int nt = (int)min<int64_t>(64, n_tok - tok0);
    for (int t = 0; t < nt; ++t)
      if (lane < G) gate_probs[(tok0 + t) * G + lane] = gl[t * GP + lane];
  }
  if (ema_part != nullptr) {
    if (group < n_groups) {
      float* part = ema_part + group * G * (C + 1);
      if (lane < G) {
        float cs = 0.f;  // column C: sum of gate g over the group's tokens, in token order
        for (int u = 0; u < 64; ++u) cs += gl[u * GP + lane];
        part[(int64_t)lane * (C + 1) + C] = cs;
      }
      // ema_accum_mfma reads the gate rows into its operands before its
      // first wave_sync and x staging write
      ema_accum_mfma<GP>(x, tok0, (int)min<int64_t>(64, n_tok - tok0), C, G, gl, part,
                         reinterpret_cast<uint16_t*>(gl));
    }
  }
}

// Prototype EMA partial sums: part p accumulates, for a slice of at most
// kEmaTok tokens, sum_t gate[t,g]*x[t,c] (columns 0..C-1) and sum_t gate[t,g]
// (column C).  The slice's gate rows are staged in LDS (zero-padded to GMAX
// gates) and read back as broadcast float4s; a thread owns a pair of
// channels (one 4-byte load per token, coalesced across the workgroup), with
// eight tokens in flight per step.  Every sum runs in token order, so the
// result does not depend on scheduling.
constexpr int kEmaThreads = 256;
constexpr int kEmaTok = 64;
constexpr int kEmaMaxParts = 4096;
constexpr int kEmaGroup = 32;  // parts summed per thread in the first reduce level

template <int DT, int GMAX>
__global__ void __launch_bounds__(kEmaThreads)
proto_accum_kernel(const typename Elem<DT>::T* __restrict__ x, int64_t n_tok, int C, int G,
                   const float* __restrict__ gate_probs, int64_t tok_per_part, float* __restrict__ partial) {
  __shared__ float4 g_lds[kEmaTok * (GMAX / 4)];
  const int part = blockIdx.x;
  const int64_t tb = (int64_t)part * tok_per_part;
  const int64_t te = min(n_tok, tb + tok_per_part);
  float* out = partial + (int64_t)part * G * (C + 1);
  if (tb >= te) {
    // trailing parts past the last token (the part count is capped and
    // rounded): their rows still take part in the reduction
    for (int64_t i = threadIdx.x; i < (int64_t)G * (C + 1); i += blockDim.x) out[i] = 0.f;
    return;
  }
  const int npair = (C + 1) / 2;
  float* gl = reinterpret_cast<float*>(g_lds);
  float a0[GMAX], a1[GMAX];
  float csum = 0.f;
  const int cp = threadIdx.x;
  for (int64_t t0 = tb; t0 < te; t0 += kEmaTok) {
    const int nt = (int)min<int64_t>(kEmaTok, te - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < kEmaTok * GMAX; i += blockDim.x) {
      const int u = i / GMAX, g = i % GMAX;
      gl[i] = (u < nt && g < G) ? gate_probs[(t0 + u) * G + g] : 0.f;
    }
    __syncthreads();
    if (threadIdx.x < GMAX) {
      // column C: lane g sums gate g over the slice, in token order
      for (int u = 0; u < nt; ++u) csum += gl[u * GMAX + threadIdx.x];
    }
    for (int c2 = cp; c2 < npair; c2 += blockDim.x) {
      const int c0 = 2 * c2;
      const bool two = c0 + 1 < C;
      if (t0 == tb || C > 2 * (int)blockDim.x) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) { a0[g] = 0.f; a1[g] = 0.f; }
      }
      if (C > 2 * (int)blockDim.x && t0 != tb) {
        // wide rows: reload the running sums of this channel pair
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) {
            a0[g] = out[(int64_t)g * (C + 1) + c0];
            if (two) a1[g] = out[(int64_t)g * (C + 1) + c0 + 1];
          }
      }
      int u = 0;
      for (; u + 8 <= nt; u += 8) {
        float x0[8], x1[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) load2<DT>(x + (t0 + u + k) * C + c0, two, x0[k], x1[k]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
#pragma unroll
          for (int q = 0; q < GMAX / 4; ++q) {
            const float4 pr = g_lds[(u + k) * (GMAX / 4) + q];
            a0[4 * q + 0] = __builtin_fmaf(pr.x, x0[k], a0[4 * q + 0]);
            a0[4 * q + 1] = __builtin_fmaf(pr.y, x0[k], a0[4 * q + 1]);
            a0[4 * q + 2] = __builtin_fmaf(pr.z, x0[k], a0[4 * q + 2]);
            a0[4 * q + 3] = __builtin_fmaf(pr.w, x0[k], a0[4 * q + 3]);
            a1[4 * q + 0] = __builtin_fmaf(pr.x, x1[k], a1[4 * q + 0]);
            a1[4 * q + 1] = __builtin_fmaf(pr.y, x1[k], a1[4 * q + 1]);
            a1[4 * q + 2] = __builtin_fmaf(pr.z, x1[k], a1[4 * q + 2]);
            a1[4 * q + 3] = __builtin_fmaf(pr.w, x1[k], a1[4 * q + 3]);
          }
        }
      }
      for (; u < nt; ++u) {
        float x0, x1;
        load2<DT>(x + (t0 + u) * C + c0, two, x0, x1);
#pragma unroll
        for (int q = 0; q < GMAX / 4; ++q) {
          const float4 pr = g_lds[u * (GMAX / 4) + q];
          a0[4 * q + 0] = __builtin_fmaf(pr.x, x0, a0[4 * q + 0]);
          a0[4 * q + 1] = __builtin_fmaf(pr.y, x0, a0[4 * q + 1]);
          a0[4 * q + 2] = __builtin_fmaf(pr.z, x0, a0[4 * q + 2]);
          a0[4 * q + 3] = __builtin_fmaf(pr.w, x0, a0[4 * q + 3]);
          a1[4 * q + 0] = __builtin_fmaf(pr.x, x1, a1[4 * q + 0]);
          a1[4 * q + 1] = __builtin_fmaf(pr.y, x1, a1[4 * q + 1]);
          a1[4 * q + 2] = __builtin_fmaf(pr.z, x1, a1[4 * q + 2]);
          a1[4 * q + 3] = __builtin_fmaf(pr.w, x1, a1[4 * q + 3]);
        }
      }
      const bool last = t0 + kEmaTok >= te;
      if (last || C > 2 * (int)blockDim.x) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          if (g < G) {
            out[(int64_t)g * (C + 1) + c0] = a0[g];
            if (two) out[(int64_t)g * (C + 1) + c0 + 1] = a1[g];
          }
        }
      }
    }
  }
  if (threadIdx.x < G) out[(int64_t)threadIdx.x * (C + 1) + C] = csum;
}

// Sum of the partial rows, in two fixed-order levels (in place): level 0
// sums rows [k*kEmaGroup, (k+1)*kEmaGroup) into row k*kEmaGroup; level 1 sums
// rows 0, kEmaGroup, 2*kEmaGroup, ... into out.  Each thread owns one column.
__global__ void __launch_bounds__(256) partial_reduce_group(float* __restrict__ partial, int n_parts, int64_t width) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= width) return;
  const int p0 = blockIdx.y * kEmaGroup;
  const int p1 = min(n_parts, p0 + kEmaGroup);
  float v[kEmaGroup];
#pragma unroll
  for (int k = 0; k < kEmaGroup; ++k) v[k] = (p0 + k < p1) ? partial[(int64_t)(p0 + k) * width + i] : 0.f;
  float s = v[0];
#pragma unroll
  for (int k = 1; k < kEmaGroup; ++k) s = s + v[k];
  partial[(int64_t)p0 * width + i] = s;
}

__global__ void __launch_bounds__(256) partial_reduce_final(const float* __restrict__ partial, int n_groups,
                                                            int64_t width, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= width) return;
  float s = 0.f;
  int k = 0;
  for (; k + 8 <= n_groups; k += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = partial[(int64_t)(k + j) * kEmaGroup * width + i];
#pragma unroll
    for (int j = 0; j < 8; ++j) s = s + v[j];
  }
  for (; k < n_groups; ++k) s = s + partial[(int64_t)k * kEmaGroup * width + i];
  out[i] = s;
}

// EMA update of prototypes / usage / confidence from the reduced sums
// (aspa.py:700-716), each product and sum rounded to the buffer dtype as the
// reference's in-place tensor ops do.  One thread per (gate, channel).
template <int DT>
__global__ void proto_ema_update_kernel(const float* __restrict__ sums, int G, int C, float decay,
                                        typename Elem<DT>::T* __restrict__ protos,
                                        typename Elem<DT>::T* __restrict__ usage,
                                        typename Elem<DT>::T* __restrict__ conf) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)G * C) return;
  const int g = (int)(i / C), c = (int)(i % C);
  const float cnt = sums[(int64_t)g * (C + 1) + C];
  const bool upd = cnt > 1e-6f;
  const float om = 1.0f - decay;
  if (upd) {
    float mean = round_to<DT>(sums[(int64_t)g * (C + 1) + c] / cnt);
    float p = load_f<DT>(protos + i);
    store_f<DT>(protos + i, round_to<DT>(round_to<DT>(p * decay) + round_to<DT>(mean * om)));
  }
  if (c == 0) {
    float u = round_to<DT>(load_f<DT>(usage + g) * decay);
    if (upd) u = round_to<DT>(u + cnt * om);
    store_f<DT>(usage + g, u);
    float cf = round_to<DT>(load_f<DT>(conf + g) * decay);
    if (upd) cf = round_to<DT>(cf + om);
    store_f<DT>(conf + g, cf);
  }
}

static int gate_pad(int G) { return G <= 8 ? 8 : G <= 16 ? 16 : G <= 32 ? 32 : 64; }

// Per-forward router inputs in one launch (one workgroup): the channel-
// interleaved weight table, the L2-normalised prototypes
// (F.normalize(P.float(), dim=-1, eps=1e-6) = P / max(||P||, 1e-6)), the
// confidence weights (confidence + 1e-6, rounded to the buffer dtype as the
// reference's tensor add) and the usage bias softmax(-(usage + 1e-6)) in the
// buffer dtype (aspa.py:636-663).
template <int WDT, int PDT, int XDT, int GP>
__global__ void __launch_bounds__(kPrepThreads)
router_prepare_kernel(const typename Elem<WDT>::T* __restrict__ w, const typename Elem<PDT>::T* __restrict__ protos,
                      const typename Elem<PDT>::T* __restrict__ conf, const typename Elem<PDT>::T* __restrict__ usage,
                      int G, int C, float* __restrict__ wpk, float* __restrict__ conf_w,
                      float* __restrict__ usage_b) {
  PFA_CRITICAL_CHAIN_PRIORITY();
  // one pass: each thread owns channels c = tid + k*kPrepThreads; the G
  // prototype norms are reduced once for all gates, then each thread writes
  // its channels' 2*GP-float rows
  __shared__ float wsum[kPrepThreads / 64][GP];
  __shared__ float denom[GP];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (wv == kPrepThreads / 64 - 1) {
    // confidence weights and usage softmax, one gate per lane of the last
    // wave (independent loads issued together, wave reductions); the other
    // waves start on the prototype norms meanwhile
    const bool has = lane < G;
    if (conf != nullptr && conf_w != nullptr && has)
      conf_w[lane] = round_to<PDT>(load_f<PDT>(conf + lane) + 1e-6f);
    if (usage != nullptr && usage_b != nullptr) {
      const float v = has ? -round_to<PDT>(load_f<PDT>(usage + lane) + 1e-6f) : -INFINITY;
      float m = v;
      for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      const float e = has ? expf(v - m) : 0.f;
      float sum = e;
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      if (has) usage_b[lane] = round_to<PDT>(e / sum);
    }
  }
  if (protos != nullptr) {
    float acc[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) acc[g] = 0.f;
    for (int c = tid; c < C; c += kPrepThreads) {
      // unconditional loads (padding gates re-read gate G-1 and are masked
      // afterwards) so that all GP loads are in flight together
      float v[GP];
#pragma unroll
      for (int g = 0; g < GP; ++g) v[g] = load_f<PDT>(protos + (int64_t)(g < G ? g : G - 1) * C + c);
#pragma unroll
      for (int g = 0; g < GP; ++g) acc[g] = g < G ? __builtin_fmaf(v[g], v[g], acc[g]) : 0.f;
    }
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      float a = acc[g];
      for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
      if (lane == 0) wsum[wv][g] = a;
    }
    __syncthreads();
    if (tid < GP) {
      float t = 0.f;
      for (int k = 0; k < kPrepThreads / 64; ++k) t += wsum[k][tid];
      denom[tid] = fmaxf(sqrtf(t), 1e-6f);
    }
    __syncthreads();
  }
  for (int c = tid; c < C; c += kPrepThreads) {
    float row[2 * GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) row[g] = load_f<WDT>(w + (int64_t)(g < G ? g : G - 1) * C + c);
    if (protos != nullptr) {
#pragma unroll
      for (int g = 0; g < GP; ++g) row[GP + g] = load_f<PDT>(protos + (int64_t)(g < G ? g : G - 1) * C + c);
    }
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      row[g] = g < G ? round_to<XDT>(row[g]) : 0.f;
      row[GP + g] = (protos != nullptr && g < G) ? row[GP + g] / denom[g] : 0.f;
    }
    float4* dst = reinterpret_cast<float4*>(wpk + (int64_t)c * 2 * GP);
#pragma unroll
    for (int k = 0; k < GP / 2; ++k) dst[k] = make_float4(row[4 * k], row[4 * k + 1], row[4 * k + 2], row[4 * k + 3]);
  }
}

template <int DT, int GP, bool PROTO>
static void launch_router_gp(const void* x, int64_t n_tok, int C, int G, const float* wpk, const float* cw,
                             const float* ub, const int32_t* g2h, int H, int topk, float temp, float thr, float pb,
                             float boost, float* gp, float* sim, float* bl, float* imp, int32_t* hi, float* hs,
                             float* stats, float* ema, hipStream_t s) {
  using ET = typename Elem<DT>::T;
  unsigned blocks = (unsigned)((n_tok + kRouterTok - 1) / kRouterTok);
  if constexpr (DT == PFA_BF16 && (GP == 8 || GP == 16)) {
    // the operand tables stay within 64 KiB of LDS
    if (C % 128 == 0 && C <= (GP == 8 ? 768 : 512)) {
      const unsigned mb = (blocks + kRmWaves - 1) / kRmWaves;
      const size_t lds = (size_t)rm_lds_bytes(C, GP, PROTO);
      router_mfma_kernel<GP, PROTO, false><<<mb, 64 * kRmWaves, lds, s>>>(
          (const uint16_t*)x, n_tok, C, G, wpk, cw, ub, g2h, H, topk, temp, thr, pb, boost, gp, sim, bl, imp, hi, hs,
          stats, ema, RouterRaw{nullptr, nullptr, nullptr, nullptr});
      return;
    }
  }
  if (GP <= 16 && C % 128 == 0)
    router_kernel<DT, GP, PROTO, 4><<<blocks, 256, 0, s>>>((const ET*)x, n_tok, C, G, wpk, cw, ub, g2h, H, topk,
                                                           temp, thr, pb, boost, gp, sim, bl, imp, hi, hs, stats,
                                                           ema);
  else
    router_kernel<DT, GP, PROTO, 1><<<blocks, 64, 0, s>>>((const ET*)x, n_tok, C, G, wpk, cw, ub, g2h, H, topk,
                                                          temp, thr, pb, boost, gp, sim, bl, imp, hi, hs, stats,
                                                          ema);
}

template <int DT>
static int launch_router(const void* x, int64_t n_tok, int C, int G, const float* wpk, bool proto, const float* cw,
                         const float* ub, const int32_t* g2h, int H, int topk, float temp, float thr, float pb,
                         float boost, float* gp, float* sim, float* bl, float* imp, int32_t* hi, float* hs,
                         float* stats, float* ema, hipStream_t s) {
#define PFA_R(GPV)                                                                                             \
  do {                                                                                                         \
    if (proto)                                                                                                 \
      launch_router_gp<DT, GPV, true>(x, n_tok, C, G, wpk, cw, ub, g2h, H, topk, temp, thr, pb, boost, gp, sim, \
                                      bl, imp, hi, hs, stats, ema, s);                                         \
    else                                                                                                       \
      launch_router_gp<DT, GPV, false>(x, n_tok, C, G, wpk, cw, ub, g2h, H, topk, temp, thr, pb, boost, gp,    \
                                       sim, bl, imp, hi, hs, stats, ema, s);                                   \
  } while (0)
  switch (gate_pad(G)) {
    case 8: PFA_R(8); break;
    case 16: PFA_R(16); break;
    case 32: PFA_R(32); break;
    default: PFA_R(64); break;
  }
#undef PFA_R
  PFA_CHECK_LAUNCH("pfa_router_topk");
  return PFA_OK;
}

template <int DT>
static void launch_accum(const void* x, int64_t n_tok, int C, int G, const float* gp, int n_parts,
                         int64_t per, float* partial, hipStream_t s) {
  using ET = typename Elem<DT>::T;
  if (G <= 8) proto_accum_kernel<DT, 8><<<n_parts, kEmaThreads, 0, s>>>((const ET*)x, n_tok, C, G, gp, per, partial);
  else if (G <= 16) proto_accum_kernel<DT, 16><<<n_parts, kEmaThreads, 0, s>>>((const ET*)x, n_tok, C, G, gp, per, partial);
  else if (G <= 32) proto_accum_kernel<DT, 32><<<n_parts, kEmaThreads, 0, s>>>((const ET*)x, n_tok, C, G, gp, per, partial);
  else proto_accum_kernel<DT, 64><<<n_parts, kEmaThreads, 0, s>>>((const ET*)x, n_tok, C, G, gp, per, partial);
}

// Telemetry partials (n_blocks, 8) summed column-wise in f64 into out[8]:
// thread t owns column t % 8 and the blocks t/8 + 128k; each pass issues
// eight independent loads before adding them, and the 128 per-column
// partials are then added in a fixed tree order (deterministic).
__global__ void __launch_bounds__(1024) router_stats_reduce_kernel(const float* __restrict__ stats, int n_blocks,
                                                                   double* __restrict__ out) {
  __shared__ double part[1024];
  const int t = threadIdx.x, c = t & 7, b0 = t >> 3;
  double acc = 0.0;
  for (int base = 0; base < n_blocks; base += 1024) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int b = base + b0 + 128 * k;
      v[k] = b < n_blocks ? stats[(int64_t)b * 8 + c] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += (double)v[k];
  }
  part[t] = acc;
  __syncthreads();
  for (int w = 512; w >= 8; w >>= 1) {
    if (t < w) part[t] += part[t + w];
    __syncthreads();
  }
  if (t < 8) out[t] = part[t];
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_router_gate_pad(int G) { return gate_pad(G); }

extern "C" int pfa_router_prepare(const void* w_router, int w_dtype, const void* protos, const void* confidence,
                                  const void* usage, int buf_dtype, int G, int C, int x_dtype, float* w_packed,
                                  float* conf_weight, float* usage_bias, void* stream) {
  clear_error();
  PFA_CHECK_ARG(w_router && w_packed && G > 0 && G <= 64 && C > 0, "pfa_router_prepare: bad arguments");
  PFA_CHECK_ARG(((uintptr_t)w_packed & 15) == 0, "pfa_router_prepare: w_packed must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int GP = gate_pad(G);
#define PFA_PREP_G(WD, PD, XD, GPV)                                                                         \
  router_prepare_kernel<WD, PD, XD, GPV><<<1, kPrepThreads, 0, s>>>(                                        \
      (const typename Elem<WD>::T*)w_router, (const typename Elem<PD>::T*)protos,                            \
      (const typename Elem<PD>::T*)confidence, (const typename Elem<PD>::T*)usage, G, C, w_packed,            \
      conf_weight, usage_bias)
#define PFA_PREP(WD, PD, XD)                              \
  do {                                                    \
    if (GP == 8) PFA_PREP_G(WD, PD, XD, 8);               \
    else if (GP == 16) PFA_PREP_G(WD, PD, XD, 16);        \
    else if (GP == 32) PFA_PREP_G(WD, PD, XD, 32);        \
    else PFA_PREP_G(WD, PD, XD, 64);                      \
  } while (0)
#define PFA_PREP_X(WD, PD)                                                 \
  switch (x_dtype) {                                                       \
    case PFA_F32: PFA_PREP(WD, PD, PFA_F32); break;                        \
    case PFA_BF16: PFA_PREP(WD, PD, PFA_BF16); break;                      \
    case PFA_F16: PFA_PREP(WD, PD, PFA_F16); break;                        \
    default: set_error("pfa_router_prepare: x dtype %d", x_dtype); return PFA_E_UNSUPPORTED; \
  }
#define PFA_PREP_P(WD)                                                     \
  switch (buf_dtype) {                                                     \
    case PFA_F32: PFA_PREP_X(WD, PFA_F32); break;                          \
    case PFA_BF16: PFA_PREP_X(WD, PFA_BF16); break;                        \
    case PFA_F16: PFA_PREP_X(WD, PFA_F16); break;                          \
    default: set_error("pfa_router_prepare: buffer dtype %d", buf_dtype); return PFA_E_UNSUPPORTED; \
  }
  switch (w_dtype) {
    case PFA_F32: PFA_PREP_P(PFA_F32); break;
    case PFA_BF16: PFA_PREP_P(PFA_BF16); break;
    case PFA_F16: PFA_PREP_P(PFA_F16); break;
    default: set_error("pfa_router_prepare: weight dtype %d", w_dtype); return PFA_E_UNSUPPORTED;
  }
#undef PFA_PREP_P
#undef PFA_PREP_X
#undef PFA_PREP
#undef PFA_PREP_G
  PFA_CHECK_LAUNCH("pfa_router_prepare");
  return PFA_OK;
}

extern "C" int pfa_router_topk(const void* x, int x_dtype, int64_t n_tok, int C, int G, const float* w_packed,
                               int use_proto, const float* conf_weight, const float* usage_bias,
                               const int32_t* gate_to_head, int H, int topk, float proto_temp, float proto_threshold,
                               float proto_blend, float usage_boost, float* gate_probs, float* sim, float* blend,
                               float* importance, int32_t* head_idx, float* head_score, float* stats_partial,
                               float* ema_partial, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n_tok >= 0 && C > 0 && G > 0 && G <= 64 && H > 0 && H <= G && topk >= 1 && topk <= H,
                "pfa_router_topk: bad sizes n_tok=%lld C=%d G=%d H=%d topk=%d", (long long)n_tok, C, G, H, topk);
  PFA_CHECK_ARG(x && w_packed && gate_to_head && importance && head_idx, "pfa_router_topk: null pointer");
  if (n_tok == 0) return PFA_OK;
  hipStream_t s = as_stream(stream);
  const bool pr = use_proto != 0;
  switch (x_dtype) {
    case PFA_F32:
      return launch_router<PFA_F32>(x, n_tok, C, G, w_packed, pr, conf_weight, usage_bias, gate_to_head, H, topk,
                                    proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim, blend,
                                    importance, head_idx, head_score, stats_partial, ema_partial, s);
    case PFA_BF16:
      return launch_router<PFA_BF16>(x, n_tok, C, G, w_packed, pr, conf_weight, usage_bias, gate_to_head, H, topk,
                                     proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim, blend,
                                     importance, head_idx, head_score, stats_partial, ema_partial, s);
    case PFA_F16:
      return launch_router<PFA_F16>(x, n_tok, C, G, w_packed, pr, conf_weight, usage_bias, gate_to_head, H, topk,
                                    proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim, blend,
                                    importance, head_idx, head_score, stats_partial, ema_partial, s);
    default:
      set_error("pfa_router_topk: unsupported dtype %d", x_dtype);
      return PFA_E_UNSUPPORTED;
  }
}

// The MFMA router with its inputs built in each workgroup: bf16 x, weights
// and prototype buffers, C a multiple of 128 up to 768 (8 gates) or 512
// (9-64 gates: 16-gate tables); up to 16 gates in one fused launch
// (pfa_router_topk_raw), 17-64 in 16-gate blocks and an epilogue launch
// (pfa_router_topk_raw_ws).
static bool router_raw_ok(int x_dtype, int w_dtype, int buf_dtype, int G, int C, bool proto, int max_g) {
  if (x_dtype != PFA_BF16 || w_dtype != PFA_BF16 || (proto && buf_dtype != PFA_BF16)) return false;
  if (G < 1 || G > max_g || C <= 0 || C % 128 != 0) return false;
  return C <= (gate_pad(G) == 8 ? 768 : 512);
}

extern "C" int pfa_router_raw_supported(int x_dtype, int w_dtype, int buf_dtype, int G, int C, int use_proto) {
  return router_raw_ok(x_dtype, w_dtype, buf_dtype, G, C, use_proto != 0, 64) ? 1 : 0;
}

extern "C" int pfa_router_raw_workspace_size(int64_t n_tok, int G, size_t* bytes) {
  clear_error();
  PFA_CHECK_ARG(bytes != nullptr && n_tok >= 0 && G > 0 && G <= 64, "pfa_router_raw_workspace_size: bad arguments");
  *bytes = G > 16 ? (size_t)(2 * G + 1) * (size_t)n_tok * sizeof(float) : 0;
  return PFA_OK;
}

extern "C" int pfa_router_topk_raw(const void* x, int x_dtype, int64_t n_tok, int C, int G, const void* w_router,
                                   int w_dtype, const void* protos, const void* confidence, const void* usage,
                                   int buf_dtype, const int32_t* gate_to_head, int H, int topk, float proto_temp,
                                   float proto_threshold, float proto_blend, float usage_boost, float* gate_probs,
                                   float* sim, float* blend, float* importance, int32_t* head_idx, float* head_score,
                                   float* stats_partial, float* ema_partial, void* stream) {
  clear_error();
  PFA_CHECK_ARG(n_tok >= 0 && C > 0 && G > 0 && G <= 64 && H > 0 && H <= G && topk >= 1 && topk <= H,
                "pfa_router_topk_raw: bad sizes n_tok=%lld C=%d G=%d H=%d topk=%d", (long long)n_tok, C, G, H, topk);
  PFA_CHECK_ARG(x && w_router && gate_to_head && importance && head_idx, "pfa_router_topk_raw: null pointer");
  const bool pr = protos != nullptr;
  if (!router_raw_ok(x_dtype, w_dtype, buf_dtype, G, C, pr, 16)) {
    set_error("pfa_router_topk_raw: unsupported (x dtype %d, weight dtype %d, buffer dtype %d, G=%d, C=%d; "
              "17-64 gates take pfa_router_topk_raw_ws)", x_dtype, w_dtype, buf_dtype, G, C);
    return PFA_E_UNSUPPORTED;
  }
  if (n_tok == 0) return PFA_OK;
  hipStream_t s = as_stream(stream);
  const RouterRaw raw{(const uint16_t*)w_router, (const uint16_t*)protos, pr ? (const uint16_t*)confidence : nullptr,
                      pr ? (const uint16_t*)usage : nullptr};
  const unsigned blocks = (unsigned)((n_tok + kRouterTok - 1) / kRouterTok);
  const unsigned mb = (blocks + kRmWaves - 1) / kRmWaves;
#define PFA_RR(GPV, PV)                                                                                          \
  router_mfma_kernel<GPV, PV, true><<<mb, 64 * kRmWaves, (size_t)rm_lds_bytes(C, GPV, PV), s>>>(                  \
      (const uint16_t*)x, n_tok, C, G, nullptr, nullptr, nullptr, gate_to_head, H, topk, proto_temp,              \
      proto_threshold, proto_blend, usage_boost, gate_probs, sim, blend, importance, head_idx, head_score,        \
      stats_partial, ema_partial, raw)
  if (gate_pad(G) == 8) {
    if (pr) PFA_RR(8, true);
    else PFA_RR(8, false);
  } else {
    if (pr) PFA_RR(16, true);
    else PFA_RR(16, false);
  }
#undef PFA_RR
  PFA_CHECK_LAUNCH("pfa_router_topk_raw");
  return PFA_OK;
}

extern "C" int pfa_router_topk_raw_ws(const void* x, int x_dtype, int64_t n_tok, int C, int G, const void* w_router,
                                      int w_dtype, const void* protos, const void* confidence, const void* usage,
                                      int buf_dtype, const int32_t* gate_to_head, int H, int topk, float proto_temp,
                                      float proto_threshold, float proto_blend, float usage_boost, float* gate_probs,
                                      float* sim, float* blend, float* importance, int32_t* head_idx,
                                      float* head_score, float* stats_partial, float* ema_partial, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (G <= 16)
    return pfa_router_topk_raw(x, x_dtype, n_tok, C, G, w_router, w_dtype, protos, confidence, usage, buf_dtype,
                               gate_to_head, H, topk, proto_temp, proto_threshold, proto_blend, usage_boost,
                               gate_probs, sim, blend, importance, head_idx, head_score, stats_partial, ema_partial,
                               stream);
  clear_error();
  PFA_CHECK_ARG(n_tok >= 0 && C > 0 && G > 0 && G <= 64 && H > 0 && H <= G && topk >= 1 && topk <= H,
                "pfa_router_topk_raw_ws: bad sizes n_tok=%lld C=%d G=%d H=%d topk=%d", (long long)n_tok, C, G, H,
                topk);
  PFA_CHECK_ARG(x && w_router && gate_to_head && importance && head_idx, "pfa_router_topk_raw_ws: null pointer");
  const bool pr = protos != nullptr;
  if (!router_raw_ok(x_dtype, w_dtype, buf_dtype, G, C, pr, 64)) {
    set_error("pfa_router_topk_raw_ws: unsupported (x dtype %d, weight dtype %d, buffer dtype %d, G=%d, C=%d)",
              x_dtype, w_dtype, buf_dtype, G, C);
    return PFA_E_UNSUPPORTED;
  }
  if (n_tok == 0) return PFA_OK;
  const size_t need = (size_t)(2 * G + 1) * (size_t)n_tok * sizeof(float);
  PFA_CHECK_ARG(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace % 16) == 0,
                "pfa_router_topk_raw_ws: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                workspace_bytes);
  hipStream_t s = as_stream(stream);
  const RouterRaw raw{(const uint16_t*)w_router, (const uint16_t*)protos, pr ? (const uint16_t*)confidence : nullptr,
                      pr ? (const uint16_t*)usage : nullptr};
  float* rl = reinterpret_cast<float*>(workspace);
  const unsigned blocks = (unsigned)((n_tok + kRouterTok - 1) / kRouterTok);
  const unsigned mb = (blocks + kRmWaves - 1) / kRmWaves;
  // XCD-aware 1-D grid (router_mfma_kernel's DOTS mapping): whole slots of
  // the eight XCDs, each slot the gate blocks of one token group
  const dim3 gd((unsigned)(((mb + 7) / 8) * 8 * ((G + 15) / 16)));
  // 16-gate blocks: logits, prototype dots and sums of squares into rl
  if (pr)
    router_mfma_kernel<16, true, true, true><<<gd, 64 * kRmWaves, (size_t)rm_lds_bytes(C, 16, true), s>>>(
        (const uint16_t*)x, n_tok, C, G, nullptr, nullptr, nullptr, gate_to_head, H, topk, proto_temp,
        proto_threshold, proto_blend, usage_boost, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
        nullptr, raw, rl);
  else
    router_mfma_kernel<16, false, true, true><<<gd, 64 * kRmWaves, (size_t)rm_lds_bytes(C, 16, false), s>>>(
        (const uint16_t*)x, n_tok, C, G, nullptr, nullptr, nullptr, gate_to_head, H, topk, proto_temp,
        proto_threshold, proto_blend, usage_boost, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
        nullptr, raw, rl);
  PFA_CHECK_LAUNCH("pfa_router_topk_raw_ws/dots");
#define PFA_RE(GPV, PV)                                                                                          \
  router_epi_kernel<GPV, PV><<<mb, 64 * kRmWaves, (size_t)rm_epi_lds_bytes(GPV), s>>>(                        \
      (const uint16_t*)x, n_tok, C, G, rl, gate_to_head, H, topk, proto_temp, proto_threshold, proto_blend,      \
      usage_boost, gate_probs, sim, blend, importance, head_idx, head_score, stats_partial, ema_partial, raw)
  if (G <= 32) {
    if (pr) PFA_RE(32, true);
    else PFA_RE(32, false);
  } else {
    if (pr) PFA_RE(64, true);
    else PFA_RE(64, false);
  }
#undef PFA_RE
  PFA_CHECK_LAUNCH("pfa_router_topk_raw_ws/epilogue");
  return PFA_OK;
}

extern "C" int pfa_router_stats_reduce(const float* stats_partial, int n_blocks, double* out, void* stream) {
  clear_error();
  PFA_CHECK_ARG(stats_partial && out && n_blocks > 0, "pfa_router_stats_reduce: bad arguments");
  router_stats_reduce_kernel<<<1, 1024, 0, as_stream(stream)>>>(stats_partial, n_blocks, out);
  PFA_CHECK_LAUNCH("pfa_router_stats_reduce");
  return PFA_OK;
}

extern "C" int pfa_router_block_count(int64_t n_tok, int* n_blocks) {
  clear_error();
  PFA_CHECK_ARG(n_blocks != nullptr && n_tok >= 0, "pfa_router_block_count: bad arguments");
  *n_blocks = (int)((n_tok + kRouterTok - 1) / kRouterTok);
  return PFA_OK;
}

extern "C" int pfa_proto_partial_count(int64_t n_tok, int* n_parts) {
  clear_error();
  PFA_CHECK_ARG(n_parts != nullptr && n_tok >= 0, "pfa_proto_partial_count: bad arguments");
  int64_t parts = (n_tok + kEmaTok - 1) / kEmaTok;
  if (parts > kEmaMaxParts) parts = kEmaMaxParts;
  if (parts < 1) parts = 1;
  *n_parts = (int)parts;
  return PFA_OK;
}

extern "C" int pfa_proto_accumulate(const void* x, int x_dtype, int64_t n_tok, int C, int G,
                                    const float* gate_probs, float* partial, int n_parts, void* stream) {
  clear_error();
  PFA_CHECK_ARG(x && gate_probs && partial && n_parts > 0 && C > 0 && G > 0 && G <= 64,
                "pfa_proto_accumulate: bad arguments");
  hipStream_t s = as_stream(stream);
  int64_t per = (n_tok + n_parts - 1) / n_parts;
  if (per < 1) per = 1;
  switch (x_dtype) {
    case PFA_F32: launch_accum<PFA_F32>(x, n_tok, C, G, gate_probs, n_parts, per, partial, s); break;
    case PFA_BF16: launch_accum<PFA_BF16>(x, n_tok, C, G, gate_probs, n_parts, per, partial, s); break;
    case PFA_F16: launch_accum<PFA_F16>(x, n_tok, C, G, gate_probs, n_parts, per, partial, s); break;
    default:
      set_error("pfa_proto_accumulate: unsupported dtype %d", x_dtype);
      return PFA_E_UNSUPPORTED;
  }
  PFA_CHECK_LAUNCH("pfa_proto_accumulate");
  return PFA_OK;
}

extern "C" int pfa_proto_partial_reduce(float* partial, int n_parts, int G, int C, float* out, void* stream) {
  clear_error();
  PFA_CHECK_ARG(partial && out && n_parts > 0 && G > 0 && C > 0, "pfa_proto_partial_reduce: bad arguments");
  int64_t width = (int64_t)G * (C + 1);
  hipStream_t s = as_stream(stream);
  const unsigned cols = (unsigned)((width + 255) / 256);
  const int groups = (n_parts + kEmaGroup - 1) / kEmaGroup;
  partial_reduce_group<<<dim3(cols, (unsigned)groups), 256, 0, s>>>(partial, n_parts, width);
  PFA_CHECK_LAUNCH("pfa_proto_partial_reduce");
  partial_reduce_final<<<cols, 256, 0, s>>>(partial, groups, width, out);
  PFA_CHECK_LAUNCH("pfa_proto_partial_reduce");
  return PFA_OK;
}

extern "C" int pfa_proto_ema_update(const float* sums, int G, int C, float decay, void* protos, void* usage,
                                    void* confidence, int dtype, void* stream) {
  clear_error();
  PFA_CHECK_ARG(sums && protos && usage && confidence && G > 0 && C > 0, "pfa_proto_ema_update: bad arguments");
  int64_t n = (int64_t)G * C;
  unsigned blocks = (unsigned)((n + 255) / 256);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case PFA_F32:
      proto_ema_update_kernel<PFA_F32><<<blocks, 256, 0, s>>>(sums, G, C, decay, (float*)protos, (float*)usage,
                                                               (float*)confidence);
      break;
    case PFA_BF16:
      proto_ema_update_kernel<PFA_BF16><<<blocks, 256, 0, s>>>(sums, G, C, decay, (uint16_t*)protos,
                                                                (uint16_t*)usage, (uint16_t*)confidence);
      break;
    case PFA_F16:
      proto_ema_update_kernel<PFA_F16><<<blocks, 256, 0, s>>>(sums, G, C, decay, (uint16_t*)protos,
                                                               (uint16_t*)usage, (uint16_t*)confidence);
      break;
    default:
      set_error("pfa_proto_ema_update: unsupported dtype %d", dtype);
      return PFA_E_UNSUPPORTED;
  }
  PFA_CHECK_LAUNCH("pfa_proto_ema_update");
  return PFA_OK;
}
