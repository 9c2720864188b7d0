// Router: per-token gate probabilities, prototype prior, importance and
// head top-k, plus the partial sums of the prototype EMA update.
//
// Mapping: one lane per token.  Router weights and normalised prototypes
// are staged once per workgroup in LDS as f32, interleaved per channel
// (lds[c][0..G) = W[:, c], lds[c][G..2G) = P[:, c]) so that every lane of a
// wave reads the same LDS words (broadcast, no bank conflicts) while it
// streams its own token row from HBM with 16-byte loads.
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

constexpr int kRouterThreads = 256;
constexpr int kRouterLdsBytes = 64 * 1024;

template <int DT, int GMAX, bool LDS>
__global__ void __launch_bounds__(kRouterThreads)
router_kernel(const typename Elem<DT>::T* __restrict__ x, int64_t n_tok, int C, int G,
              const typename Elem<DT>::T* __restrict__ w_router, const float* __restrict__ proto_norm,
              const float* __restrict__ conf_weight, const float* __restrict__ usage_bias,
              const int32_t* __restrict__ gate_to_head, int H, int topk, float proto_temp,
              float proto_threshold, float proto_blend, float usage_boost, float* __restrict__ gate_probs,
              float* __restrict__ sim_out, float* __restrict__ blend_out, float* __restrict__ importance,
              int32_t* __restrict__ head_idx, float* __restrict__ head_score) {
  extern __shared__ float lds_w[];  // [C][2G]
  const bool use_proto = proto_norm != nullptr;
  const int G2 = 2 * G;
  if constexpr (LDS) {
    for (int i = threadIdx.x; i < C * G; i += blockDim.x) {
      int g = i / C, c = i % C;
      lds_w[c * G2 + g] = load_f<DT>(w_router + i);
      lds_w[c * G2 + G + g] = use_proto ? proto_norm[i] : 0.f;
    }
    __syncthreads();
  }

  for (int64_t tok = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;; tok += (int64_t)gridDim.x * blockDim.x) {
    // Uniform loop exit per workgroup is not required (no barriers below).
    if (tok >= n_tok) break;
    const typename Elem<DT>::T* xr = x + tok * C;
    float logit[GMAX], dotp[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) { logit[g] = 0.f; dotp[g] = 0.f; }
    float sq = 0.f;

    auto accum = [&](int c, float xv) {
      sq = __builtin_fmaf(xv, xv, sq);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G) {
          float wv, pv;
          if constexpr (LDS) { wv = lds_w[c * G2 + g]; pv = lds_w[c * G2 + G + g]; }
          else {
            wv = load_f<DT>(w_router + (int64_t)g * C + c);
            pv = use_proto ? proto_norm[(int64_t)g * C + c] : 0.f;
          }
          logit[g] = __builtin_fmaf(xv, wv, logit[g]);
          dotp[g] = __builtin_fmaf(xv, pv, dotp[g]);
        }
      }
    };

    if ((C % 8) == 0 && (DT != PFA_F32 || true)) {
      for (int c0 = 0; c0 < C; c0 += 8) {
        float xv[8];
        load8<DT>(xr + c0, xv);
#pragma unroll
        for (int j = 0; j < 8; ++j) accum(c0 + j, xv[j]);
      }
    } else {
      for (int c = 0; c < C; ++c) accum(c, load_f<DT>(xr + c));
    }

    // --- SwitchRouter: logits in x dtype, softmax in f32 rounded to x dtype.
    float gate[GMAX];
    float lmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) { logit[g] = round_to<DT>(logit[g]); lmax = fmaxf(lmax, logit[g]); }
    float lsum = 0.f;
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) { gate[g] = expf(logit[g] - lmax); lsum = lsum + gate[g]; }
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) gate[g] = round_to<DT>(gate[g] / lsum);

    float sim_max = 0.f, blend_scalar = 0.f;
    if (use_proto) {
      float nrm = sqrtf(sq);
      float inv_den = fmaxf(nrm, 1e-6f);
      float sims[GMAX];
      sim_max = -INFINITY;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) { sims[g] = dotp[g] / inv_den; sim_max = fmaxf(sim_max, sims[g]); }
      // proto_probs = softmax(sims / temp)
      float pp[GMAX];
      float smax = -INFINITY;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) { pp[g] = sims[g] / proto_temp; smax = fmaxf(smax, pp[g]); }
      float ssum = 0.f;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) { pp[g] = expf(pp[g] - smax); ssum = ssum + pp[g]; }
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) pp[g] = pp[g] / ssum;
      float den = fmaxf(1e-6f, 1.0f - proto_threshold);
      blend_scalar = fminf(fmaxf((sim_max - proto_threshold) / den, 0.f), 1.f);
      if (conf_weight != nullptr) {
        float cs = 0.f;
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) { pp[g] = pp[g] * conf_weight[g]; cs = cs + pp[g]; }
        cs = fmaxf(cs, 1e-6f);
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) pp[g] = pp[g] / cs;
      }
      float blend = proto_blend * blend_scalar;
      float one_m = 1.0f - blend;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) gate[g] = gate[g] * one_m + pp[g] * blend;
      if (usage_bias != nullptr && usage_boost > 0.f) {
        float scale_u = (1.0f - blend_scalar) * usage_boost;
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) gate[g] = gate[g] + usage_bias[g] * scale_u;
      }
      float gs = 0.f;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) { gate[g] = fmaxf(gate[g], 0.f); gs = gs + gate[g]; }
      gs = fmaxf(gs, 1e-6f);
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) gate[g] = gate[g] / gs;
    }

    float gmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) gmax = fmaxf(gmax, gate[g]);
    float imp = use_proto ? (gmax * (1.0f - blend_scalar) + sim_max * blend_scalar) : gmax;

    if (gate_probs) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) gate_probs[tok * G + g] = gate[g];
    }
    if (sim_out) sim_out[tok] = sim_max;
    if (blend_out) blend_out[tok] = blend_scalar;
    importance[tok] = imp;

    // head_probs = gate_probs @ onehot(gate_to_head); top-k (ties -> lower head).
    float hp[GMAX];
#pragma unroll
    for (int h = 0; h < GMAX; ++h) hp[h] = 0.f;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G) {
        int hg = gate_to_head[g];
#pragma unroll
        for (int h = 0; h < GMAX; ++h)
          if (h == hg) hp[h] = hp[h] + gate[g];
      }
    }
    uint64_t taken = 0;
    for (int j = 0; j < topk; ++j) {
      float bv = 0.f;
      int bi = -1;
#pragma unroll
      for (int h = 0; h < GMAX; ++h) {
        if (h < H && !((taken >> h) & 1ull)) {
          if (bi < 0 || better(hp[h], h, bv, bi)) { bv = hp[h]; bi = h; }
        }
      }
      taken |= 1ull << bi;
      head_idx[tok * topk + j] = bi;
      if (head_score) head_score[tok * topk + j] = bv;
    }
  }
}

// Prototype EMA partial sums: part p accumulates, for a contiguous slice of
// tokens, sum_t gate[t,g]*x[t,c] (columns 0..C-1) and sum_t gate[t,g]
// (column C).  Threads stride over channels so x rows are read coalesced.
constexpr int kEmaThreads = 256;
constexpr int kEmaMaxParts = 1024;

template <int DT, int GMAX>
__global__ void __launch_bounds__(kEmaThreads)
proto_accum_kernel(const typename Elem<DT>::T* __restrict__ x, int64_t n_tok, int C, int G,
                   const float* __restrict__ gate_probs, int64_t tok_per_part, float* __restrict__ partial) {
  const int part = blockIdx.x;
  const int64_t t0 = (int64_t)part * tok_per_part;
  const int64_t t1 = min(n_tok, t0 + tok_per_part);
  float* out = partial + (int64_t)part * G * (C + 1);
  for (int c = threadIdx.x; c <= C; c += blockDim.x) {
    float acc[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) acc[g] = 0.f;
    for (int64_t t = t0; t < t1; ++t) {
      float xv = (c < C) ? load_f<DT>(x + t * C + c) : 1.0f;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) acc[g] = __builtin_fmaf(gate_probs[t * G + g], xv, acc[g]);
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) out[(int64_t)g * (C + 1) + c] = acc[g];
  }
}

__global__ void partial_reduce_kernel(const float* __restrict__ partial, int n_parts, int64_t width,
                                      float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= width) return;
  float s = 0.f;
  for (int p = 0; p < n_parts; ++p) s = s + partial[(int64_t)p * width + i];
  out[i] = s;
}

template <int DT>
static int launch_router(const void* x, int64_t n_tok, int C, int G, const void* w, const float* pn,
                         const float* cw, const float* ub, const int32_t* g2h, int H, int topk, float temp,
                         float thr, float pb, float boost, float* gp, float* sim, float* bl, float* imp,
                         int32_t* hi, float* hs, hipStream_t s) {
  using ET = typename Elem<DT>::T;
  size_t lds = (size_t)C * 2 * G * sizeof(float);
  bool use_lds = lds <= (size_t)kRouterLdsBytes;
  int64_t blocks = (n_tok + kRouterThreads - 1) / kRouterThreads;
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
#define PFA_ROUTER_LAUNCH(GM)                                                                          \
  do {                                                                                                 \
    if (use_lds)                                                                                       \
      router_kernel<DT, GM, true><<<(unsigned)blocks, kRouterThreads, lds, s>>>(                       \
          (const ET*)x, n_tok, C, G, (const ET*)w, pn, cw, ub, g2h, H, topk, temp, thr, pb, boost, gp, \
          sim, bl, imp, hi, hs);                                                                       \
    else                                                                                               \
      router_kernel<DT, GM, false><<<(unsigned)blocks, kRouterThreads, 0, s>>>(                        \
          (const ET*)x, n_tok, C, G, (const ET*)w, pn, cw, ub, g2h, H, topk, temp, thr, pb, boost, gp, \
          sim, bl, imp, hi, hs);                                                                       \
  } while (0)
  if (G <= 8) PFA_ROUTER_LAUNCH(8);
  else if (G <= 16) PFA_ROUTER_LAUNCH(16);
  else if (G <= 32) PFA_ROUTER_LAUNCH(32);
  else PFA_ROUTER_LAUNCH(64);
#undef PFA_ROUTER_LAUNCH
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

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_router_topk(const void* x, int x_dtype, int64_t n_tok, int C, int G, const void* w_router,
                               const float* proto_norm, const float* conf_weight, const float* usage_bias,
                               const int32_t* gate_to_head, int H, int topk, float proto_temp,
                               float proto_threshold, float proto_blend, float usage_boost, float* gate_probs,
                               float* sim, float* blend, float* importance, int32_t* head_idx, float* head_score,
                               void* stream) {
  clear_error();
  PFA_CHECK_ARG(n_tok >= 0 && C > 0 && G > 0 && G <= 64 && H > 0 && H <= G && topk >= 1 && topk <= H,
                "pfa_router_topk: bad sizes n_tok=%lld C=%d G=%d H=%d topk=%d", (long long)n_tok, C, G, H, topk);
  PFA_CHECK_ARG(x && w_router && gate_to_head && importance && head_idx, "pfa_router_topk: null pointer");
  if (n_tok == 0) return PFA_OK;
  hipStream_t s = as_stream(stream);
  switch (x_dtype) {
    case PFA_F32:
      return launch_router<PFA_F32>(x, n_tok, C, G, w_router, proto_norm, conf_weight, usage_bias, gate_to_head, H,
                                    topk, proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim,
                                    blend, importance, head_idx, head_score, s);
    case PFA_BF16:
      return launch_router<PFA_BF16>(x, n_tok, C, G, w_router, proto_norm, conf_weight, usage_bias, gate_to_head,
                                     H, topk, proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim,
                                     blend, importance, head_idx, head_score, s);
    case PFA_F16:
      return launch_router<PFA_F16>(x, n_tok, C, G, w_router, proto_norm, conf_weight, usage_bias, gate_to_head, H,
                                    topk, proto_temp, proto_threshold, proto_blend, usage_boost, gate_probs, sim,
                                    blend, importance, head_idx, head_score, s);
    default:
      set_error("pfa_router_topk: unsupported dtype %d", x_dtype);
      return PFA_E_UNSUPPORTED;
  }
}

extern "C" int pfa_proto_partial_count(int64_t n_tok, int* n_parts) {
  clear_error();
  PFA_CHECK_ARG(n_parts != nullptr && n_tok >= 0, "pfa_proto_partial_count: bad arguments");
  int64_t parts = (n_tok + 255) / 256;
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

extern "C" int pfa_proto_partial_reduce(const float* partial, int n_parts, int G, int C, float* out, void* stream) {
  clear_error();
  PFA_CHECK_ARG(partial && out && n_parts > 0 && G > 0 && C > 0, "pfa_proto_partial_reduce: bad arguments");
  int64_t width = (int64_t)G * (C + 1);
  partial_reduce_kernel<<<(unsigned)((width + 255) / 256), 256, 0, as_stream(stream)>>>(partial, n_parts, width, out);
  PFA_CHECK_LAUNCH("pfa_proto_partial_reduce");
  return PFA_OK;
}
