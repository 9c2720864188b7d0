// Library plumbing: version, thread-local error string, zero fill, RoPE.
#include <cstdarg>
#include <cstdio>

#include "pfa_common.h"

// Elementwise RoPE arithmetic must round each product separately.
#pragma clang fp contract(off)

namespace pfa {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

// Vector-store zero fill: 16 bytes per lane per step, grid-stride.
__global__ void __launch_bounds__(256) zero_fill_kernel(uint4* p, size_t n16) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t step = (size_t)gridDim.x * blockDim.x;
  for (; i < n16; i += step) p[i] = make_uint4(0, 0, 0, 0);
}
__global__ void zero_fill_tail(uint8_t* p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// RoPE in place on the q and k thirds of a (B, T, 3, H, D) buffer.  One
// thread rotates 4 (even, odd) pairs = 8 consecutive elements of one head of
// q or k (16-byte loads of x, cos and sin):
//   out_even = r(r(x_e*cos_e) + r(-x_o*sin_e)),  out_odd = r(r(x_o*cos_o) + r(x_e*sin_o))
// where r() rounds to the tensor dtype, matching q*cos + rotate_half(q)*sin
// evaluated as three elementwise ops in that dtype.  D must be a multiple
// of 8 (the host falls back to the per-pair kernel otherwise).
template <int DT>
__global__ void __launch_bounds__(256) rope8_kernel(typename Elem<DT>::T* qkv, int64_t n_groups, int64_t T, int H,
                                                    int D, const typename Elem<DT>::T* cos_tab,
                                                    const typename Elem<DT>::T* sin_tab, int nparts) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_groups) return;
  const int per_head = D / 8;
  const int C = H * D;
  int64_t gidx = i % per_head;
  int64_t rest = i / per_head;
  int h = (int)(rest % H);
  rest /= H;
  int which = (int)(rest % nparts) + (2 - nparts);  // 0 = q, 1 = k (k only when nparts == 1)
  int64_t bt = rest / nparts;
  int64_t t = bt % T;
  typename Elem<DT>::T* base = qkv + bt * (3 * (int64_t)C) + which * C + h * D + 8 * gidx;
  float xv[8], cv[8], sv[8], o[8];
  load8<DT>(base, xv);
  load8<DT>(cos_tab + t * D + 8 * gidx, cv);
  load8<DT>(sin_tab + t * D + 8 * gidx, sv);
  rope_rotate8<DT>(xv, cv, sv, o);
  store8<DT>(base, o);
}

// Token-row variant for D = 64: a token row has nparts*H*8 groups of 8
// elements (q heads, then k heads; k heads only when nparts == 1), which
// share one table row.  A 256-thread workgroup rotates 256 / groups whole
// rows (one row, looping, when a row has more groups than threads).  Index
// math is shifts and one compare per group (no 64-bit division per element).
// zout (k only, or null): the (rows, H*64) attention output, whose row bt
// gets zeros from the same threads (group e writes elements 8e .. 8e+7).
template <int DT>
__global__ void __launch_bounds__(256) rope64_row_kernel(typename Elem<DT>::T* qkv, int64_t rows, int64_t T,
                                                         int H, const typename Elem<DT>::T* cos_tab,
                                                         const typename Elem<DT>::T* sin_tab, int nparts,
                                                         typename Elem<DT>::T* zout) {
  const int groups = nparts * H * 8;
  const bool wide = groups >= 256;
  const int rpw = wide ? 1 : 256 / groups;
  const int sub = wide ? 0 : (int)threadIdx.x / groups;
  if (sub >= rpw) return;
  const int64_t bt = (int64_t)blockIdx.x * rpw + sub;
  if (bt >= rows) return;
  const int64_t t = (int64_t)((uint32_t)bt % (uint32_t)T);  // rows < 2^31 (host check)
  const int C = H * 64;
  typename Elem<DT>::T* row = qkv + bt * (3 * (int64_t)C);
  const int hw0 = (2 - nparts) * H;  // k heads only when nparts == 1
  const int e0 = wide ? (int)threadIdx.x : (int)threadIdx.x - sub * groups;
  const int step = wide ? (int)blockDim.x : groups;
  for (int e = e0; e < groups; e += step) {
    const int g8 = e & 7;           // 8-element group within the head
    const int hw = hw0 + (e >> 3);  // q head hw, or k head hw - H
    const int off = (hw >= H ? C + (hw - H) * 64 : hw * 64) + 8 * g8;
    float xv[8], cv[8], sv[8], o[8];
    load8<DT>(row + off, xv);
    load8<DT>(cos_tab + t * 64 + 8 * g8, cv);
    load8<DT>(sin_tab + t * 64 + 8 * g8, sv);
    rope_rotate8<DT>(xv, cv, sv, o);
    store8<DT>(row + off, o);
    if (zout != nullptr) {
      const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      store8<DT>(zout + bt * (int64_t)C + 8 * e, z);
    }
  }
}

// Per-pair variant for head dims that are not a multiple of 8.
template <int DT>
__global__ void __launch_bounds__(256) rope_kernel(typename Elem<DT>::T* qkv, int64_t n_pairs, int64_t T,
                                                   int H, int D, const typename Elem<DT>::T* cos_tab,
                                                   const typename Elem<DT>::T* sin_tab, int nparts) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_pairs) return;
  const int half = D / 2;
  const int C = H * D;
  int64_t pair = i % half;
  int64_t rest = i / half;
  int h = (int)(rest % H);
  rest /= H;
  int which = (int)(rest % nparts) + (2 - nparts);  // 0 = q, 1 = k (k only when nparts == 1)
  int64_t bt = rest / nparts;
  int64_t t = bt % T;
  typename Elem<DT>::T* base = qkv + bt * (3 * (int64_t)C) + which * C + h * D + 2 * pair;
  float xe = load_f<DT>(base), xo = load_f<DT>(base + 1);
  float ce = load_f<DT>(cos_tab + t * D + 2 * pair), co = load_f<DT>(cos_tab + t * D + 2 * pair + 1);
  float se = load_f<DT>(sin_tab + t * D + 2 * pair), so = load_f<DT>(sin_tab + t * D + 2 * pair + 1);
  float e = round_to<DT>(round_to<DT>(xe * ce) + round_to<DT>(-xo * se));
  float o = round_to<DT>(round_to<DT>(xo * co) + round_to<DT>(xe * so));
  store_f<DT>(base, e);
  store_f<DT>(base + 1, o);
}

}  // namespace pfa

using namespace pfa;

extern "C" int pfa_version(void) { return 100; }

extern "C" const char* pfa_last_error_string(void) { return g_last_error.c_str(); }

extern "C" int pfa_zero_fill(void* ptr, size_t bytes, void* stream) {
  clear_error();
  if (bytes == 0) return PFA_OK;
  PFA_CHECK_ARG(ptr != nullptr, "pfa_zero_fill: null pointer");
  hipStream_t s = as_stream(stream);
  size_t head_pad = (16 - ((uintptr_t)ptr & 15)) & 15;
  if (head_pad > bytes) head_pad = bytes;
  if (head_pad) {
    zero_fill_tail<<<1, 16, 0, s>>>((uint8_t*)ptr, head_pad);
    PFA_CHECK_LAUNCH("pfa_zero_fill");
  }
  uint8_t* body = (uint8_t*)ptr + head_pad;
  size_t rem = bytes - head_pad;
  size_t n16 = rem / 16;
  if (n16) {
    size_t blocks = (n16 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    zero_fill_kernel<<<(unsigned)blocks, 256, 0, s>>>((uint4*)body, n16);
    PFA_CHECK_LAUNCH("pfa_zero_fill");
  }
  size_t tail = rem - n16 * 16;
  if (tail) {
    zero_fill_tail<<<1, 16, 0, s>>>(body + n16 * 16, tail);
    PFA_CHECK_LAUNCH("pfa_zero_fill");
  }
  return PFA_OK;
}

// zero_out (k only, or null): a (B, T, H*D) output to fill with zeros in the
// same pass (D = 64 row kernel) or by pfa_zero_fill after it.
static int rope_inplace_impl(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                             const void* sin_tab, int nparts, void* stream, void* zero_out, bool* zeroed);
static int rope_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                        const void* sin_tab, int nparts, void* stream, void* zero_out = nullptr) {
  bool zeroed = false;
  const int rc = rope_inplace_impl(qkv, dtype, B, T, H, D, cos_tab, sin_tab, nparts, stream, zero_out, &zeroed);
  if (rc != PFA_OK || zero_out == nullptr || zeroed) return rc;
  const size_t esz = dtype == PFA_F32 ? 4 : 2;
  return pfa_zero_fill(zero_out, (size_t)B * (size_t)T * (size_t)H * (size_t)D * esz, stream);
}
static int rope_inplace_impl(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                             const void* sin_tab, int nparts, void* stream, void* zero_out, bool* zeroed) {
  PFA_CHECK_ARG(qkv && cos_tab && sin_tab, "pfa_rope_qk_inplace: null pointer");
  PFA_CHECK_ARG(zero_out == nullptr || nparts == 1, "pfa_rope_qk_inplace: the zero output goes with k only");
  PFA_CHECK_ARG(B >= 0 && T >= 0 && H > 0 && D > 0 && D % 2 == 0,
                "pfa_rope_qk_inplace: bad shape B=%d T=%lld H=%d D=%d", B, (long long)T, H, D);
  hipStream_t s = as_stream(stream);
  const bool vec = (D % 8) == 0 && ((uintptr_t)qkv % 16) == 0 && ((uintptr_t)cos_tab % 16) == 0 &&
                   ((uintptr_t)sin_tab % 16) == 0;
  const bool zvec = zero_out == nullptr || ((uintptr_t)zero_out % 16) == 0;
  if (vec && zvec && D == 64 && (int64_t)B * T < INT32_MAX && H <= 256) {
    const int64_t rows = (int64_t)B * T;
    if (rows == 0) return PFA_OK;
    const int groups = nparts * H * 8;
    const int64_t rpw = groups >= 256 ? 1 : 256 / groups;
    const unsigned threads = 256;
    const unsigned nblk = (unsigned)((rows + rpw - 1) / rpw);
    switch (dtype) {
      case PFA_F32:
        rope64_row_kernel<PFA_F32><<<nblk, threads, 0, s>>>((float*)qkv, rows, T, H, (const float*)cos_tab,
                                                                      (const float*)sin_tab, nparts,
                                                                      (float*)zero_out);
        break;
      case PFA_BF16:
        rope64_row_kernel<PFA_BF16><<<nblk, threads, 0, s>>>((uint16_t*)qkv, rows, T, H, (const uint16_t*)cos_tab,
                                                                       (const uint16_t*)sin_tab, nparts,
                                                                       (uint16_t*)zero_out);
        break;
      case PFA_F16:
        rope64_row_kernel<PFA_F16><<<nblk, threads, 0, s>>>((uint16_t*)qkv, rows, T, H, (const uint16_t*)cos_tab,
                                                                      (const uint16_t*)sin_tab, nparts,
                                                                      (uint16_t*)zero_out);
        break;
      default:
        set_error("pfa_rope_qk_inplace: unsupported dtype %d", dtype);
        return PFA_E_UNSUPPORTED;
    }
    PFA_CHECK_LAUNCH("pfa_rope_qk_inplace");
    *zeroed = true;
    return PFA_OK;
  }
  if (vec) {
    int64_t n_groups = (int64_t)B * T * nparts * H * (D / 8);
    if (n_groups == 0) return PFA_OK;
    unsigned blocks = (unsigned)((n_groups + 255) / 256);
    switch (dtype) {
      case PFA_F32:
        rope8_kernel<PFA_F32><<<blocks, 256, 0, s>>>((float*)qkv, n_groups, T, H, D, (const float*)cos_tab,
                                                      (const float*)sin_tab, nparts);
        break;
      case PFA_BF16:
        rope8_kernel<PFA_BF16><<<blocks, 256, 0, s>>>((uint16_t*)qkv, n_groups, T, H, D,
                                                       (const uint16_t*)cos_tab, (const uint16_t*)sin_tab, nparts);
        break;
      case PFA_F16:
        rope8_kernel<PFA_F16><<<blocks, 256, 0, s>>>((uint16_t*)qkv, n_groups, T, H, D,
                                                      (const uint16_t*)cos_tab, (const uint16_t*)sin_tab, nparts);
        break;
      default:
        set_error("pfa_rope_qk_inplace: unsupported dtype %d", dtype);
        return PFA_E_UNSUPPORTED;
    }
    PFA_CHECK_LAUNCH("pfa_rope_qk_inplace");
    return PFA_OK;
  }
  int64_t n_pairs = (int64_t)B * T * nparts * H * (D / 2);
  if (n_pairs == 0) return PFA_OK;
  unsigned blocks = (unsigned)((n_pairs + 255) / 256);
  switch (dtype) {
    case PFA_F32:
      rope_kernel<PFA_F32><<<blocks, 256, 0, s>>>((float*)qkv, n_pairs, T, H, D, (const float*)cos_tab,
                                                   (const float*)sin_tab, nparts);
      break;
    case PFA_BF16:
      rope_kernel<PFA_BF16><<<blocks, 256, 0, s>>>((uint16_t*)qkv, n_pairs, T, H, D,
                                                    (const uint16_t*)cos_tab, (const uint16_t*)sin_tab, nparts);
      break;
    case PFA_F16:
      rope_kernel<PFA_F16><<<blocks, 256, 0, s>>>((uint16_t*)qkv, n_pairs, T, H, D,
                                                   (const uint16_t*)cos_tab, (const uint16_t*)sin_tab, nparts);
      break;
    default:
      set_error("pfa_rope_qk_inplace: unsupported dtype %d", dtype);
      return PFA_E_UNSUPPORTED;
  }
  PFA_CHECK_LAUNCH("pfa_rope_qk_inplace");
  return PFA_OK;
}

extern "C" int pfa_rope_qk_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                                   const void* sin_tab, void* stream) {
  clear_error();
  return rope_inplace(qkv, dtype, B, T, H, D, cos_tab, sin_tab, 2, stream);
}

extern "C" int pfa_rope_k_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                                  const void* sin_tab, void* stream) {
  clear_error();
  return rope_inplace(qkv, dtype, B, T, H, D, cos_tab, sin_tab, 1, stream);
}

extern "C" int pfa_rope_k_zero_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D, const void* cos_tab,
                                       const void* sin_tab, void* zero_out, void* stream) {
  clear_error();
  PFA_CHECK_ARG(zero_out != nullptr, "pfa_rope_k_zero_inplace: null output");
  return rope_inplace(qkv, dtype, B, T, H, D, cos_tab, sin_tab, 1, stream, zero_out);
}
