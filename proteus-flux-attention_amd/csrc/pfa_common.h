// Shared device helpers and host-side error plumbing for libpfa_hip.so.
// gfx950 (CDNA4) only: wave64, 160 KiB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string>

#include "../../include/pfa_hip.h"

namespace pfa {

constexpr int kWave = 64;

// ---------------------------------------------------------------------
// Host: error reporting.  The message lives in a thread-local string so
// that concurrent callers on different threads do not overwrite it.
// ---------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define PFA_CHECK_ARG(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      ::pfa::set_error(__VA_ARGS__);      \
      return PFA_E_INVALID;               \
    }                                     \
  } while (0)

#define PFA_CHECK_LAUNCH(what)                                              \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess) {                                                 \
      ::pfa::set_error("%s: launch failed: %s", what, hipGetErrorString(_e)); \
      return (int)_e;                                                       \
    }                                                                       \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------
// Device: scalar conversions.  bf16 is handled as raw uint16 bits.
// f32 -> bf16 rounds to nearest even (NaN kept quiet).
// ---------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __half_as_ushort(__float2half(f));
}

// Round a float to the precision of a storage type and back (emulates an
// elementwise op whose result tensor has that dtype).
template <int DT>
__device__ __forceinline__ float round_to(float f) {
  if constexpr (DT == PFA_BF16) return bf16_to_f32(f32_to_bf16(f));
  else if constexpr (DT == PFA_F16) return f16_to_f32(f32_to_f16(f));
  else return f;
}

template <int DT> struct Elem;
template <> struct Elem<PFA_F32> { using T = float; };
template <> struct Elem<PFA_BF16> { using T = uint16_t; };
template <> struct Elem<PFA_F16> { using T = uint16_t; };
template <> struct Elem<PFA_I8> { using T = int8_t; };

template <int DT>
__device__ __forceinline__ float load_f(const typename Elem<DT>::T* p) {
  if constexpr (DT == PFA_F32) return *p;
  else if constexpr (DT == PFA_BF16) return bf16_to_f32(*p);
  else if constexpr (DT == PFA_F16) return f16_to_f32(*p);
  else return (float)(*p);
}
template <int DT>
__device__ __forceinline__ void store_f(typename Elem<DT>::T* p, float f) {
  if constexpr (DT == PFA_F32) *p = f;
  else if constexpr (DT == PFA_BF16) *p = f32_to_bf16(f);
  else if constexpr (DT == PFA_F16) *p = f32_to_f16(f);
}

// Kernels on the forward's critical chain (router, packing, prototype
// tables) run beside the projection GEMM and the anchor pass, which are
// queued on another stream and fill the CUs; they raise their waves' issue
// priority (s_setprio: instruction arbitration within a SIMD only, no effect
// on dispatch order, memory or results).
#define PFA_CRITICAL_CHAIN_PRIORITY() __builtin_amdgcn_s_setprio(2)

// Maximum over the four lanes l, l^16, l^32, l^48 of a wave64 (the four
// 16-lane rows), with the gfx950 row-swap permutes (VALU, no LDS round
// trip): permlane32_swap pairs each lane with l^32 and permlane16_swap with
// l^16.
__device__ __forceinline__ float max_over_rows4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// RoPE on 8 consecutive elements (4 interleaved (even, odd) pairs):
//   o_e = r(r(x_e c_e) + r(-x_o s_e)),  o_o = r(r(x_o c_o) + r(x_e s_o))
// where r() rounds to the tensor dtype, matching q*cos + rotate_half(q)*sin
// evaluated as three elementwise ops in that dtype.  Shared by every kernel
// that rotates rows, so all of them produce the same bits.
// For bf16 the roundings use the hardware converter (v_cvt_pk_bf16_f32,
// round to nearest even: the same bits as round_to<PFA_BF16> for every
// non-NaN value; a NaN comes out as a NaN).
template <int DT>
__device__ __forceinline__ float rope_round(float f) {
  if constexpr (DT == PFA_BF16) return (float)(__bf16)f;
  else return round_to<DT>(f);
}

template <int DT>
__device__ __forceinline__ void rope_rotate8(const float (&xv)[8], const float (&cv)[8], const float (&sv)[8],
                                             float (&o)[8]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float xe = xv[2 * p], xo = xv[2 * p + 1];
    o[2 * p] = rope_round<DT>(rope_round<DT>(xe * cv[2 * p]) + rope_round<DT>(-xo * sv[2 * p]));
    o[2 * p + 1] = rope_round<DT>(rope_round<DT>(xo * cv[2 * p + 1]) + rope_round<DT>(xe * sv[2 * p + 1]));
  }
}

// Load 8 consecutive elements (d .. d+7) as floats; the address must be
// aligned to 8 elements.
template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::T* p, float (&o)[8]) {
  if constexpr (DT == PFA_F32) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else if constexpr (DT == PFA_BF16) {
    uint4 a = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else if constexpr (DT == PFA_F16) {
    uint4 a = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
      o[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
  } else {
    uint2 a = *reinterpret_cast<const uint2*>(p);
    uint32_t w[2] = {a.x, a.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o[i] = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xffu);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(typename Elem<DT>::T* p, const float (&v)[8]) {
  if constexpr (DT == PFA_F32) {
    float4* q = reinterpret_cast<float4*>(p);
    q[0] = make_float4(v[0], v[1], v[2], v[3]);
    q[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint16_t lo, hi;
      if constexpr (DT == PFA_BF16) { lo = f32_to_bf16(v[2 * i]); hi = f32_to_bf16(v[2 * i + 1]); }
      else { lo = f32_to_f16(v[2 * i]); hi = f32_to_f16(v[2 * i + 1]); }
      w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Orders LDS/global accesses of the lanes of one wave (a wave-local barrier;
// kernels that keep per-wave LDS regions use it instead of __syncthreads).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Order used by every top-k in this library: larger value first, equal
// values -> smaller index first.  NaN compares as smaller than anything
// else (two NaNs: smaller index first), so the order is strict and total.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return (va > vb) || (va == vb && ia < ib) || (vb != vb && (va == va || ia < ib));
}

// ---- LDS DMA tiles (shared by the attention passes and the linear kernel) --
// Swizzle of unpadded 128-byte LDS rows: the 16-byte chunk c of row r sits in
// chunk slot 8r + (c ^ tile_swz(r)).  Eight consecutive rows read at one chunk
// fall in eight bank groups, and so do four rows x 32 bytes of a transpose
// read.
__device__ __forceinline__ int tile_swz(int r) {
  return (((r & 3) << 1) | ((r >> 2) & 1)) ^ (((r >> 3) & 1) << 1);
}

// LDS DMA of 16 bytes per lane: lane l's bytes from g land at LDS byte
// address lds_wave + 16*l (lds_wave is the same for the whole wave).
// Written as assembly so that the compiler does not wait for the transfer
// before every LDS read: completion is waited for explicitly
// (dma_wait_barrier).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// M0 is named as clobbered; no kernel of this library uses M0 otherwise (no
// LDS DMA builtins, GWS, message or relative-indexing instructions), so no
// value of the compiler's lives in it across the statement.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds_wave) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_wave) : "memory", "m0");
}
// The same from a wave-uniform 64-bit base (scalar registers) plus a 32-bit
// byte offset per lane: no 64-bit address in vector registers.
__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t off, uint32_t lds_wave) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_wave)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// Wait until at most N of this wave's vector memory operations are
// outstanding and its LDS reads are done, then meet the other waves.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// ---- 64-key K/V tiles in LDS for the bf16 MFMA attention kernels --------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// Four bf16 of one head dim from four consecutive key rows of a V tile, by
// the gfx950 LDS transpose read: within each 16-lane row of the wave, lane
// 4a+b receives element b of the 8-byte chunks addressed by lanes a, a+4,
// a+8, a+12.  Lane m of the row addresses key row0 + m/4, dims
// d0 + 4*(m%4) .. +3, so lane i = 4a+b gets V[row0 + k][d0 + i], k = 0..3.
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4_t;
__device__ __forceinline__ i16x4_t ds_tr4(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(p));
}

// A 64-key tile (K and V, 64 x 64 bf16 each) in LDS gives the MFMA
// fragments through two calls: kfrag(kb, dc) is the lane's 8 K elements
// (key 16kb + lane%16, dims 32dc + 8*(lane/16) ..+7) and vtr(kc, h, db) the
// address the lane passes to the transpose read for keys
// 32kc + 16h + 4*(lane/16) .. +3, dims 16db ..+15.
//
// SwzTile: unpadded 128-byte rows filled by LDS DMA (global_load_lds, 16
// bytes per lane at consecutive LDS addresses).  The 16-byte chunk c of key
// row r (dims 8c..8c+7) sits in chunk slot 8r + (c ^ tile_swz(r)): eight
// consecutive rows read at one chunk (the K fragments) fall in eight
// different bank groups, and so do the four rows x 32 bytes of each
// transpose read.
constexpr int kSwzKeys = 64;                      // keys of a swizzled tile
constexpr int kSwzTileElems = kSwzKeys * 64;      // one unpadded K or V tile, bf16 elements
// per-lane element offsets into a SwzTile, fixed for the kernel
struct SwzLane {
  int ko[2];  // K fragment, dc = 0, 1 (plus 1024 * kb)
  int vo[4];  // transpose read, db = 0..3 (plus 64 * (32kc + 16h))
  __device__ __forceinline__ void init() {
    const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
    const int c0 = g ^ tile_swz(r16);
    ko[0] = r16 * 64 + 8 * c0;
    ko[1] = r16 * 64 + 8 * (c0 ^ 4);
    const int m = r16, row = 4 * g + (m >> 2);
    const int cv = ((m & 3) >> 1) ^ tile_swz(row);
#pragma unroll
    for (int db = 0; db < 4; ++db) vo[db] = row * 64 + 8 * ((2 * db) ^ cv) + 4 * (m & 1);
  }
};
struct SwzTile {
  const uint16_t* base;  // K tile, V tile at base + kSwzTileElems
  const SwzLane& L;
  __device__ __forceinline__ const uint16_t* kfrag(int kb, int dc) const { return base + 1024 * kb + L.ko[dc]; }
  __device__ __forceinline__ const uint16_t* vtr(int kc, int h, int db) const {
    return base + kSwzTileElems + 64 * (32 * kc + 16 * h) + L.vo[db];
  }
};

// One 64-key tile by DMA into a SwzTile (256 threads): thread tid moves chunk
// slot tid%8 of key rows tid/8 and tid/8 + 32 (keys key0, key1) of K and of
// V: four 16-byte transfers, each wave filling 1 KB runs of chunk slots.
// lds_w is the tile's LDS byte address plus 1 KB per wave index
// (wave-uniform); kb/vb are bf16 rows with token strides ks_t/vs_t.
// cmask (D/8 - 1 for rows of D <= 64 elements, a power of two): the chunk
// slots of logical chunks past D/8 receive source chunk (c & cmask), a
// finite copy of the row's own data that a zero q chunk cancels.
constexpr int kDmaPerTile = 4;
__device__ __forceinline__ void dma_tile(const uint16_t* __restrict__ kb, const uint16_t* __restrict__ vb,
                                         uint32_t ks_t, uint32_t vs_t, int key0, int key1, uint32_t lds_w,
                                         uint32_t cmask = 7u) {
  const int tid = threadIdx.x;
  const int c = 8 * (int)((uint32_t)((tid & 7) ^ tile_swz(tid >> 3)) & cmask);  // rows tid/8, tid/8 + 32: one swizzle
  // element offsets: one 32 x 32 -> 64-bit multiply each (keys and row
  // strides are below 2^31)
  const uint64_t k0 = (uint64_t)(uint32_t)key0 * ks_t, k1 = (uint64_t)(uint32_t)key1 * ks_t;
  const uint64_t v0 = (uint64_t)(uint32_t)key0 * vs_t, v1 = (uint64_t)(uint32_t)key1 * vs_t;
  lds_dma16(kb + c + k0, lds_w);
  lds_dma16(kb + c + k1, lds_w + 4096);
  lds_dma16(vb + c + v0, lds_w + 2 * kSwzTileElems);
  lds_dma16(vb + c + v1, lds_w + 2 * kSwzTileElems + 4096);
}

// dma_tile for K and V with 64-element rows (row stride 64) from
// wave-uniform bases, every key below 2^24 (byte offsets fit in 32 bits).
__device__ __forceinline__ void dma_tile_rows64(const uint16_t* kb, const uint16_t* vb, int key0, int key1,
                                                uint32_t lds_w) {
  const int tid = threadIdx.x;
  const uint32_t c = 8u * (uint32_t)((tid & 7) ^ tile_swz(tid >> 3));
  const uint32_t o0 = ((uint32_t)key0 * 64u + c) * 2u, o1 = ((uint32_t)key1 * 64u + c) * 2u;
  lds_dma16_s(kb, o0, lds_w);
  lds_dma16_s(kb, o1, lds_w + 4096);
  lds_dma16_s(vb, o0, lds_w + 2 * kSwzTileElems);
  lds_dma16_s(vb, o1, lds_w + 2 * kSwzTileElems + 4096);
}


}  // namespace pfa
