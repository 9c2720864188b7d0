// The projection GEMMs of the forward (QKV in, attention out): y = x W^T
// (+ bias) in bf16 with f32 accumulation, on hipBLASLt.  These are plain
// library GEMMs; what this file adds is the choice of kernel.  hipBLASLt's
// first heuristic pick for the config-3 QKV shape (M = 65,536 tokens, N =
// 1,536, K = 512) ran at ~30% of dense MFMA peak, while other solutions in
// its own candidate list run the same product ~30% faster.  So the first
// call for a shape, outside graph capture, times the leading candidates on
// the caller's stream and keeps the fastest one whose result is bitwise the
// same on two runs (split-K solutions that reduce with atomics are not);
// later calls and captured calls reuse it.
//
// Row-major y (M, N) = x (M, K) W (N, K)^T is the column-major product
// y^T (N x M) = op_T(A) B with A = W^T stored K x N (lda = K) and B = x^T
// stored K x M (ldb = K): hipBLASLt's "TN" problem, m = N, n = M, k = K.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "pfa_common.h"

using namespace pfa;

namespace {

constexpr int kCandidates = 24;                          // heuristic candidates timed per shape
constexpr size_t kWorkspaceBytes = (size_t)64 << 20;     // per device, allocated once
constexpr int kTimedRuns = 3;

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool tuned = false;   // algo chosen by timing (false: heuristic first pick)
  bool timed = false;   // a timing pass ran (tuned or not, it is not repeated)
};

struct DeviceState {
  hipblasLtHandle_t handle = nullptr;
  void* ws = nullptr;
};

using Key = std::tuple<int, int64_t, int, int, bool>;  // device, M, N, K, bias

std::mutex g_mu;
std::map<int, DeviceState> g_dev;
std::map<Key, Plan> g_plans;

__global__ void count_diff_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t n,
                                  unsigned int* __restrict__ diff) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  unsigned int d = 0;
  for (; i < n; i += stride) d |= a[i] ^ b[i];
  if (__ballot(d != 0) != 0 && (threadIdx.x & 63) == 0) atomicOr(diff, 1u);
}

int fail_blas(const char* what, hipblasStatus_t st) {
  set_error("pfa_linear: %s failed (hipblasStatus %d)", what, (int)st);
  return PFA_E_UNSUPPORTED;
}

#define PFA_BLAS(call, what)                                  \
  do {                                                        \
    hipblasStatus_t _st = (call);                             \
    if (_st != HIPBLAS_STATUS_SUCCESS) return fail_blas(what, _st); \
  } while (0)

int device_state(int dev, DeviceState** out) {
  auto it = g_dev.find(dev);
  if (it == g_dev.end()) {
    DeviceState st;
    PFA_BLAS(hipblasLtCreate(&st.handle), "hipblasLtCreate");
    hipError_t e = hipMalloc(&st.ws, kWorkspaceBytes);
    if (e != hipSuccess) {
      (void)hipblasLtDestroy(st.handle);
      set_error("pfa_linear: workspace allocation failed: %s", hipGetErrorString(e));
      return (int)e;
    }
    it = g_dev.emplace(dev, st).first;
  }
  *out = &it->second;
  return PFA_OK;
}

int make_plan(int64_t M, int N, int K, const void* bias, Plan* p) {
  PFA_BLAS(hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "MatmulDescCreate");
  const hipblasOperation_t opA = HIPBLAS_OP_T, opB = HIPBLAS_OP_N;
  PFA_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opA, sizeof(opA)), "TRANSA");
  PFA_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opB, sizeof(opB)), "TRANSB");
  if (bias != nullptr) {
    const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bt = HIP_R_16BF;
    PFA_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)), "EPILOGUE");
    PFA_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)),
             "BIAS_DATA_TYPE");
  }
  PFA_BLAS(hipblasLtMatrixLayoutCreate(&p->la, HIP_R_16BF, K, N, K), "layout A");
  PFA_BLAS(hipblasLtMatrixLayoutCreate(&p->lb, HIP_R_16BF, K, M, K), "layout B");
  PFA_BLAS(hipblasLtMatrixLayoutCreate(&p->lc, HIP_R_16BF, N, M, N), "layout C");
  return PFA_OK;
}

hipblasStatus_t run(const DeviceState& ds, const Plan& p, const hipblasLtMatmulAlgo_t& algo, const void* x,
                    const void* w, const void* bias, void* y, hipStream_t s) {
  if (bias != nullptr) {
    hipblasStatus_t st =
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    if (st != HIPBLAS_STATUS_SUCCESS) return st;
  }
  const float alpha = 1.f, beta = 0.f;
  return hipblasLtMatmul(ds.handle, p.desc, &alpha, w, p.la, x, p.lb, &beta, y, p.lc, y, p.lc, &algo, ds.ws,
                         kWorkspaceBytes, s);
}

// Times the heuristic candidates on stream s with the call's own operands
// (y is overwritten; the caller's product follows) and picks the fastest
// deterministic one.  Returns PFA_OK with p->algo set, tuned or not.
int tune(const DeviceState& ds, Plan* p, int64_t M, int N, const void* x, const void* w, const void* bias, void* y,
         hipStream_t s, bool capturing) {
  hipblasLtMatmulPreference_t pref;
  PFA_BLAS(hipblasLtMatmulPreferenceCreate(&pref), "PreferenceCreate");
  const uint64_t wsb = kWorkspaceBytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
  std::vector<hipblasLtMatmulHeuristicResult_t> res(kCandidates);
  int got = 0;
  hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(ds.handle, p->desc, p->la, p->lb, p->lc, p->lc, pref,
                                                       kCandidates, res.data(), &got);
  (void)hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || got <= 0) return fail_blas("AlgoGetHeuristic", st);
  p->algo = res[0].algo;
  p->tuned = false;
  if (capturing) return PFA_OK;  // no timing inside a capture
  p->timed = true;
  if (got == 1) return PFA_OK;

  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return PFA_OK;
  std::vector<std::pair<float, int>> times;
  for (int c = 0; c < got; ++c) {
    if (res[c].state != HIPBLAS_STATUS_SUCCESS || res[c].workspaceSize > kWorkspaceBytes) continue;
    if (run(ds, *p, res[c].algo, x, w, bias, y, s) != HIPBLAS_STATUS_SUCCESS) continue;  // warm-up
    (void)hipEventRecord(e0, s);
    bool ok = true;
    for (int r = 0; r < kTimedRuns && ok; ++r) ok = run(ds, *p, res[c].algo, x, w, bias, y, s) == HIPBLAS_STATUS_SUCCESS;
    (void)hipEventRecord(e1, s);
    if (!ok || hipEventSynchronize(e1) != hipSuccess) {
      (void)hipGetLastError();
      continue;
    }
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    times.emplace_back(ms, c);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  std::sort(times.begin(), times.end());
  // the fastest candidate that writes the same bits twice
  const size_t ybytes = (size_t)M * (size_t)N * 2;
  void* y2 = nullptr;
  unsigned int* flag = nullptr;
  if (times.empty() || hipMalloc(&y2, ybytes) != hipSuccess) return PFA_OK;
  if (hipMalloc(&flag, sizeof(unsigned int)) != hipSuccess) {
    (void)hipFree(y2);
    return PFA_OK;
  }
  for (const auto& tc : times) {
    const hipblasLtMatmulAlgo_t& a = res[tc.second].algo;
    if (run(ds, *p, a, x, w, bias, y, s) != HIPBLAS_STATUS_SUCCESS) continue;
    if (run(ds, *p, a, x, w, bias, y2, s) != HIPBLAS_STATUS_SUCCESS) continue;
    unsigned int h = 0;
    (void)hipMemsetAsync(flag, 0, sizeof(unsigned int), s);
    count_diff_kernel<<<1024, 256, 0, s>>>((const uint16_t*)y, (const uint16_t*)y2, (int64_t)(ybytes / 2), flag);
    (void)hipMemcpyAsync(&h, flag, sizeof(unsigned int), hipMemcpyDeviceToHost, s);
    if (hipStreamSynchronize(s) != hipSuccess) break;
    if (h == 0) {
      p->algo = a;
      p->tuned = true;
      break;
    }
  }
  (void)hipFree(flag);
  (void)hipFree(y2);
  return PFA_OK;
}

}  // namespace

extern "C" int pfa_linear(const void* x, int dtype, int64_t M, int K, const void* w, int N, const void* bias,
                          void* y, void* stream) {
  clear_error();
  PFA_CHECK_ARG(M >= 0 && K > 0 && N > 0, "pfa_linear: bad sizes M=%lld N=%d K=%d", (long long)M, N, K);
  if (dtype != PFA_BF16) {
    set_error("pfa_linear: only bf16 is supported (got dtype %d)", dtype);
    return PFA_E_UNSUPPORTED;
  }
  if (M == 0) return PFA_OK;
  PFA_CHECK_ARG(x && w && y, "pfa_linear: null pointer");
  PFA_CHECK_ARG(M < INT32_MAX, "pfa_linear: M too large (%lld)", (long long)M);
  hipStream_t s = as_stream(stream);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("pfa_linear: hipGetDevice failed");
    return PFA_E_INVALID;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusNone;
  const bool capturing = cap != hipStreamCaptureStatusNone;

  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* ds = nullptr;
  if (capturing && g_dev.find(dev) == g_dev.end()) {
    set_error("pfa_linear: first call on a device inside a graph capture (run it once outside the capture)");
    return PFA_E_INVALID;
  }
  int rc = device_state(dev, &ds);
  if (rc != PFA_OK) return rc;
  const Key key{dev, M, N, K, bias != nullptr};
  auto it = g_plans.find(key);
  if (it == g_plans.end() || (!it->second.timed && !capturing)) {
    if (it == g_plans.end()) {
      Plan p;
      rc = make_plan(M, N, K, bias, &p);
      if (rc != PFA_OK) return rc;
      it = g_plans.emplace(key, p).first;
    }
    rc = tune(*ds, &it->second, M, N, x, w, bias, y, s, capturing);
    if (rc != PFA_OK) return rc;
  }
  hipblasStatus_t st = run(*ds, it->second, it->second.algo, x, w, bias, y, s);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail_blas("hipblasLtMatmul", st);
  return PFA_OK;
}

// 1 when the shape's kernel was chosen by timing, 0 when not yet (or never
// called), so that a caller can tune before a graph capture.
extern "C" int pfa_linear_tuned(int64_t M, int N, int K, int has_bias) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_plans.find(Key{dev, M, N, K, has_bias != 0});
  return it != g_plans.end() && it->second.tuned ? 1 : 0;
}
