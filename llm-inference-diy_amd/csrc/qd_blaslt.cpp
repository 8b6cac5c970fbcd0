// Plain fp16 products of the matrix-core prefill through hipBLASLt.
//
// The prompt's QKV, o-proj and c_proj projections are plain GEMMs
// (qwen_infer.cu:462, :542, :593 call the reference's tensor-core GEMM for
// them), and so are gate and up taken as one product of 2 * inter columns, so
// from 128 rows up they go to the vendor library.  For Qwen-1.8B its kernels
// took 49 / 27 / 58 us for the 2048-row QKV / o-proj / c_proj in a kernel trace
// of the engine's prefill, against 71 us for QKV and 126 us for o-proj plus
// c_proj with this library's 128 x 128 MFMA tile; whole MFMA prompts of 255 /
// 383 / 511 tokens took 2.6 / 3.1 / 3.2 ms against 3.2 / 4.5 / 5.1 ms with the
// split-K 64 x 64 tile.  At 127 rows and fewer the two tie (2.2 ms) and the
// tile, which needs no heuristic query for a new shape (~0.3 ms per prompt
// length on first use), stays.  The fused products (the gate/up GEMM with the
// SwiGLU epilogue below 128 rows, the flash attention) stay hand-written.
//
// Row-major y[t][n] = x[t][:] . w[n][:] is the column-major product
// D (n x t, ld ldy) = op(A) B with A = w viewed as a k x n column-major matrix
// (ld k) transposed, and B = x viewed as k x t (ld ldx).  The residual form is
// beta = 1 with C = residual: y = half(residual + sum), one rounding where the
// hand-written kernels round the sum first; both are within the QD_GEMM_MFMA
// bound (every output within an fp16 ulp of the float64 value plus the fp32
// summation bound).
#include <hipblaslt/hipblaslt.h>

#include <array>
#include <atomic>
#include <map>
#include <mutex>

#include "qd_internal.h"

namespace qd {
namespace {

constexpr int kMaxDevices = 64;
constexpr size_t kWorkspaceBytes = 64u << 20;

struct Algo {
  bool ok;
  hipblasLtMatmulAlgo_t algo;
};

struct DeviceState {
  hipblasLtHandle_t handle = nullptr;
  void* workspace = nullptr;
  bool unavailable = false;     // creation failed once: never retried
  std::map<std::array<long long, 7>, Algo> algos;
};

std::mutex g_mu;
DeviceState g_state[kMaxDevices];
std::atomic<int> g_vendor{1};   // qd_gemm_vendor_enable

// Descriptors of one product, destroyed with the object.
struct Desc {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  ~Desc() {
    if (c) (void)hipblasLtMatrixLayoutDestroy(c);
    if (b) (void)hipblasLtMatrixLayoutDestroy(b);
    if (a) (void)hipblasLtMatrixLayoutDestroy(a);
    if (op) (void)hipblasLtMatmulDescDestroy(op);
  }
  bool make(const BatchedGemvParams& p) {
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    return hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&a, HIP_R_16F, p.k, p.n, p.k) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&b, HIP_R_16F, p.k, p.t, p.ldx) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&c, HIP_R_16F, p.n, p.t, p.ldy) == HIPBLAS_STATUS_SUCCESS;
  }
};

long long align_class(const void* x, const void* w, const void* y, const void* r) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                         reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(r);
  return (long long)(bits & 15u);
}

}  // namespace

hipError_t blaslt_gemm_nt(const BatchedGemvParams& p, int epi, hipStream_t stream) {
  if (!g_vendor.load(std::memory_order_relaxed)) return hipErrorNotSupported;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipErrorNotSupported;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState& d = g_state[dev];
  if (d.unavailable) return hipErrorNotSupported;
  if (!d.handle) {
    if (hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) {
      d.handle = nullptr;
      d.unavailable = true;
      return hipErrorNotSupported;
    }
    if (hipMalloc(&d.workspace, kWorkspaceBytes) != hipSuccess) {
      d.workspace = nullptr;
      (void)hipblasLtDestroy(d.handle);
      d.handle = nullptr;
      d.unavailable = true;
      return hipErrorNotSupported;
    }
  }
  Desc desc;
  if (!desc.make(p)) return hipErrorNotSupported;
  const void* res = epi ? static_cast<const void*>(p.res) : static_cast<const void*>(p.y);
  const std::array<long long, 7> key{p.n, p.k, p.t, p.ldx, p.ldy, epi,
                                     align_class(p.x, p.w, p.y, res)};
  auto it = d.algos.find(key);
  if (it == d.algos.end()) {
    Algo algo{false, {}};
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
      const uint64_t ws = kWorkspaceBytes;
      hipblasLtMatmulHeuristicResult_t result{};
      int found = 0;
      if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
          hipblasLtMatmulAlgoGetHeuristic(d.handle, desc.op, desc.a, desc.b, desc.c, desc.c, pref, 1,
                                          &result, &found) == HIPBLAS_STATUS_SUCCESS &&
          found > 0) {
        algo.ok = true;
        algo.algo = result.algo;
      }
      (void)hipblasLtMatmulPreferenceDestroy(pref);
    }
    it = d.algos.emplace(key, algo).first;
  }
  if (!it->second.ok) return hipErrorNotSupported;
  const float alpha = 1.0f, beta = epi ? 1.0f : 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(d.handle, desc.op, &alpha, p.w, desc.a, p.x, desc.b, &beta, res, desc.c, p.y,
                      desc.c, &it->second.algo, d.workspace, kWorkspaceBytes, stream);
  return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace qd

extern "C" int qd_gemm_vendor_enable(int enable) { return qd::g_vendor.exchange(enable ? 1 : 0); }
