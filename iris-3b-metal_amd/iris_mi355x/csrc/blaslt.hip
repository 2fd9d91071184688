// Plain GEMMs on hipBLASLt. F.linear with an optional FP32 bias and BF16 output (no fused
// epilogue), for the weight shapes where the vendor kernels measured faster inside the denoise
// step than this library's: the single-stream blocks' SwiGLU down projection w2 (2560 x 6848) and
// the pixel stage's adaLN (16384 x 2560), compress (1280 x 4096), q|k|v (3840 x 1280), proj
// (1280 x 1280) and expand (4096 x 1280) projections, 4096-4352 rows each. The fused GEMMs
// (SwiGLU, q|k|v|gate, the grouped dual-stream launches, SiLU) stay on gemm.hip's kernels.
//
// Per device: one handle, created on the first call; per problem (m, n, k, strides, bias or
// not) a matmul descriptor, layouts and the heuristic's first algorithm among those that take
// no workspace, cached (for these shapes the heuristic's first choice takes none at any
// workspace cap, so the launches use no device memory beyond their operands). Set-up (the
// handle, a problem's plan and its kernel objects) may allocate, so a problem first met while
// its stream is being captured into a graph is declined (the caller's own kernel runs); the
// engine runs every forward once eagerly before recording it, so the recorded graph holds the
// hipBLASLt launches.
#include "blaslt.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace iris {
namespace {

struct Plan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

using Key = std::tuple<int, int, int, long, long, long, bool>;  // m, n, k, lda, ldb, ldc, bias

struct DeviceState {
  bool tried = false;
  hipblasLtHandle_t handle = nullptr;
  std::map<Key, Plan> plans;
};

std::mutex g_mutex;
std::map<int, DeviceState> g_devices;

bool ok(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS; }

// Row-major C[m, n] = A[m, k] W[n, k]^T is column-major C^T (n x m) = W (k x n)^T A^T (k x m):
// hipBLASLt's A is the weight, transposed; its B the activations; its D the output, ld = ldc.
Plan make_plan(hipblasLtHandle_t handle, int m, int n, int k, long lda, long ldb, long ldc, bool bias) {
  Plan p;
  hipblasLtMatmulPreference_t pref = nullptr;
  bool good = ok(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  good = good && ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  good = good && ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  if (bias) {
    const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bias_type = HIP_R_32F;
    good = good && ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)));
    good = good &&
           ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type, sizeof(bias_type)));
  }
  good = good && ok(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, k, n, ldb));
  good = good && ok(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, k, m, lda));
  good = good && ok(hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, n, m, ldc));
  good = good && ok(hipblasLtMatmulPreferenceCreate(&pref));
  const uint64_t ws = 0;  // algorithms without a workspace only
  good = good && ok(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)));
  hipblasLtMatmulHeuristicResult_t result{};
  int found = 0;
  good = good && ok(hipblasLtMatmulAlgoGetHeuristic(handle, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, &result, &found));
  good = good && found > 0 && result.workspaceSize == 0;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (good) {
    p.algo = result.algo;
    p.ok = true;
  }
  return p;
}

}  // namespace

bool blaslt_wanted(int m, int n, int k) {
  static constexpr int kShapes[][2] = {{2560, 6848}, {16384, 2560}, {1280, 4096}, {3840, 1280}, {1280, 1280}, {4096, 1280}};
  if (m < 2048) return false;  // measured at 4096-4352 rows
  for (const auto& s : kShapes)
    if (s[0] == n && s[1] == k) return true;
  return false;
}

bool blaslt_linear(const bf16* a, const bf16* w, const float* bias, bf16* c, int m, int n, int k, long lda, long ldb,
                   long ldc, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(g_mutex);
  DeviceState& st = g_devices[dev];
  const Key key{m, n, k, lda, ldb, ldc, bias != nullptr};
  auto it = st.plans.find(key);
  if (it == st.plans.end()) {
    if (capture != hipStreamCaptureStatusNone) return false;  // set-up only outside capture
    if (!st.tried) {
      st.tried = true;
      if (!ok(hipblasLtCreate(&st.handle))) st.handle = nullptr;
    }
    if (!st.handle) return false;
    it = st.plans.emplace(key, make_plan(st.handle, m, n, k, lda, ldb, ldc, bias != nullptr)).first;
  }
  Plan& p = it->second;
  if (!p.ok) return false;
  if (bias && !ok(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias))))
    return false;
  const float alpha = 1.0f, beta = 0.0f;
  return ok(hipblasLtMatmul(st.handle, p.desc, &alpha, w, p.la, a, p.lb, &beta, c, p.lc, c, p.lc, &p.algo, nullptr, 0,
                            stream));
}

}  // namespace iris
