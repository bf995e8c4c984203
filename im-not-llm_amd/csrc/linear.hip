// Linear layers of the encoder on hipBLASLt: y = alpha * x . W^T + beta * y.
//
// The projections and the MLP of an encoder layer are plain GEMMs, so they go
// to the library GEMM (hipBLASLt's gfx950 kernels), not to a hand-written
// kernel. This wrapper keeps the row-major, bias-free `Linear` convention of
// the reference (candle_nn::Linear as built by linear_no_bias in
// crates/inl-text/src/qwen3/mod.rs:99-104,188-209): x [m, k] rows, W [n, k]
// rows (the checkpoint's [out, in] layout), y [m, n] rows. beta = 1 adds the
// product into y, which is how the residual additions of a pre-norm block
// (qwen3/mod.rs:291-296) fold into the o_proj and down_proj GEMMs.
//
// Column-major view used for hipBLASLt: y^T [n, m] = W [n, k] . x^T [k, m],
// i.e. A = W stored [k, n] (ld = w_stride) transposed, B = x stored [k, m]
// (ld = x_stride), C = D = y stored [n, m] (ld = y_stride).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "inl_common.hpp"

namespace inl {

namespace {

constexpr int kMaxDevices = 64;

struct GemmKey {
  int dev;
  int64_t m, n, k, xs, ws, ys;
  int32_t din, dout;
  bool acc;
  size_t wsb;
  bool operator<(const GemmKey& o) const {
    return std::tie(dev, m, n, k, xs, ws, ys, din, dout, acc, wsb) <
           std::tie(o.dev, o.m, o.n, o.k, o.xs, o.ws, o.ys, o.din, o.dout, o.acc, o.wsb);
  }
};

struct GemmPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
};

// Per-device handles and per-shape plans, created on first use and kept
// until the process ends (a shape's heuristic query costs far more than the
// GEMM of a small batch). A new shape's plan times up to kTuneCandidates of
// hipBLASLt's heuristic algorithms on the call's own operands and keeps the
// fastest; at the encoder's small token counts the first heuristic choice is
// up to 13 % slower than the best of the list (778 x 4096 x 1024 f32). Under
// stream capture, where nothing can be timed, the first choice is taken.
std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<GemmKey, GemmPlan> g_plans;

int lt_fail(hipblasStatus_t st, const char* what) {
  return fail(INL_E_HIP, std::string("linear: ") + what + " failed (hipBLASLt status " + std::to_string((int)st) + ")");
}

#define INL_LT_TRY(expr)                                   \
  do {                                                     \
    hipblasStatus_t inl_st_ = (expr);                      \
    if (inl_st_ != HIPBLAS_STATUS_SUCCESS) return lt_fail(inl_st_, #expr); \
  } while (0)

hipDataType hip_type(int32_t dt) { return dt == INL_BF16 ? HIP_R_16BF : HIP_R_32F; }

constexpr int kTuneCandidates = 16;
constexpr int kTuneRuns = 5;

// Average time of `runs` launches of one algorithm, or a negative value if
// it fails. Output to `c_tmp` (the call's y is not touched).
float time_algo(hipblasLtHandle_t h, const GemmPlan& pl, const hipblasLtMatmulAlgo_t& algo, const void* x,
                const void* w, void* c_tmp, float alpha, float beta, void* ws, size_t wsb, hipStream_t st,
                hipEvent_t e0, hipEvent_t e1) {
  auto run = [&]() {
    return hipblasLtMatmul(h, pl.op, &alpha, w, pl.a, x, pl.b, &beta, c_tmp, pl.c, c_tmp, pl.c, &algo, ws, wsb, st);
  };
  for (int i = 0; i < 2; ++i)
    if (run() != HIPBLAS_STATUS_SUCCESS) return -1.f;
  if (hipEventRecord(e0, st) != hipSuccess) return -1.f;
  for (int i = 0; i < kTuneRuns; ++i)
    if (run() != HIPBLAS_STATUS_SUCCESS) return -1.f;
  float ms = 0.f;
  if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
      hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
    return -1.f;
  return ms;
}

// Called with g_mu held. x, w, ws and the stream are the call's, for timing.
int plan_for(const GemmKey& key, hipblasLtHandle_t* handle, GemmPlan** out, const void* x, const void* w,
             float alpha, float beta, void* ws, hipStream_t stream) {
  if (!g_handle[key.dev]) INL_LT_TRY(hipblasLtCreate(&g_handle[key.dev]));
  *handle = g_handle[key.dev];
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return INL_OK;
  }
  GemmPlan pl;
  INL_LT_TRY(hipblasLtMatmulDescCreate(&pl.op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  INL_LT_TRY(hipblasLtMatmulDescSetAttribute(pl.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  INL_LT_TRY(hipblasLtMatmulDescSetAttribute(pl.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&pl.a, hip_type(key.din), (uint64_t)key.k, (uint64_t)key.n, key.ws));
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&pl.b, hip_type(key.din), (uint64_t)key.k, (uint64_t)key.m, key.xs));
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&pl.c, hip_type(key.dout), (uint64_t)key.n, (uint64_t)key.m, key.ys));
  hipblasLtMatmulPreference_t pref = nullptr;
  INL_LT_TRY(hipblasLtMatmulPreferenceCreate(&pref));
  const uint64_t cap = key.wsb;
  hipblasStatus_t st =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap, sizeof(cap));
  hipblasLtMatmulHeuristicResult_t res[kTuneCandidates];
  int found = 0;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulAlgoGetHeuristic(*handle, pl.op, pl.a, pl.b, pl.c, pl.c, pref, kTuneCandidates, res, &found);
  (void)hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(st, "hipblasLtMatmulAlgoGetHeuristic");
  if (found < 1)
    return fail(INL_E_UNSUPPORTED, "linear: hipBLASLt has no algorithm for m=" + std::to_string(key.m) +
                                       " n=" + std::to_string(key.n) + " k=" + std::to_string(key.k) +
                                       " within the given workspace");
  int best = 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (found > 1 && hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
    // a scratch output of the GEMM's shape (rows of y_stride), zeroed
    void* c_tmp = nullptr;
    const size_t c_bytes = (size_t)key.m * key.ys * (key.dout == INL_BF16 ? 2 : 4);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&c_tmp, c_bytes) == hipSuccess && hipMemsetAsync(c_tmp, 0, c_bytes, stream) == hipSuccess &&
        hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
      float best_ms = -1.f;
      for (int i = 0; i < found; ++i) {
        const float ms = time_algo(*handle, pl, res[i].algo, x, w, c_tmp, alpha, beta, ws, key.wsb, stream, e0, e1);
        if (ms >= 0.f && (best_ms < 0.f || ms < best_ms)) {
          best_ms = ms;
          best = i;
        }
      }
    }
    (void)hipGetLastError();
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (c_tmp) {
      (void)hipStreamSynchronize(stream);
      (void)hipFree(c_tmp);
    }
  } else {
    (void)hipGetLastError();
  }
  pl.algo = res[best].algo;
  pl.ws = res[best].workspaceSize;
  *out = &g_plans.emplace(key, pl).first->second;
  return INL_OK;
}

}  // namespace

}  // namespace inl

extern "C" int inl_linear_workspace_size(size_t* bytes) {
  if (!bytes) return inl::fail(INL_E_INVALID, "linear: bytes out-pointer is NULL");
  *bytes = (size_t)32 << 20;
  return INL_OK;
}

extern "C" int inl_linear_fwd(int64_t m, int64_t n, int64_t k, int32_t in_dtype, const void* x, int64_t x_stride,
                              const void* w, int64_t w_stride, int32_t out_dtype, void* y, int64_t y_stride,
                              float alpha, float beta, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace inl;
  if (m < 0 || n <= 0 || k <= 0) return fail(INL_E_INVALID, "linear: m must be >= 0, n and k > 0");
  if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype) || (in_dtype == INL_F32 && out_dtype != INL_F32))
    return fail(INL_E_INVALID, "linear: dtypes must be f32 -> f32, bf16 -> bf16 or bf16 -> f32");
  const int64_t xs = x_stride ? x_stride : k, ws = w_stride ? w_stride : k, ys = y_stride ? y_stride : n;
  if (xs < k || ws < k || ys < n) return fail(INL_E_INVALID, "linear: a row stride is shorter than its row");
  if (m == 0) return INL_OK;
  if (!x || !w || !y) return fail(INL_E_INVALID, "linear: NULL x, w or y");
  if (workspace_bytes && !workspace) return fail(INL_E_INVALID, "linear: workspace is NULL");
  int dev = 0;
  INL_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(INL_E_UNSUPPORTED, "linear: device ordinal beyond 63");
  const GemmKey key{dev, m, n, k, xs, ws, ys, in_dtype, out_dtype, beta != 0.f, workspace_bytes};
  hipblasLtHandle_t h = nullptr;
  GemmPlan* pl = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    int rc = plan_for(key, &h, &pl, x, w, alpha, beta, workspace, (hipStream_t)stream);
    if (rc) return rc;
  }
  INL_LT_TRY(hipblasLtMatmul(h, pl->op, &alpha, w, pl->a, x, pl->b, &beta, y, pl->c, y, pl->c, &pl->algo,
                             workspace, workspace_bytes, (hipStream_t)stream));
  return INL_OK;
}
