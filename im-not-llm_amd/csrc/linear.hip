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
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

#include "inl_common.hpp"

namespace inl {

namespace {

constexpr int kMaxDevices = 64;

// A GEMM shape without its row count m: everything but m is fixed by the
// model (widths, strides, dtypes), while m is the batch's packed token count
// and changes from batch to batch.
struct ShapeKey {
  int dev;
  int64_t n, k, xs, ws, ys;
  int32_t din, dout;
  bool acc;
  size_t wsb;
  bool operator<(const ShapeKey& o) const {
    return std::tie(dev, n, k, xs, ws, ys, din, dout, acc, wsb) <
           std::tie(o.dev, o.n, o.k, o.xs, o.ws, o.ys, o.din, o.dout, o.acc, o.wsb);
  }
};

// Row counts are grouped in power-of-two buckets, (2^(b-1), 2^b] (bucket 6
// holds every m <= 64): one timing pass per (shape, bucket) chooses the
// algorithm that every other m of the bucket reuses once hipBLASLt confirms
// it supports that m.
int bucket_of(int64_t m) {
  int b = 6;
  while (b < 62 && ((int64_t)1 << b) < m) ++b;
  return b;
}

struct Bucket {
  hipblasLtMatmulDesc_t op = nullptr;   // shared by every m of the shape (kept until the process ends)
  bool tuned = false;
  hipblasLtMatmulAlgo_t algo{};
};

// Layouts and algorithm of one exact m.
struct Exact {
  hipblasLtMatmulDesc_t op = nullptr;   // the bucket's (not owned) unless own_op
  bool own_op = false;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  ~Exact() {
    for (hipblasLtMatrixLayout_t l : {a, b, c})
      if (l) (void)hipblasLtMatrixLayoutDestroy(l);
    if (own_op && op) (void)hipblasLtMatmulDescDestroy(op);
  }
};

// Per-device handles, per-(shape, bucket) choices and a bounded cache of
// exact-m layouts (oldest evicted first; entries in use are shared_ptrs, so
// an eviction never frees what a concurrent call still holds). A bucket's
// first call times up to kTuneCandidates of hipBLASLt's heuristic algorithms
// on the call's own operands and keeps the fastest: at the encoder's small
// token counts the first heuristic choice is up to 13 % slower than the best
// of the list (778 x 4096 x 1024 f32). That call allocates a scratch output,
// clears it and synchronises the stream; every later call of the bucket does
// none of these. Under stream capture, where nothing can be timed, the first
// choice is taken and the bucket stays untimed.
constexpr int kTuneCandidates = 16;
constexpr int kTuneRuns = 5;
constexpr size_t kMaxExact = 512;
constexpr size_t kMaxBuckets = 4096;

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<std::pair<ShapeKey, int>, Bucket> g_buckets;
std::map<std::pair<ShapeKey, int64_t>, std::shared_ptr<Exact>> g_exact;
std::deque<std::pair<ShapeKey, int64_t>> g_exact_order;
int64_t g_tunings = 0;

int lt_fail(hipblasStatus_t st, const char* what) {
  return fail(INL_E_HIP, std::string("linear: ") + what + " failed (hipBLASLt status " + std::to_string((int)st) + ")");
}

#define INL_LT_TRY(expr)                                   \
  do {                                                     \
    hipblasStatus_t inl_st_ = (expr);                      \
    if (inl_st_ != HIPBLAS_STATUS_SUCCESS) return lt_fail(inl_st_, #expr); \
  } while (0)

hipDataType hip_type(int32_t dt) { return dt == INL_BF16 ? HIP_R_16BF : HIP_R_32F; }

// Average time of `runs` launches of one algorithm, or a negative value if
// it fails. Output to `c_tmp` (the call's y is not touched).
float time_algo(hipblasLtHandle_t h, const Exact& ex, const hipblasLtMatmulAlgo_t& algo, const void* x,
                const void* w, void* c_tmp, float alpha, float beta, void* ws, size_t wsb, hipStream_t st,
                hipEvent_t e0, hipEvent_t e1) {
  auto run = [&]() {
    return hipblasLtMatmul(h, ex.op, &alpha, w, ex.a, x, ex.b, &beta, c_tmp, ex.c, c_tmp, ex.c, &algo, ws, wsb, st);
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

int make_op(hipblasLtMatmulDesc_t* op) {
  INL_LT_TRY(hipblasLtMatmulDescCreate(op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  INL_LT_TRY(hipblasLtMatmulDescSetAttribute(*op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  INL_LT_TRY(hipblasLtMatmulDescSetAttribute(*op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  return INL_OK;
}

int make_layouts(const ShapeKey& key, int64_t m, Exact* ex) {
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&ex->a, hip_type(key.din), (uint64_t)key.k, (uint64_t)key.n, key.ws));
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&ex->b, hip_type(key.din), (uint64_t)key.k, (uint64_t)m, key.xs));
  INL_LT_TRY(hipblasLtMatrixLayoutCreate(&ex->c, hip_type(key.dout), (uint64_t)key.n, (uint64_t)m, key.ys));
  return INL_OK;
}

// Called with g_mu held. x, w, ws and the stream are the call's, for timing.
int entry_for(const ShapeKey& key, int64_t m, hipblasLtHandle_t* handle, std::shared_ptr<Exact>* out, const void* x,
              const void* w, float alpha, float beta, void* ws, hipStream_t stream) {
  if (!g_handle[key.dev]) INL_LT_TRY(hipblasLtCreate(&g_handle[key.dev]));
  *handle = g_handle[key.dev];
  const std::pair<ShapeKey, int64_t> ek{key, m};
  auto it = g_exact.find(ek);
  if (it != g_exact.end()) {
    *out = it->second;
    return INL_OK;
  }
  const std::pair<ShapeKey, int> bk{key, bucket_of(m)};
  auto bit = g_buckets.find(bk);
  Bucket scratch_bucket;
  Bucket* bu = nullptr;
  if (bit != g_buckets.end()) {
    bu = &bit->second;
  } else if (g_buckets.size() < kMaxBuckets) {
    bu = &g_buckets[bk];
  } else {
    bu = &scratch_bucket;   // past the cap: nothing new is kept; this call picks untimed
  }
  if (!bu->op) {
    const int rc = make_op(&bu->op);
    if (rc) return rc;
  }
  auto ex = std::make_shared<Exact>();
  ex->op = bu->op;
  ex->own_op = bu == &scratch_bucket;
  int rc = make_layouts(key, m, ex.get());
  if (rc) return rc;
  bool have = false;
  if (bu->tuned) {
    // the bucket's choice, if hipBLASLt confirms it supports this m
    hipblasLtMatmulAlgo_t algo = bu->algo;
    size_t need = 0;
    if (hipblaslt_ext::matmulIsAlgoSupported(*handle, ex->op, &alpha, ex->a, ex->b, &beta, ex->c, ex->c, algo, need) ==
            HIPBLAS_STATUS_SUCCESS &&
        need <= key.wsb) {
      ex->algo = algo;
      have = true;
    }
  }
  if (!have) {
    hipblasLtMatmulPreference_t pref = nullptr;
    INL_LT_TRY(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t cap = key.wsb;
    hipblasStatus_t st =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap, sizeof(cap));
    hipblasLtMatmulHeuristicResult_t res[kTuneCandidates];
    int found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulAlgoGetHeuristic(*handle, ex->op, ex->a, ex->b, ex->c, ex->c, pref, kTuneCandidates, res,
                                           &found);
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(st, "hipblasLtMatmulAlgoGetHeuristic");
    if (found < 1)
      return fail(INL_E_UNSUPPORTED, "linear: hipBLASLt has no algorithm for m=" + std::to_string(m) +
                                         " n=" + std::to_string(key.n) + " k=" + std::to_string(key.k) +
                                         " within the given workspace");
    int best = 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool can_time = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
    if (found > 1 && can_time && !bu->tuned && bu != &scratch_bucket) {
      // a scratch output of the GEMM's shape (rows of y_stride), zeroed
      void* c_tmp = nullptr;
      const size_t c_bytes = (size_t)m * key.ys * (key.dout == INL_BF16 ? 2 : 4);
      hipEvent_t e0 = nullptr, e1 = nullptr;
      if (hipMalloc(&c_tmp, c_bytes) == hipSuccess && hipMemsetAsync(c_tmp, 0, c_bytes, stream) == hipSuccess &&
          hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        float best_ms = -1.f;
        for (int i = 0; i < found; ++i) {
          const float ms = time_algo(*handle, *ex, res[i].algo, x, w, c_tmp, alpha, beta, ws, key.wsb, stream, e0, e1);
          if (ms >= 0.f && (best_ms < 0.f || ms < best_ms)) {
            best_ms = ms;
            best = i;
          }
        }
        bu->tuned = best_ms >= 0.f;
        if (bu->tuned) {
          bu->algo = res[best].algo;
          ++g_tunings;
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
    ex->algo = res[best].algo;
  }
  if (bu == &scratch_bucket) {
    *out = ex;   // not cached; the op desc goes with the entry
    return INL_OK;
  }
  if (g_exact.size() >= kMaxExact) {
    g_exact.erase(g_exact_order.front());
    g_exact_order.pop_front();
  }
  g_exact.emplace(ek, ex);
  g_exact_order.push_back(ek);
  *out = ex;
  return INL_OK;
}

}  // namespace

}  // namespace inl

extern "C" int inl_linear_stats(int64_t* tunings, int64_t* buckets, int64_t* cached_shapes) {
  std::lock_guard<std::mutex> lock(inl::g_mu);
  if (tunings) *tunings = inl::g_tunings;
  if (buckets) *buckets = (int64_t)inl::g_buckets.size();
  if (cached_shapes) *cached_shapes = (int64_t)inl::g_exact.size();
  return INL_OK;
}

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
  const ShapeKey key{dev, n, k, xs, ws, ys, in_dtype, out_dtype, beta != 0.f, workspace_bytes};
  hipblasLtHandle_t h = nullptr;
  std::shared_ptr<Exact> ex;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    int rc = entry_for(key, m, &h, &ex, x, w, alpha, beta, workspace, (hipStream_t)stream);
    if (rc) return rc;
  }
  INL_LT_TRY(hipblasLtMatmul(h, ex->op, &alpha, w, ex->a, x, ex->b, &beta, y, ex->c, y, ex->c, &ex->algo,
                             workspace, workspace_bytes, (hipStream_t)stream));
  return INL_OK;
}
