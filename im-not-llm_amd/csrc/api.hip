// Error reporting and argument checks shared by the library's entry points.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "inl_common.hpp"

namespace inl {

namespace {
thread_local std::string g_last_error;

}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  std::string m = std::string(what) + ": " + hipGetErrorString(err);
  return fail(INL_E_HIP, m);
}

int check_cu(int32_t n, const int32_t* cu, int64_t* total) {
  *total = 0;
  if (n == 0) return INL_OK;
  if (cu[0] != 0) return fail(INL_E_INVALID, "cu_seqlens[0] must be 0");
  for (int32_t b = 0; b < n; ++b)
    if (cu[b + 1] < cu[b]) return fail(INL_E_INVALID, "cu_seqlens must be nondecreasing");
  *total = cu[n];
  return INL_OK;
}

HostStage::~HostStage() {
  if (done) {
    if (pending) (void)hipEventSynchronize(done);
    (void)hipEventDestroy(done);
  }
  if (buf) (void)hipHostFree(buf);
}

int HostStage::reserve(size_t bytes) {
  if (pending) {
    INL_HIP_TRY(hipEventSynchronize(done));
    pending = false;
  }
  if (!done) INL_HIP_TRY(hipEventCreateWithFlags(&done, hipEventDisableTiming));
  if (bytes <= cap) return INL_OK;
  if (buf) {
    INL_HIP_TRY(hipHostFree(buf));
    buf = nullptr;
    cap = 0;
  }
  const size_t want = std::max<size_t>(bytes + bytes / 4, (size_t)1 << 16);
  INL_HIP_TRY(hipHostMalloc((void**)&buf, want, hipHostMallocDefault));
  cap = want;
  return INL_OK;
}

int HostStage::record(hipStream_t st) {
  INL_HIP_TRY(hipEventRecord(done, st));
  pending = true;
  return INL_OK;
}

int set_max_dynamic_lds(const void* fn, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  INL_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({fn, dev})) return INL_OK;
  INL_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
  done.insert({fn, dev});
  return INL_OK;
}

}  // namespace inl

extern "C" const char* inl_last_error(void) { return inl::g_last_error.c_str(); }

extern "C" int32_t inl_abi_version(void) { return INL_HIP_ABI_VERSION; }
