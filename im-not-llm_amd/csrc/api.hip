// Error reporting, argument checks and host->device staging shared by the
// library's entry points.
#include <cstdio>
#include <cstring>
#include <string>

#include "inl_common.hpp"

namespace inl {

namespace {
thread_local std::string g_last_error;

// Pinned staging buffer of the calling thread for small host->device uploads
// (tile schedules). The event guards reuse: the previous upload must have
// left the buffer before it is overwritten.
struct Staging {
  void* host = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
  ~Staging() {
    // Process teardown: the runtime may already be gone; ignore failures.
    if (done) (void)hipEventDestroy(done);
    if (host) (void)hipHostFree(host);
  }
};
thread_local Staging g_staging;
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

int upload_async(void* dst, const void* src, size_t bytes, hipStream_t stream) {
  Staging& s = g_staging;
  if (s.pending) {
    INL_HIP_TRY(hipEventSynchronize(s.done));
    s.pending = false;
  }
  if (!s.done) INL_HIP_TRY(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
  if (bytes > s.cap) {
    if (s.host) INL_HIP_TRY(hipHostFree(s.host));
    s.host = nullptr;
    s.cap = 0;
    size_t cap = 4096;
    while (cap < bytes) cap *= 2;
    INL_HIP_TRY(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
    s.cap = cap;
  }
  std::memcpy(s.host, src, bytes);
  INL_HIP_TRY(hipMemcpyAsync(dst, s.host, bytes, hipMemcpyHostToDevice, stream));
  INL_HIP_TRY(hipEventRecord(s.done, stream));
  s.pending = true;
  return INL_OK;
}

}  // namespace inl

extern "C" const char* inl_last_error(void) { return inl::g_last_error.c_str(); }

extern "C" int32_t inl_abi_version(void) { return INL_HIP_ABI_VERSION; }
