// Shared definitions of the gfx950 encoder-attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/inl_hip.h"

namespace inl {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Thread-local message of the last failure (returned by inl_last_error).
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t err, const char* what);

#define INL_HIP_TRY(expr)                                   \
  do {                                                      \
    hipError_t inl_err_ = (expr);                           \
    if (inl_err_ != hipSuccess) return ::inl::hip_fail(inl_err_, #expr); \
  } while (0)

inline int dtype_size(int32_t dt) { return dt == INL_BF16 ? 2 : 4; }
inline bool dtype_ok(int32_t dt) { return dt == INL_F32 || dt == INL_BF16; }

// Raise a kernel's dynamic LDS limit to `bytes`, once per (kernel, device).
int set_max_dynamic_lds(const void* fn, int bytes);

// Validate cu_seqlens (host): cu[0] == 0 and nondecreasing. Returns the token
// count through `total`.
int check_cu(int32_t n, const int32_t* cu, int64_t* total);

// inl_norm_rope_fwd with heads >= w2_heads normalised with
// weight2: the q and k heads of one fused QKV row in one launch.
int norm_rope_launch(const inl_norm_rope_desc* d, const void* x, void* y, const void* weight,
                     const void* weight2, int32_t w2_heads, const int32_t* rows, const float* cos,
                     const float* sin, const float* cos2, const float* sin2, void* stream);
// The same with per-head ranges: heads [0, w2_heads) normalised with weight,
// [w2_heads, w3_heads) with weight2, the rest with none; heads from
// rope_heads on are not rotated (one launch for a fused q/k/v row).
int norm_rope_launch_ex(const inl_norm_rope_desc* d, const void* x, void* y, const void* weight,
                        const void* weight2, int32_t w2_heads, int32_t w3_heads, int32_t rope_heads,
                        const int32_t* rows, const float* cos, const float* sin, const float* cos2,
                        const float* sin2, void* stream);

// Pinned host staging for a runner's per-call uploads (token ids, positions,
// offsets, attention schedules). A call waits until the copies of the
// previous call have consumed the buffer (one event), fills it, issues its
// hipMemcpyAsync calls from it and records the event again: the source of
// every copy outlives the copy, and the copies are truly asynchronous (no
// pageable staging inside the runtime). The buffer grows on demand (pinned
// allocations happen only then) and is freed with the runner.
struct HostStage {
  char* buf = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
  HostStage() = default;
  HostStage(const HostStage&) = delete;
  HostStage& operator=(const HostStage&) = delete;
  ~HostStage();
  // wait for the previous call's copies, then hold at least `bytes`
  int reserve(size_t bytes);
  // after this call's copies were issued on `st`
  int record(hipStream_t st);
};

// inl_attn_plan_create_in without the upload: the plan reads its schedule
// from `dev_sched` (workspace_bytes long), and `blob` receives the bytes the
// caller must copy there before the plan's first launch.
int attn_plan_prepare(const inl_attn_desc* desc, void* dev_sched, size_t workspace_bytes, std::vector<char>* blob,
                      inl_attn_plan** plan);

}  // namespace inl
