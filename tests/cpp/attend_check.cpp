// Test shim: drives the C++ interface of include/inl_attention.hpp from
// pytest through ctypes (in-process, so no child process touches the GPU).
// Each hook catches inl::Error and returns its status and message.

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "inl_attention.hpp"

namespace {
int report(const inl::Error& e, char* msg, int cap) {
  if (msg && cap > 0) {
    std::strncpy(msg, e.what(), (size_t)cap - 1);
    msg[cap - 1] = 0;
  }
  return e.status();
}
}  // namespace

extern "C" int inl_test_resolve(int request, int device, int dtype, int head_dim, int64_t padded,
                                int64_t* score_rows, char* msg, int cap) {
  try {
    auto b = inl::AttentionBackend::resolve((inl::AttentionRequest)request, (inl::DeviceKind)device, dtype, head_dim);
    *score_rows = (int64_t)b.score_rows((size_t)padded);
    return 0;
  } catch (const inl::Error& e) {
    return report(e, msg, cap);
  }
}

// form 0: causal, left padding pads[b] (Qwen3); form 1: right padding with
// real lengths lens[b], `causal` and `window`. Runs attend `repeat` times
// (the later calls reuse the mask's plan).
extern "C" int inl_test_attend(int form, const int32_t* pad_or_len, int B, int T, int causal, int window, int hq,
                               int hkv, int d, int dtype, int out_dtype, float scale, const void* q, const void* k,
                               const void* v, void* out, void* stream, int repeat, char* msg, int cap) {
  try {
    auto be = inl::AttentionBackend::resolve(inl::AttentionRequest::Fused, inl::DeviceKind::Hip, dtype, d);
    std::vector<int32_t> pl(pad_or_len, pad_or_len + B);
    inl::BatchMask mask = form == 0 ? inl::BatchMask::causal_left_padded(be, pl, T)
                                    : inl::BatchMask::right_padded(be, pl, T, causal != 0, window);
    const inl::Tensor4 tq{q, dtype, B, T, hq, d, 0}, tk{k, dtype, B, T, hkv, d, 0}, tv{v, dtype, B, T, hkv, d, 0};
    const inl::MutTensor4 to{out, out_dtype, B, T, hq, d, 0};
    for (int r = 0; r < repeat; ++r) inl::attend(be, tq, tk, tv, mask, scale, hkv > 0 ? hq / hkv : 0, to, stream);
    return 0;
  } catch (const inl::Error& e) {
    return report(e, msg, cap);
  }
}
