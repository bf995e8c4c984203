// Host-side C++ mirror of the reference's attention backend, batch mask and
// attend (crates/inl-core/src/attention.rs:40-234) over the C ABI. No device
// code: the kernels run through inl_attn_plan_create / inl_attn_fwd.

#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "inl_attention.hpp"

namespace inl {

namespace {

[[noreturn]] void raise(int status) { throw Error(status, inl_last_error()); }
[[noreturn]] void raise(int status, const std::string& msg) { throw Error(status, msg); }

// The head dims and dtypes the HIP kernels take (attn_fwd.hip select_kernel).
std::string fused_unavailable(DeviceKind device, int32_t dtype, int32_t head_dim) {
  if (device != DeviceKind::Hip) return "no fused kernel for a CPU device in the HIP library";
  if (dtype != INL_F32 && dtype != INL_BF16) return "the HIP kernel requires dtype f32 or bf16";
  if (head_dim < 8 || head_dim > 256 || head_dim % 8 != 0)
    return "the HIP kernel does not support head_dim " + std::to_string(head_dim);
  return "";
}

}  // namespace

AttentionBackend AttentionBackend::resolve(AttentionRequest request, DeviceKind device, int32_t dtype,
                                           int32_t head_dim) {
  switch (request) {
    case AttentionRequest::Eager:
    case AttentionRequest::Tiled:
      raise(INL_E_UNSUPPORTED, std::string("attention = \"") +
                                   (request == AttentionRequest::Eager ? "eager" : "tiled") +
                                   "\" is not provided by the HIP library; use \"fused\" or \"auto\"");
    case AttentionRequest::Auto:
    case AttentionRequest::Fused: {
      const std::string why = fused_unavailable(device, dtype, head_dim);
      if (!why.empty()) raise(INL_E_UNSUPPORTED, "attention = \"fused\" is unavailable: " + why);
      return AttentionBackend(HipFused);
    }
  }
  raise(INL_E_INVALID, "attention: unknown request");
}

BatchMask::BatchMask(std::vector<int32_t> lens, std::vector<int32_t> starts, int32_t seq_len, bool causal,
                     int32_t window)
    : lens_(std::move(lens)), starts_(std::move(starts)), seq_len_(seq_len), causal_(causal), window_(window) {
  cu_.assign(lens_.size() + 1, 0);
  for (size_t b = 0; b < lens_.size(); ++b) cu_[b + 1] = cu_[b] + lens_[b];
}

BatchMask BatchMask::causal_left_padded(AttentionBackend, std::vector<int32_t> pad_lens, int32_t seq_len) {
  if (seq_len < 0) raise(INL_E_INVALID, "BatchMask: negative seq_len");
  std::vector<int32_t> lens(pad_lens.size()), starts(pad_lens.size());
  for (size_t b = 0; b < pad_lens.size(); ++b) {
    if (pad_lens[b] < 0 || pad_lens[b] > seq_len)
      raise(INL_E_INVALID, "BatchMask: pad length " + std::to_string(pad_lens[b]) + " outside [0, seq_len]");
    lens[b] = seq_len - pad_lens[b];
    starts[b] = (int32_t)b * seq_len + pad_lens[b];
  }
  return BatchMask(std::move(lens), std::move(starts), seq_len, true, -1);
}

BatchMask BatchMask::right_padded(AttentionBackend, std::vector<int32_t> lens, int32_t seq_len, bool causal,
                                  int32_t window) {
  if (seq_len < 0) raise(INL_E_INVALID, "BatchMask: negative seq_len");
  if (window < -1) raise(INL_E_INVALID, "BatchMask: window must be -1 or a radius >= 0");
  std::vector<int32_t> starts(lens.size());
  for (size_t b = 0; b < lens.size(); ++b) {
    if (lens[b] < 0 || lens[b] > seq_len)
      raise(INL_E_INVALID, "BatchMask: length " + std::to_string(lens[b]) + " outside [0, seq_len]");
    starts[b] = (int32_t)b * seq_len;
  }
  return BatchMask(std::move(lens), std::move(starts), seq_len, causal, window);
}

BatchMask::~BatchMask() {
  if (plan_) inl_attn_plan_destroy(plan_);
}

BatchMask::BatchMask(BatchMask&& o) noexcept
    : lens_(std::move(o.lens_)), starts_(std::move(o.starts_)), cu_(std::move(o.cu_)), seq_len_(o.seq_len_),
      causal_(o.causal_), window_(o.window_), plan_(o.plan_), key_(o.key_) {
  o.plan_ = nullptr;
}

BatchMask& BatchMask::operator=(BatchMask&& o) noexcept {
  if (this != &o) {
    if (plan_) inl_attn_plan_destroy(plan_);
    lens_ = std::move(o.lens_);
    starts_ = std::move(o.starts_);
    cu_ = std::move(o.cu_);
    seq_len_ = o.seq_len_;
    causal_ = o.causal_;
    window_ = o.window_;
    plan_ = o.plan_;
    key_ = o.key_;
    o.plan_ = nullptr;
  }
  return *this;
}

// The plan of the first attend is kept; a later attend with other heads,
// dims, scale or dtypes (another layer kind) replaces it.
const inl_attn_plan* BatchMask::plan_for(const inl_attn_desc& d) const {
  const bool same = plan_ && key_.h_q == d.h_q && key_.h_kv == d.h_kv && key_.head_dim == d.head_dim &&
                    key_.scale == d.scale && key_.dtype == d.dtype && key_.out_dtype == d.out_dtype &&
                    key_.q_row_stride == d.q_row_stride && key_.k_row_stride == d.k_row_stride &&
                    key_.v_row_stride == d.v_row_stride && key_.o_row_stride == d.o_row_stride;
  if (same) return plan_;
  inl_attn_plan* fresh = nullptr;
  const int rc = inl_attn_plan_create(&d, &fresh);
  if (rc) raise(rc);
  if (plan_) inl_attn_plan_destroy(plan_);
  plan_ = fresh;
  key_ = d;
  return plan_;
}

void attend(AttentionBackend backend, const Tensor4& q, const Tensor4& k, const Tensor4& v, const BatchMask& mask,
            float scale, int n_rep, const MutTensor4& out, void* stream) {
  (void)backend;
  if (n_rep < 1) raise(INL_E_INVALID, "attend: n_rep must be >= 1");
  const int64_t B = mask.batch(), T = mask.seq_len();
  auto shape_ok = [&](int64_t b, int64_t t, int64_t h, int64_t d) {
    return b == B && t == T && h > 0 && d == q.d;
  };
  if (!shape_ok(q.b, q.t, q.h, q.d) || !shape_ok(k.b, k.t, k.h, k.d) || !shape_ok(v.b, v.t, v.h, v.d) ||
      !shape_ok(out.b, out.t, out.h, out.d))
    raise(INL_E_INVALID, "attend: q, k, v and out must be [B, T, H, D] with the mask's B and T and one D");
  if (k.h != v.h || q.h != k.h * n_rep || out.h != q.h)
    raise(INL_E_INVALID, "attend: q and out need n_rep * Nkv heads, k and v Nkv heads");
  if (k.dtype != q.dtype || v.dtype != q.dtype)
    raise(INL_E_INVALID, "attend: q, k and v must share one dtype");
  inl_attn_desc d;
  std::memset(&d, 0, sizeof d);
  d.n_texts = (int32_t)B;
  d.cu_seqlens_host = mask.cu_.data();
  d.h_q = (int32_t)q.h;
  d.h_kv = (int32_t)k.h;
  d.head_dim = (int32_t)q.d;
  d.causal = mask.causal_ ? 1 : 0;
  d.window = mask.window_;
  d.scale = scale;
  d.dtype = q.dtype;
  d.out_dtype = out.dtype;
  d.q_row_stride = q.row_stride;
  d.k_row_stride = k.row_stride;
  d.v_row_stride = v.row_stride;
  d.o_row_stride = out.row_stride;
  d.seq_starts_host = mask.starts_.data();
  if (B == 0) return;
  const inl_attn_plan* plan = mask.plan_for(d);
  const int rc = inl_attn_fwd(plan, q.data, k.data, v.data, out.data, stream);
  if (rc) raise(rc);
}

}  // namespace inl
