/* C++ host interface above the C ABI: the attention backend, batch mask and
 * `attend` of crates/inl-core/src/attention.rs, for callers written in C++.
 *
 * Same names, argument meaning and error behaviour as the reference:
 *   - AttentionRequest / AttentionBackend::resolve (attention.rs:40-89):
 *     "auto" and "fused" resolve to the HIP kernels when the device, dtype
 *     and head_dim allow; "fused" otherwise fails with the reference's
 *     message, "attention = \"fused\" is unavailable: <reason>". This
 *     library holds no eager or tiled path, so those requests fail too
 *     (the reference would fall back to candle's tiled GEMMs).
 *   - score_rows (attention.rs:114-123): the fused kernel keeps no score
 *     rows, so 0.
 *   - BatchMask (attention.rs:126-160): the padding of one forward pass.
 *     The reference builds its additive mask once per forward and every layer
 *     reads it. Here the mask is index arithmetic in the kernel, and what is
 *     built once per forward and reused by every layer is the device tile plan
 *     (on the first attend).
 *   - attend (attention.rs:215-234): attention of q over k, v, GQA with
 *     n_rep query heads per KV head, rows of padding unspecified (not
 *     written).
 * Layout: tensors are [B, T, H, D] on the device, one token row of H*D
 * values, which is the layout before the reference's transpose(1, 2). The
 * custom op takes it directly, so that copy disappears.
 * Errors are thrown as inl::Error, carrying the C ABI status and message;
 * the Rust side maps the same status to candle_core::Error::Msg. */
#ifndef INL_ATTENTION_HPP
#define INL_ATTENTION_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "inl_hip.h"

namespace inl {

class Error : public std::runtime_error {
 public:
  Error(int status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
  int status() const { return status_; }

 private:
  int status_;
};

enum class AttentionRequest { Auto, Fused, Tiled, Eager };
enum class DeviceKind { Cpu, Hip };

class AttentionBackend {
 public:
  enum Kind { HipFused };
  /* attention.rs:73-89 */
  static AttentionBackend resolve(AttentionRequest request, DeviceKind device, int32_t dtype, int32_t head_dim);
  /* attention.rs:114-123 */
  size_t score_rows(size_t /*padded*/) const { return 0; }
  Kind kind() const { return kind_; }

 private:
  explicit AttentionBackend(Kind k) : kind_(k) {}
  Kind kind_;
};

/* A [B, T, H, D] device tensor; row_stride = elements between token rows
 * (0 = H * D). */
struct Tensor4 {
  const void* data;
  int32_t dtype;  /* enum inl_dtype */
  int64_t b, t, h, d;
  int64_t row_stride;
};
struct MutTensor4 {
  void* data;
  int32_t dtype;
  int64_t b, t, h, d;
  int64_t row_stride;
};

/* The padding of one forward pass over a [B, T] batch, and the attention
 * form of the model that runs it. It caches the device plan of its last
 * attend, so one thread uses a mask at a time (the reference runs a forward
 * under a per-model mutex, crates/inl-text/src/native.rs:580-583). */
class BatchMask {
 public:
  /* attention.rs:139-153: Qwen3, causal, left padding pad_lens[b] per row
   * (0 <= pad < seq_len). */
  static BatchMask causal_left_padded(AttentionBackend backend, std::vector<int32_t> pad_lens, int32_t seq_len);
  /* The right-padded forms of gemma2.rs:499-523 (window = sliding radius),
   * modernbert.rs:594-617 (window = local_attention / 2), qwen3_5.rs:914-934
   * (causal = is_causal) and vision.rs:567-574: real lengths lens[b]
   * (0 <= len <= seq_len), window -1 for none. */
  static BatchMask right_padded(AttentionBackend backend, std::vector<int32_t> lens, int32_t seq_len, bool causal,
                                int32_t window);
  ~BatchMask();
  BatchMask(BatchMask&& o) noexcept;
  BatchMask& operator=(BatchMask&& o) noexcept;
  BatchMask(const BatchMask&) = delete;
  BatchMask& operator=(const BatchMask&) = delete;

  int32_t batch() const { return (int32_t)lens_.size(); }
  int32_t seq_len() const { return seq_len_; }

 private:
  friend void attend(AttentionBackend, const Tensor4&, const Tensor4&, const Tensor4&, const BatchMask&, float, int,
                     const MutTensor4&, void*);
  BatchMask(std::vector<int32_t> lens, std::vector<int32_t> starts, int32_t seq_len, bool causal, int32_t window);
  const inl_attn_plan* plan_for(const inl_attn_desc& d) const;

  std::vector<int32_t> lens_, starts_, cu_;
  int32_t seq_len_;
  bool causal_;
  int32_t window_;
  mutable inl_attn_plan* plan_ = nullptr;
  mutable inl_attn_desc key_{};
};

/* attention.rs:215-234: out[b, t, :, :] = attention for every real token row
 * (t of row b inside its text); other rows are left as they are. q: [B, T,
 * n_rep * Nkv, D]; k, v: [B, T, Nkv, D]; out: [B, T, n_rep * Nkv, D]. */
void attend(AttentionBackend backend, const Tensor4& q, const Tensor4& k, const Tensor4& v, const BatchMask& mask,
            float scale, int n_rep, const MutTensor4& out, void* stream);

}  // namespace inl

#endif /* INL_ATTENTION_HPP */
