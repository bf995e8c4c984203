// Packed batch planner (host code only).
//
// The reference's engines pad every batch to its longest input and cap
// `inputs x longest` padded tokens (crates/inl-text/src/native.rs:698-735,
// crates/inl-sparse/src/native.rs:557-582, crates/inl-late/src/native.rs:
// 694-719, crates/inl-vision/src/engine.rs:782-798). With packed varlen
// attention a batch holds only its real tokens, so the cap applies to their
// sum. Inputs stay in the caller's order (the engines sort longest-first
// beforehand where they want to).

#include <cstdint>

#include "inl_common.hpp"

extern "C" int inl_plan_packed_batches(const int32_t* lengths, int64_t n, int64_t max_items, int64_t max_tokens,
                                       int64_t* batch_end, int64_t* n_batches) {
  using namespace inl;
  if (!n_batches) return fail(INL_E_INVALID, "plan_packed_batches: n_batches is NULL");
  *n_batches = 0;
  if (n < 0) return fail(INL_E_INVALID, "plan_packed_batches: negative input count");
  if (max_items < 1 || max_tokens < 1)
    return fail(INL_E_INVALID, "plan_packed_batches: max_items and max_tokens must be >= 1");
  if (n == 0) return INL_OK;
  if (!lengths || !batch_end) return fail(INL_E_INVALID, "plan_packed_batches: NULL array");
  for (int64_t i = 0; i < n; ++i)
    if (lengths[i] < 0) return fail(INL_E_INVALID, "plan_packed_batches: negative length");
  int64_t nb = 0, start = 0, tokens = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t len = lengths[i] > 0 ? lengths[i] : 1;
    // The first input of a batch is always taken, whatever its size.
    if (i > start && (i - start + 1 > max_items || tokens + len > max_tokens)) {
      batch_end[nb++] = i;
      start = i;
      tokens = 0;
    }
    tokens += len;
  }
  batch_end[nb++] = n;
  *n_batches = nb;
  return INL_OK;
}
