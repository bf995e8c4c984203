// Host-code driver for the ASan/UBSan build of the library (built with
// --cuda-host-only by im-not-llm_amd/sanitize.py: no device code, no GPU).
// It runs every entry point whose work is host-side only - the attention
// planner behind inl_attn_workspace_size and kernel selection, the batch
// planner, the RoPE table and position helpers, the workspace sizers - over
// random and adversarial inputs, and every device entry point with arguments
// its host checks refuse (so none reaches the device). The sanitizers turn
// any out-of-bounds access, overflow or undefined shift into a failure.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "inl_encoder.h"
#include "inl_gdn.h"
#include "inl_hip.h"

namespace {

std::mt19937_64 rng(20261202);
int failures = 0;
long cases = 0;

int64_t pick(int64_t lo, int64_t hi) { return std::uniform_int_distribution<int64_t>(lo, hi)(rng); }

void expect(bool ok, const char* what) {
  ++cases;
  if (!ok) {
    ++failures;
    std::fprintf(stderr, "FAIL: %s (%s)\n", what, inl_last_error());
  }
}

std::vector<int32_t> random_cu(int n, int max_len) {
  std::vector<int32_t> cu(n + 1, 0);
  for (int b = 0; b < n; ++b) {
    int len;
    switch (pick(0, 5)) {
      case 0: len = 0; break;
      case 1: len = 1; break;
      case 2: len = (int)pick(1, 64); break;
      case 3: len = (int)pick(60, 300); break;
      default: len = (int)pick(0, max_len); break;
    }
    cu[b + 1] = cu[b] + len;
  }
  return cu;
}

void attention_descs() {
  const int dims[] = {8, 16, 24, 64, 72, 128, 136, 200, 256, 264, 7, 0};
  const int windows[] = {-1, -1, 0, 1, 63, 64, 128, 256, 512, 100000};
  for (int it = 0; it < 4000; ++it) {
    const int n = (int)pick(0, 40);
    std::vector<int32_t> cu = random_cu(n, it % 10 == 0 ? 9000 : 2100);
    std::vector<int32_t> starts(n);
    for (int b = 0; b < n; ++b) starts[b] = cu[b] + (int)pick(0, 3);
    inl_attn_desc d;
    std::memset(&d, 0, sizeof d);
    d.n_texts = n;
    d.cu_seqlens_host = cu.data();
    d.h_kv = (int)(int[]){1, 1, 2, 4, 8}[pick(0, 4)];
    d.h_q = d.h_kv * (int)(int[]){1, 2, 3, 8, 16}[pick(0, 4)];
    if (pick(0, 20) == 0) d.h_q += 1;  // not a multiple of h_kv
    d.head_dim = dims[pick(0, 11)];
    d.causal = (int)pick(0, 1);
    d.window = windows[pick(0, 9)];
    d.scale = 0.125f;
    d.dtype = (int)pick(0, 1);
    d.out_dtype = (int)pick(0, 1);
    d.q_row_stride = pick(0, 1) ? 0 : (int64_t)d.h_q * d.head_dim + 8 * pick(0, 4);
    d.k_row_stride = pick(0, 1) ? 0 : (int64_t)d.h_kv * d.head_dim + 8 * pick(0, 4);
    d.v_row_stride = d.k_row_stride;
    d.o_row_stride = 0;
    d.flags = (int)pick(0, 1);
    d.seq_starts_host = pick(0, 3) == 0 && n > 0 ? starts.data() : nullptr;
    size_t bytes = 0;
    const int rc = inl_attn_workspace_size(&d, &bytes);
    expect(rc == INL_OK || (rc < 0 && std::strlen(inl_last_error()) > 0), "workspace size status");
    const char* name = nullptr;
    const int rk = inl_attn_kernel_name(&d, &name);
    expect(rk != INL_OK || (name && std::strlen(name) > 0), "kernel name");
    if (rc == INL_OK) expect(rk == INL_OK, "a desc with a workspace size has a kernel");
    // the one-shot form refuses a workspace that is too small before any device call
    if (rc == INL_OK && bytes > 16)
      expect(inl_attn_varlen_fwd(&d, nullptr, nullptr, nullptr, nullptr, reinterpret_cast<void*>(256), bytes - 16,
                                 nullptr) < 0,
             "one-shot refuses a short workspace");
  }
  // adversarial: decreasing cu, null cu, huge text, negative window < -1
  int32_t bad_cu[] = {0, 10, 5};
  inl_attn_desc d;
  std::memset(&d, 0, sizeof d);
  d.n_texts = 2; d.cu_seqlens_host = bad_cu; d.h_q = 4; d.h_kv = 2; d.head_dim = 64; d.window = -1; d.scale = 1.f;
  size_t bytes;
  expect(inl_attn_workspace_size(&d, &bytes) < 0, "decreasing cu refused");
  d.cu_seqlens_host = nullptr;
  expect(inl_attn_workspace_size(&d, &bytes) < 0, "null cu refused");
  int32_t huge[] = {0, 1 << 22};
  d.n_texts = 1; d.cu_seqlens_host = huge;
  expect(inl_attn_workspace_size(&d, &bytes) < 0, "text beyond the tile-range fields refused");
  int32_t ok_cu[] = {0, 100};
  d.cu_seqlens_host = ok_cu; d.window = -2;
  expect(inl_attn_workspace_size(&d, &bytes) < 0, "window < -1 refused");
}

void batch_planner() {
  for (int it = 0; it < 3000; ++it) {
    const int64_t n = pick(0, 300);
    std::vector<int32_t> len(n);
    for (auto& l : len) l = (int32_t)pick(0, pick(0, 1) ? 16 : 9000);
    const int64_t items = pick(0, 70), tokens = pick(0, 1) ? pick(1, 200000) : pick(0, 3000);
    std::vector<int64_t> ends(n + 1);
    int64_t nb = -1;
    const int rc = inl_plan_packed_batches(len.data(), n, items, tokens, ends.data(), &nb);
    if (rc == INL_OK) {
      bool ok = nb >= 0 && nb <= n && (n == 0 || ends[nb - 1] == n);
      for (int64_t i = 1; ok && i < nb; ++i) ok = ends[i] > ends[i - 1];
      expect(ok, "planner batches cover the inputs in order");
    } else {
      expect(std::strlen(inl_last_error()) > 0, "planner error message");
    }
  }
}

void rope_and_positions() {
  for (int it = 0; it < 500; ++it) {
    const int dim = (int)pick(-2, 300), pos = (int)pick(-1, 600), mode = (int)pick(-1, 2);
    std::vector<float> c((size_t)(pos > 0 ? pos : 1) * (dim > 1 ? dim / 2 : 1)), s(c.size());
    const int rc = inl_rope_table_host(dim, 1e4 * pick(1, 100), pos, mode, c.data(), s.data());
    expect(rc == INL_OK || rc < 0, "rope table status");
    const int n = (int)pick(0, 30);
    std::vector<int32_t> cu = random_cu(n, 500);
    if (pick(0, 5) == 0 && n > 1) std::swap(cu[1], cu[2]);
    std::vector<int32_t> p(cu[n] + 1);
    const int rp = inl_positions_host(n, cu.data(), p.data());
    expect(rp == INL_OK || rp < 0, "positions status");
  }
}

void sizers_and_refusals() {
  for (int it = 0; it < 500; ++it) {
    size_t bytes;
    const int rows = (int)pick(-1, 1 << 20), vocab = (int)pick(-1, 1 << 20);
    const int rc = inl_splade_decoder_workspace_size(rows, vocab, &bytes);
    expect(rc == INL_OK || rc < 0, "decoder workspace size status");
  }
  size_t ws;
  expect(inl_linear_workspace_size(&ws) == INL_OK && ws > 0, "linear workspace size");
  expect(inl_linear_fwd(-1, 8, 8, INL_F32, nullptr, 0, nullptr, 0, INL_F32, nullptr, 0, 1.f, 0.f, nullptr, 0,
                        nullptr) < 0, "linear refuses m < 0");
  int32_t offs[] = {0, 4};
  expect(inl_splade_decoder_max_fwd(1, offs, nullptr, 0, 33, nullptr, 0, 10, INL_BF16, nullptr, nullptr, 0,
                                    nullptr) < 0, "decoder refuses hidden % 32");
  expect(inl_gdn_conv_fwd(4, 1, nullptr, 8, 9, INL_F32, nullptr, 0, nullptr, nullptr, 0, nullptr) < 0,
         "conv refuses 9 taps");
  expect(inl_gdn_rule_fwd(4, 1, nullptr, 2, 3, 8, 8, INL_F32, nullptr, 0, nullptr, nullptr, 0, nullptr, 0,
                          nullptr) < 0, "rule refuses nv % nk");
  expect(inl_gdn_unit_lower_inverse_fwd(1, 65, nullptr, nullptr, nullptr) < 0, "inverse refuses 65");
  expect(inl_gdn_gated_norm_fwd(1, 1, 129, INL_F32, INL_F32, nullptr, 0, nullptr, 0, nullptr, 1e-6f, nullptr, 0,
                                nullptr) < 0, "gated norm refuses dv 129");
  expect(inl_pool_last_fwd(-1, nullptr, 8, 0, INL_F32, nullptr, nullptr, 1e-6f, 0, nullptr, nullptr) < 0,
         "pool_last refuses n < 0");
  // EmbeddingGemma 2 runner: every refusal below happens before any device call
  inl_gemma2* g = nullptr;
  expect(inl_gemma2_create(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &g) < 0 && !g,
         "gemma2 refuses a NULL config");
  inl_gemma2_config gc{};
  gc.vocab = 64; gc.hidden = 32; gc.intermediate = 64; gc.layers = 2; gc.heads = 4; gc.kv_heads = 2;
  gc.head_dim = 16; gc.ple_dim = 16; gc.embedding_dim = 24; gc.sliding_window = 3; gc.eps = 1e-6f;
  gc.theta_sliding = 1e4; gc.theta_full = 1e6; gc.max_positions = 64; gc.dtype = INL_F32;
  expect(inl_gemma2_create(&gc, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &g) < 0 && !g,
         "gemma2 refuses NULL weights");
  gc.hidden = 30;
  expect(inl_gemma2_create(&gc, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &g) < 0 && !g,
         "gemma2 refuses hidden % 8");
  gc.hidden = 32;
  gc.kv_heads = 3;
  const char dummy[16] = {};
  std::vector<inl_gemma2_layer_weights> lw(2);
  for (auto& l : lw) {
    const void* d = dummy;
    l.qkv_proj = l.o_proj = l.gate_up_proj = l.down_proj = l.q_norm = l.k_norm = l.input_norm = d;
    l.post_attention_norm = l.pre_feedforward_norm = l.post_feedforward_norm = l.ple_input_gate = d;
    l.ple_projection = l.ple_post_norm = l.layer_scalar = d;
  }
  expect(inl_gemma2_create(&gc, dummy, lw.data(), dummy, dummy, dummy, dummy, &g) < 0 && !g,
         "gemma2 refuses KV heads that do not divide the heads");
  gc.kv_heads = 2;
  lw[1].head_dim = 24;
  expect(inl_gemma2_create(&gc, dummy, lw.data(), dummy, dummy, dummy, dummy, &g) < 0 && !g,
         "gemma2 refuses a head_dim override that is not 8 x a power of two");
  lw[1].head_dim = 512;  // 8 x a power of two, but beyond the attention kernels' 256
  expect(inl_gemma2_create(&gc, dummy, lw.data(), dummy, dummy, dummy, dummy, &g) < 0 && !g,
         "gemma2 refuses a head_dim above 256");
  lw[1].head_dim = 32;   // both layers sliding: 16 and 32 cannot share the kind's one RoPE table
  expect(inl_gemma2_create(&gc, dummy, lw.data(), dummy, dummy, dummy, dummy, &g) < 0 && !g,
         "gemma2 refuses two head dims within one layer kind");
  size_t gb = 0;
  expect(inl_gemma2_workspace_size(nullptr, 1, nullptr, &gb) < 0, "gemma2 workspace refuses NULL");
  expect(inl_gemma2_encode(nullptr, 1, nullptr, nullptr, 1, nullptr, nullptr, 0, nullptr) < 0,
         "gemma2 encode refuses NULL");
  expect(inl_gemma2_destroy(nullptr) == INL_OK, "gemma2 destroy of NULL");
}

}  // namespace

int main() {
  attention_descs();
  batch_planner();
  rope_and_positions();
  sizers_and_refusals();
  std::printf("%ld cases, %d failures\n", cases, failures);
  return failures ? 1 : 0;
}
