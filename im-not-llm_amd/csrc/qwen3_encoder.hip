// Qwen3 encoder runner: the whole forward of crates/inl-text/src/qwen3/
// mod.rs (Qwen3Model::forward_last :339-358 and Qwen3Embedder::embed
// :438-470) on one GPU, over packed texts, composed from the library's own
// entry points:
//
//   embed (f32 residual stream)
//   per layer (DecoderLayer::forward, :280-297):
//     x   = rms_norm(residual) * input_norm                 (inl_rms_norm_rows_fwd)
//     qkv = x . [Wq; Wk; Wv]^T                              (inl_linear_fwd)
//     q, k = rope(rms_norm(q|k) * q|k_norm), in place        (inl_norm_rope_fwd: q and k
//                                                             heads in one launch)
//     a   = causal GQA attention over the texts             (inl_attn_fwd)
//     residual += a . Wo^T                                  (inl_linear_fwd, beta 1)
//     x   = rms_norm(residual) * post_attention_norm
//     gu  = x . [Wgate; Wup]^T
//     m   = silu(gate) * up                                 (inl_swiglu_fwd)
//     residual += m . Wdown^T                               (beta 1)
//   embeddings = l2(rms_norm(residual[last row]) * norm)    (inl_pool_last_fwd)
//
// The attention schedule is planned once per call into the workspace and
// reused by every layer; nothing is allocated per call.
//
// A call first uploads the batch (ids, positions, offsets, the attention
// schedule) on the caller's stream, then issues the ~10 launches per layer.
// At small batches those launches cost more host time than their kernels
// take, so the launch sequence is kept as a HIP graph per batch shape: the
// first call with a given (device, cu_seqlens, workspace, output) runs
// eagerly, the second captures the sequence on a private stream and
// instantiates it, and every call after that uploads the batch and launches
// the graph on the caller's stream. The captured kernels read the batch from
// the same workspace addresses, so the graph is valid for any ids of that
// shape. A graph holding a memset node (a library call may record one) is
// discarded and the encoder stays eager: such nodes are not replayed
// reliably here.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/inl_encoder.h"
#include "inl_common.hpp"

struct inl_qwen3 {
  inl_qwen3_config cfg;
  const void* embed = nullptr;
  std::vector<inl_qwen3_layer_weights> layers;
  float* final_norm_f32 = nullptr;  // device, owned
  float* cos = nullptr;             // device, owned: [max_positions, head_dim / 2]
  float* sin = nullptr;
  // the launch-sequence graph of the last batch shape (see above)
  std::mutex mu;
  bool graphs = true;
  int g_dev = -1;
  std::vector<int32_t> g_cu;
  void* g_ws = nullptr;
  float* g_out = nullptr;
  int g_runs = 0;                    // calls with this key so far
  hipGraphExec_t g_exec = nullptr;
  hipStream_t cap = nullptr;         // private capture stream (default priority)
  std::mutex stage_mu;               // one call at a time fills the staging buffer
  inl::HostStage stage;              // pinned source of the per-call uploads
};

namespace inl {

namespace {

size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

struct Layout {
  size_t ids, pos, cu, resid, x, a, b, sched, gemm, total;
  int64_t a_w, b_w;  // row widths (elements) of the two activation buffers
};

int layout(const inl_qwen3* e, int32_t n_texts, const int32_t* cu, Layout* L) {
  const inl_qwen3_config& c = e->cfg;
  const int64_t n = n_texts > 0 ? cu[n_texts] : 0;
  const int es = dtype_size(c.dtype);
  const int64_t qkv_w = (int64_t)(c.heads + 2 * c.kv_heads) * c.head_dim;
  L->a_w = std::max<int64_t>(qkv_w, 2 * (int64_t)c.intermediate);
  L->b_w = std::max<int64_t>((int64_t)c.heads * c.head_dim, c.intermediate);
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += up256(bytes); return o; };
  L->ids = take(n * 4);
  L->pos = take(n * 4);
  L->cu = take((size_t)(n_texts + 1) * 4);
  L->resid = take((size_t)n * c.hidden * 4);
  L->x = take((size_t)n * c.hidden * es);
  L->a = take((size_t)n * L->a_w * es);
  L->b = take((size_t)n * L->b_w * es);
  inl_attn_desc d{};
  d.n_texts = n_texts;
  d.cu_seqlens_host = cu;
  d.h_q = c.heads;
  d.h_kv = c.kv_heads;
  d.head_dim = c.head_dim;
  d.causal = 1;
  d.window = -1;
  d.scale = 1.0f;
  d.dtype = c.dtype;
  d.out_dtype = c.dtype;
  d.q_row_stride = d.k_row_stride = d.v_row_stride = L->a_w;
  d.o_row_stride = L->b_w;
  d.flags = c.attn_flags;
  size_t sched = 0;
  int rc = inl_attn_workspace_size(&d, &sched);
  if (rc) return rc;
  L->sched = take(std::max<size_t>(sched, 16));
  size_t gemm = 0;
  rc = inl_linear_workspace_size(&gemm);
  if (rc) return rc;
  L->gemm = take(gemm);
  L->total = off;
  return INL_OK;
}

// The graph of `seq` for this batch key, or eager launches (see the file
// comment). `seq(stream)` issues the whole launch sequence onto `stream`.
template <typename Seq>
int run_sequence(inl_qwen3* e, int32_t n_texts, const int32_t* cu, void* ws, float* out, hipStream_t st,
                 Seq&& seq) {
  std::lock_guard<std::mutex> g(e->mu);
  if (!e->graphs) return seq((void*)st);
  int dev = -1;
  INL_HIP_TRY(hipGetDevice(&dev));
  const bool same = dev == e->g_dev && ws == e->g_ws && out == e->g_out &&
                    (int)e->g_cu.size() == n_texts + 1 && std::equal(cu, cu + n_texts + 1, e->g_cu.begin());
  if (!same) {
    if (e->g_exec) (void)hipGraphExecDestroy(e->g_exec);
    e->g_exec = nullptr;
    e->g_dev = dev;
    e->g_ws = ws;
    e->g_out = out;
    e->g_cu.assign(cu, cu + n_texts + 1);
    e->g_runs = 0;
  }
  if (e->g_exec) {
    INL_HIP_TRY(hipGraphLaunch(e->g_exec, st));
    return INL_OK;
  }
  if (e->g_runs++ == 0) return seq((void*)st);   // first call of a shape: eager
  // second call: capture on the private stream, then launch on the caller's
  if (!e->cap) INL_HIP_TRY(hipStreamCreateWithFlags(&e->cap, hipStreamNonBlocking));
  INL_HIP_TRY(hipStreamBeginCapture(e->cap, hipStreamCaptureModeThreadLocal));
  const int rc = seq((void*)e->cap);
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(e->cap, &graph);
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  if (end != hipSuccess || !graph) {
    if (graph) (void)hipGraphDestroy(graph);
    e->graphs = false;   // capture is not available here: stay eager
    (void)hipGetLastError();
    return seq((void*)st);
  }
  size_t n_nodes = 0;
  hipError_t err = hipGraphGetNodes(graph, nullptr, &n_nodes);
  std::vector<hipGraphNode_t> nodes(n_nodes);
  if (err == hipSuccess && n_nodes) err = hipGraphGetNodes(graph, nodes.data(), &n_nodes);
  bool memset = false;
  for (size_t i = 0; err == hipSuccess && i < n_nodes; ++i) {
    hipGraphNodeType t;
    err = hipGraphNodeGetType(nodes[i], &t);
    memset = memset || t == hipGraphNodeTypeMemset;
  }
  if (err == hipSuccess && !memset) err = hipGraphInstantiate(&e->g_exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (err != hipSuccess || memset || !e->g_exec) {
    e->g_exec = nullptr;
    e->graphs = false;
    (void)hipGetLastError();
    return seq((void*)st);
  }
  INL_HIP_TRY(hipGraphLaunch(e->g_exec, st));
  return INL_OK;
}

int check_config(const inl_qwen3_config* c) {
  if (!c) return fail(INL_E_INVALID, "qwen3: config is NULL");
  if (c->vocab <= 0 || c->hidden <= 0 || c->intermediate <= 0 || c->layers <= 0 || c->heads <= 0 ||
      c->kv_heads <= 0 || c->heads % c->kv_heads || c->head_dim <= 0 || c->max_positions <= 0 ||
      !(c->eps >= 0.f) || !(c->rope_theta > 0.0) || !dtype_ok(c->dtype))
    return fail(INL_E_INVALID, "qwen3: bad config");
  if (c->hidden % 8 || c->intermediate % 8)
    return fail(INL_E_UNSUPPORTED, "qwen3: hidden and intermediate must be multiples of 8");
  return INL_OK;
}

}  // namespace

}  // namespace inl

extern "C" int inl_qwen3_create(const inl_qwen3_config* cfg, const void* embed_tokens,
                                const inl_qwen3_layer_weights* layers, const void* final_norm,
                                inl_qwen3** enc) {
  using namespace inl;
  if (!enc) return fail(INL_E_INVALID, "qwen3: encoder out-pointer is NULL");
  *enc = nullptr;
  int rc = check_config(cfg);
  if (rc) return rc;
  if (!embed_tokens || !layers || !final_norm) return fail(INL_E_INVALID, "qwen3: NULL weights");
  for (int i = 0; i < cfg->layers; ++i) {
    const inl_qwen3_layer_weights& l = layers[i];
    if (!l.qkv_proj || !l.o_proj || !l.gate_up_proj || !l.down_proj || !l.q_norm || !l.k_norm ||
        !l.input_norm || !l.post_attention_norm)
      return fail(INL_E_INVALID, "qwen3: NULL weight in layer " + std::to_string(i));
  }
  inl_qwen3* e = new (std::nothrow) inl_qwen3();
  if (!e) return fail(INL_E_NOMEM, "qwen3: host allocation failed");
  e->cfg = *cfg;
  e->embed = embed_tokens;
  e->layers.assign(layers, layers + cfg->layers);
  const int half = cfg->head_dim / 2;
  std::vector<float> c((size_t)cfg->max_positions * half), s(c.size());
  rc = inl_rope_table_host(cfg->head_dim, cfg->rope_theta, cfg->max_positions, 0, c.data(), s.data());
  std::vector<float> fn(cfg->hidden);
  if (!rc) {
    hipError_t err = hipMalloc(&e->cos, c.size() * 4);
    if (err == hipSuccess) err = hipMalloc(&e->sin, s.size() * 4);
    if (err == hipSuccess) err = hipMalloc(&e->final_norm_f32, (size_t)cfg->hidden * 4);
    if (err == hipSuccess) err = hipMemcpy(e->cos, c.data(), c.size() * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(e->sin, s.data(), s.size() * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess) {
      if (cfg->dtype == INL_F32) {
        err = hipMemcpy(e->final_norm_f32, final_norm, (size_t)cfg->hidden * 4, hipMemcpyDeviceToDevice);
      } else {
        std::vector<uint16_t> b(cfg->hidden);
        err = hipMemcpy(b.data(), final_norm, (size_t)cfg->hidden * 2, hipMemcpyDeviceToHost);
        for (int i = 0; i < cfg->hidden && err == hipSuccess; ++i) {
          const uint32_t bits = (uint32_t)b[i] << 16;
          memcpy(&fn[i], &bits, 4);
        }
        if (err == hipSuccess) err = hipMemcpy(e->final_norm_f32, fn.data(), (size_t)cfg->hidden * 4, hipMemcpyHostToDevice);
      }
    }
    if (err != hipSuccess) rc = hip_fail(err, "qwen3: setting up tables");
  }
  if (rc) {
    (void)inl_qwen3_destroy(e);
    return rc;
  }
  *enc = e;
  return INL_OK;
}

extern "C" int inl_qwen3_destroy(inl_qwen3* e) {
  if (!e) return INL_OK;
  if (e->g_exec) (void)hipGraphExecDestroy(e->g_exec);
  if (e->cap) (void)hipStreamDestroy(e->cap);
  for (float* p : {e->cos, e->sin, e->final_norm_f32})
    if (p) (void)hipFree(p);
  delete e;
  return INL_OK;
}

extern "C" int inl_qwen3_graph_info(inl_qwen3* e, int32_t* enabled, int32_t* held) {
  using namespace inl;
  if (!e || !enabled || !held) return fail(INL_E_INVALID, "qwen3: bad arguments");
  std::lock_guard<std::mutex> g(e->mu);
  *enabled = e->graphs ? 1 : 0;
  *held = e->g_exec ? 1 : 0;
  return INL_OK;
}

extern "C" int inl_qwen3_set_graphs(inl_qwen3* e, int32_t enable) {
  using namespace inl;
  if (!e) return fail(INL_E_INVALID, "qwen3: encoder is NULL");
  std::lock_guard<std::mutex> g(e->mu);
  e->graphs = enable != 0;
  if (e->g_exec) (void)hipGraphExecDestroy(e->g_exec);
  e->g_exec = nullptr;
  e->g_runs = 0;
  e->g_cu.clear();
  return INL_OK;
}

extern "C" int inl_qwen3_workspace_size(const inl_qwen3* e, int32_t n_texts, const int32_t* cu, size_t* bytes) {
  using namespace inl;
  if (!e || !bytes || n_texts < 0 || (n_texts > 0 && !cu)) return fail(INL_E_INVALID, "qwen3: bad arguments");
  int64_t total = 0;
  int rc = check_cu(n_texts, cu, &total);
  if (rc) return rc;
  Layout L;
  rc = layout(e, n_texts, cu, &L);
  if (rc) return rc;
  *bytes = L.total;
  return INL_OK;
}

extern "C" int inl_qwen3_encode(inl_qwen3* e, int32_t n_texts, const int32_t* cu, const int32_t* ids_host,
                                float* out, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace inl;
  if (!e || n_texts < 0 || (n_texts > 0 && (!cu || !out))) return fail(INL_E_INVALID, "qwen3: bad arguments");
  if (n_texts == 0) return INL_OK;
  int64_t n = 0;
  int rc = check_cu(n_texts, cu, &n);
  if (rc) return rc;
  const inl_qwen3_config& c = e->cfg;
  for (int b = 0; b < n_texts; ++b) {
    const int32_t t = cu[b + 1] - cu[b];
    if (t <= 0) return fail(INL_E_INVALID, "qwen3: text " + std::to_string(b) + " is empty");
    if (t > c.max_positions)
      return fail(INL_E_INVALID, "qwen3: text " + std::to_string(b) + " is longer than max_positions");
  }
  if (!ids_host) return fail(INL_E_INVALID, "qwen3: ids_host is NULL");
  for (int64_t i = 0; i < n; ++i)
    if (ids_host[i] < 0 || ids_host[i] >= c.vocab)
      return fail(INL_E_INVALID, "qwen3: token id " + std::to_string(ids_host[i]) + " at " + std::to_string(i) +
                                     " is outside the vocabulary");
  Layout L;
  rc = layout(e, n_texts, cu, &L);
  if (rc) return rc;
  if (!workspace || workspace_bytes < L.total || ((uintptr_t)workspace & 255))
    return fail(INL_E_INVALID, "qwen3: workspace is NULL, unaligned (256 B) or smaller than inl_qwen3_workspace_size()");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int32_t* d_ids = (int32_t*)(ws + L.ids);
  int32_t* d_pos = (int32_t*)(ws + L.pos);
  int32_t* d_cu = (int32_t*)(ws + L.cu);
  float* resid = (float*)(ws + L.resid);
  char* x = ws + L.x;
  char* A = ws + L.a;
  char* B = ws + L.b;
  void* gws = ws + L.gemm;
  size_t gws_bytes = 0;
  rc = inl_linear_workspace_size(&gws_bytes);
  if (rc) return rc;

  // the attention plan of this batch, used by every layer
  const int dt = c.dtype, es = dtype_size(dt);
  const int64_t qd = (int64_t)c.heads * c.head_dim, kvd = (int64_t)c.kv_heads * c.head_dim;
  const int64_t qkv_w = qd + 2 * kvd;
  inl_attn_desc ad{};
  ad.n_texts = n_texts;
  ad.cu_seqlens_host = cu;
  ad.h_q = c.heads;
  ad.h_kv = c.kv_heads;
  ad.head_dim = c.head_dim;
  ad.causal = 1;
  ad.window = -1;
  ad.scale = 1.0f / std::sqrt((float)c.head_dim);
  ad.dtype = dt;
  ad.out_dtype = dt;
  ad.q_row_stride = ad.k_row_stride = ad.v_row_stride = L.a_w;
  ad.o_row_stride = L.b_w;
  ad.flags = c.attn_flags;
  inl_attn_plan* plan = nullptr;
  std::vector<char> blob;
  rc = attn_plan_prepare(&ad, ws + L.sched, L.gemm - L.sched, &blob, &plan);
  if (rc) return rc;

  // Uploads from the runner's pinned staging buffer: ids, text-local
  // positions and offsets (the workspace's first three regions, mirrored byte
  // for byte), then the plan's schedule.
  {
    std::lock_guard<std::mutex> lock(e->stage_mu);
    const size_t head = L.cu + (size_t)(n_texts + 1) * 4;   // L.ids == 0
    rc = e->stage.reserve(up256(head) + blob.size());
    if (!rc) {
      char* hb = e->stage.buf;
      std::memcpy(hb + L.ids, ids_host, (size_t)n * 4);
      rc = inl_positions_host(n_texts, cu, (int32_t*)(hb + L.pos));
      std::memcpy(hb + L.cu, cu, (size_t)(n_texts + 1) * 4);
      hipError_t err = rc ? hipSuccess : hipMemcpyAsync(ws, hb, head, hipMemcpyHostToDevice, st);
      if (!rc && err == hipSuccess && !blob.empty()) {
        std::memcpy(hb + up256(head), blob.data(), blob.size());
        err = hipMemcpyAsync(ws + L.sched, hb + up256(head), blob.size(), hipMemcpyHostToDevice, st);
      }
      if (err != hipSuccess) rc = hip_fail(err, "qwen3: uploads");
      if (!rc) rc = e->stage.record(st);
    }
  }
  if (rc) {
    (void)inl_attn_plan_destroy(plan);
    return rc;
  }

  // the launch sequence, onto stream `sq` (the caller's, or the capture stream)
  auto sequence = [&](void* sq) -> int {
  inl_norm_rope_desc nr{};
  nr.n_tokens = n;
  nr.head_dim = c.head_dim;
  nr.x_row_stride = nr.y_row_stride = L.a_w;
  nr.dtype = nr.out_dtype = dt;
  nr.norm = 1;
  nr.eps = c.eps;
  nr.rotary_dim = c.head_dim;
  nr.sections = 1;
  nr.table_rows = c.max_positions;
  // in bf16 the reference keeps its tables and the normed q/k in bf16
  nr.round_tables = nr.round_norm = dt == INL_BF16;

  void* stream = sq;
  int rc = inl_embed_fwd(n, d_ids, e->embed, c.vocab, c.hidden, dt, resid, c.hidden, stream);
  for (int i = 0; i < c.layers && !rc; ++i) {
    const inl_qwen3_layer_weights& w = e->layers[i];
    rc = inl_rms_norm_rows_fwd(n, c.hidden, resid, c.hidden, w.input_norm, dt, c.eps, dt, x, c.hidden, stream);
    if (!rc) rc = inl_linear_fwd(n, qkv_w, c.hidden, dt, x, c.hidden, w.qkv_proj, c.hidden, dt, A, L.a_w, 1.f, 0.f,
                                 gws, gws_bytes, stream);
    if (!rc && c.heads % 4 == 0) {
      // q and k heads are adjacent in the QKV row: one launch, k_norm from head `heads` on
      nr.heads = c.heads + c.kv_heads;
      rc = norm_rope_launch(&nr, A, A, w.q_norm, w.k_norm, c.heads, d_pos, e->cos, e->sin, nullptr, nullptr,
                            stream);
    } else if (!rc) {
      nr.heads = c.heads;
      rc = inl_norm_rope_fwd(&nr, A, A, w.q_norm, d_pos, e->cos, e->sin, nullptr, nullptr, stream);
      if (!rc) {
        nr.heads = c.kv_heads;
        rc = inl_norm_rope_fwd(&nr, A + qd * es, A + qd * es, w.k_norm, d_pos, e->cos, e->sin, nullptr, nullptr,
                               stream);
      }
    }
    if (!rc) rc = inl_attn_fwd(plan, A, A + qd * es, A + (qd + kvd) * es, B, stream);
    if (!rc) rc = inl_linear_fwd(n, c.hidden, qd, dt, B, L.b_w, w.o_proj, qd, INL_F32, resid, c.hidden, 1.f, 1.f,
                                 gws, gws_bytes, stream);
    if (!rc) rc = inl_rms_norm_rows_fwd(n, c.hidden, resid, c.hidden, w.post_attention_norm, dt, c.eps, dt, x,
                                        c.hidden, stream);
    if (!rc) rc = inl_linear_fwd(n, 2 * (int64_t)c.intermediate, c.hidden, dt, x, c.hidden, w.gate_up_proj, c.hidden,
                                 dt, A, L.a_w, 1.f, 0.f, gws, gws_bytes, stream);
    if (!rc) rc = inl_swiglu_fwd(n, c.intermediate, dt, A, L.a_w, B, L.b_w, stream);
    if (!rc) rc = inl_linear_fwd(n, c.hidden, c.intermediate, dt, B, L.b_w, w.down_proj, c.intermediate, INL_F32,
                                 resid, c.hidden, 1.f, 1.f, gws, gws_bytes, stream);
  }
  if (!rc) rc = inl_pool_last_fwd(n_texts, d_cu, c.hidden, c.hidden, INL_F32, resid, e->final_norm_f32, c.eps, 0,
                                  out, stream);
  return rc;
  };

  rc = run_sequence(e, n_texts, cu, workspace, out, st, sequence);
  const int rc2 = inl_attn_plan_destroy(plan);
  return rc ? rc : rc2;
}
