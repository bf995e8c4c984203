// EmbeddingGemma 2 text-tower runner: Gemma2Model::forward_pooled of
// crates/inl-text/src/gemma2.rs (:612-662) on one GPU, over packed texts,
// composed from the library's entry points and three element-wise kernels of
// its own:
//
//   h   = embed(ids) * sqrt(hidden)              (f32 residual stream; the
//                                                 scale rounded to bf16 in
//                                                 bf16, as :576-587 does)
//   per layer (Layer::forward, :473-494):
//     p   = rms_norm(h0 . Wple_i^T / sqrt(hidden)) * ple_norm, h0 the scaled
//           embedding and Wple_i this layer's rows of the per-layer-input
//           projection (:625-628, one layer's slice at a time)
//     x   = rms_norm(h) * input_norm
//     qkv = x . [Wq; Wk; Wv]^T                   (inl_gemm_bf16_fwd in bf16,
//                                                 inl_linear_fwd in f32)
//     q, k = rope(rms_norm(q|k) * q|k_norm); v = rms_norm(v)   (:389-408,
//                                                 inl_norm_rope_fwd)
//     a   = attention, scale 1, bidirectional; sliding layers windowed
//                                                (:409-441, inl_attn_fwd)
//     h  += rms_norm(a . Wo^T) * post_attention_norm
//     m   = gelu_tanh(x' . Wgate^T) * (x' . Wup^T), x' = rms_norm(h) *
//           pre_feedforward_norm                 (:249-254)
//     h  += rms_norm(m . Wdown^T) * post_feedforward_norm
//     g   = gelu_tanh(h . Wgate_ple^T) * per_layer[:, layer]      (:279-283)
//     h   = (h + rms_norm(g . Wproj_ple^T) * post_ple_norm) * layer_scalar
//   e   = l2(mean over each text of rms_norm(h) * norm, projected)
//                                                (:647-661)
//
// Every "h += rms_norm(t) * w" is one pass of post_add_kernel, which also
// writes the next GEMM's input (the next norm of h, or h itself in the GEMM
// dtype). The attention plans (one per distinct layer shape: window, head
// dim, KV heads) are built once per call into the workspace.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/inl_encoder.h"
#include "inl_common.hpp"
#include "lanes.hpp"

struct inl_gemma2 {
  inl_gemma2_config cfg;
  const void* embed = nullptr;
  const void* ple_proj = nullptr;
  const void* ple_norm = nullptr;
  const void* final_norm = nullptr;
  const void* emb_proj = nullptr;
  std::vector<inl_gemma2_layer_weights> layers;
  int hd_kind[2] = {0, 0};            // head_dim of the RoPE table of sliding (0) and full (1) layers
  float* cos[2] = {nullptr, nullptr};  // device, owned: [max_positions, hd_kind / 2]
  float* sin[2] = {nullptr, nullptr};
  std::mutex mu;                       // one encode at a time (the staging buffer is shared)
  inl::HostStage stage;                // pinned source of the per-call uploads
};

namespace inl {

namespace {

template <typename T>
__device__ __forceinline__ float ldv(const char* p, int64_t i) {
  if constexpr (sizeof(T) == 2) return (float)reinterpret_cast<const bf16*>(p)[i];
  else return reinterpret_cast<const float*>(p)[i];
}
template <typename T>
__device__ __forceinline__ void stv(char* p, int64_t i, float v) {
  if constexpr (sizeof(T) == 2) reinterpret_cast<bf16*>(p)[i] = (bf16)v;
  else reinterpret_cast<float*>(p)[i] = v;
}

// h[t, :] = f32(table[ids[t], :]) * scale, and x[t, :] = h[t, :] in TX (the
// input of the per-layer-input projections). The host checks the ids.
template <typename TT, typename TX>
__global__ __launch_bounds__(256) void embed_scale_kernel(const int32_t* ids, const char* table, int32_t hidden,
                                                          float scale, float* h, char* x) {
  const int64_t t = blockIdx.x;
  const int64_t row = (int64_t)ids[t] * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float v = ldv<TT>(table, row + i);
    if constexpr (sizeof(TT) == 2) v = (float)(bf16)(v * scale);   // the reference's product is bf16
    else v *= scale;
    h[t * hidden + i] = v;
    stv<TX>(x, t * hidden + i, v);
  }
}

// One wave per row of `dim` (<= 64 * NPL) values:
//   h = (h + t / sqrt(mean(t^2) + eps) * w1) * s       (s = *scalar, or 1)
//   x = h / sqrt(mean(h^2) + eps) * w2   if w2, else x = h   (in TX)
// t and h are f32; w1, w2 and the scalar are in TW.
template <typename TW, typename TX, int NPL>
__global__ __launch_bounds__(256) void post_add_kernel(int64_t rows, int32_t dim, float* h, const float* t,
                                                       const char* w1, const char* scalar, float eps,
                                                       const char* w2, char* x) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float* hr = h + r * dim;
  const float* tr = t + r * dim;
  float tv[NPL], hv[NPL];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = lane + 64 * j;
    tv[j] = i < dim ? tr[i] : 0.f;
    hv[j] = i < dim ? hr[i] : 0.f;
    ss += tv[j] * tv[j];
  }
  const float inv1 = 1.0f / sqrtf(wave_sum(ss) / (float)dim + eps);
  const float s = scalar ? ldv<TW>(scalar, 0) : 1.f;
  float ss2 = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int i = lane + 64 * j;
    if (i < dim) {
      hv[j] = (hv[j] + tv[j] * inv1 * ldv<TW>(w1, i)) * s;
      hr[i] = hv[j];
    }
    ss2 += hv[j] * hv[j];
  }
  char* xr = x + r * dim * (int64_t)sizeof(TX);
  if (w2) {
    const float inv2 = 1.0f / sqrtf(wave_sum(ss2) / (float)dim + eps);
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = lane + 64 * j;
      if (i < dim) stv<TX>(xr, i, hv[j] * inv2 * ldv<TW>(w2, i));
    }
  } else {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = lane + 64 * j;
      if (i < dim) stv<TX>(xr, i, hv[j]);
    }
  }
}

// post_add_kernel with 16-byte accesses: lane l handles the 4-element
// groups l, l + 64, ... of the row (dim a multiple of 4, rows and weights
// 16-byte / 8-byte aligned), NV groups at most. t and h stream with the
// non-temporal policy: nothing reads t again, and h only after the next
// GEMMs; x, which the next GEMM reads at once, is stored normally. (On the
// configuration-3 encode: 272 -> 225 us per call.)
template <typename TW, typename TX, int NV>
__global__ __launch_bounds__(256) void post_add_vec_kernel(int64_t rows, int32_t dim, float* h, const float* t,
                                                           const char* w1, const char* scalar, float eps,
                                                           const char* w2, char* x) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int ng = dim >> 2;
  f32x4* hr = reinterpret_cast<f32x4*>(h + r * dim);
  const f32x4* tr = reinterpret_cast<const f32x4*>(t + r * dim);
  auto w4 = [&](const char* w, int g) __attribute__((always_inline)) {
    f32x4 o;
    if constexpr (sizeof(TW) == 2) {
      const bf16x4 b = reinterpret_cast<const bf16x4*>(w)[g];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (float)b[e];
    } else {
      o = reinterpret_cast<const f32x4*>(w)[g];
    }
    return o;
  };
  f32x4 tv[NV], hv[NV];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int g = lane + 64 * j;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    tv[j] = g < ng ? __builtin_nontemporal_load(&tr[g]) : z;
    hv[j] = g < ng ? __builtin_nontemporal_load(&hr[g]) : z;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += tv[j][e] * tv[j][e];
  }
  const float inv1 = 1.0f / sqrtf(wave_sum(ss) / (float)dim + eps);
  const float s = scalar ? ldv<TW>(scalar, 0) : 1.f;
  float ss2 = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int g = lane + 64 * j;
    if (g < ng) {
      const f32x4 wv = w4(w1, g);
#pragma unroll
      for (int e = 0; e < 4; ++e) hv[j][e] = (hv[j][e] + tv[j][e] * inv1 * wv[e]) * s;
      __builtin_nontemporal_store(hv[j], &hr[g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) ss2 += hv[j][e] * hv[j][e];
    }
  }
  char* xr = x + r * dim * (int64_t)sizeof(TX);
  const float inv2 = w2 ? 1.0f / sqrtf(wave_sum(ss2) / (float)dim + eps) : 1.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int g = lane + 64 * j;
    if (g < ng) {
      f32x4 o = hv[j];
      if (w2) {
        const f32x4 wv = w4(w2, g);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = o[e] * inv2 * wv[e];
      }
      if constexpr (sizeof(TX) == 2) {
        bf16x4 b;
#pragma unroll
        for (int e = 0; e < 4; ++e) b[e] = (bf16)o[e];
        reinterpret_cast<bf16x4*>(xr)[g] = b;
      } else {
        reinterpret_cast<f32x4*>(xr)[g] = o;
      }
    }
  }
}

// y[r, i] = gelu_tanh(a[r, i]) * b[r, i], i < n, all in T, rows strided
// (elements): the GEGLU gate of the MLP and of the per-layer-input block.
// gelu_tanh(v) = v / 2 * (1 + tanh(sqrt(2 / pi) * (v + 0.044715 v^3))) in f32.
template <typename T>
__global__ __launch_bounds__(256) void gelu_gate_kernel(int64_t rows, int32_t n, const char* a, int64_t as,
                                                        const char* b, int64_t bs, char* y, int64_t ys) {
  const int64_t total = rows * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / n;
    const int i = (int)(e - r * n);
    const float v = ldv<T>(a, r * as + i);
    const float g = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    stv<T>(y, r * ys + i, g * ldv<T>(b, r * bs + i));
  }
}

// y[i] = x[i] (f32) in T
template <typename T>
__global__ __launch_bounds__(256) void cast_kernel(int64_t n, const float* x, char* y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    stv<T>(y, i, x[i]);
}

int grid_for(int64_t n) { return (int)std::min<int64_t>((n + 255) / 256, 8192); }

// Row counts above which a forward is refused when any of its GEMMs would go
// to hipBLASLt (f32 runners, or bf16 shapes outside the hand-written GEMM's
// limits): hipBLASLt's own initialisation failed ("Could not initialize
// Tensile host") in the one configuration-3 run that reached it with
// 139,124 rows, and the process then crashed inside the library; the
// largest row count it has passed tests with here is 1,408.
constexpr int64_t kLibGemmMaxRows = 16384;

bool own_gemm_ok(int64_t n, int64_t k, int64_t xs, int64_t ws, int64_t ys) {
  return k % 32 == 0 && n % 8 == 0 && xs % 8 == 0 && ws % 8 == 0 && ys % 8 == 0;
}

// The runner's GEMMs: bf16 ones on the hand-written kernel when the shape is
// within its limits (every shape of the real EmbeddingGemma 2 text tower is),
// f32 ones and any other shape on hipBLASLt (inl_linear_fwd).
int gemm(int32_t dt, int64_t m, int64_t n, int64_t k, const void* x, int64_t xs, const void* w, int64_t ws,
         int32_t out_dt, void* y, int64_t ys, float alpha, void* gws, size_t gws_bytes, void* stream) {
  if (dt == INL_BF16 && own_gemm_ok(n, k, xs, ws, ys))
    return inl_gemm_bf16_fwd(m, n, k, x, xs, w, ws, out_dt, y, ys, alpha, 0.f, stream);
  return inl_linear_fwd(m, n, k, dt, x, xs, w, ws, out_dt, y, ys, alpha, 0.f, gws, gws_bytes, stream);
}

int launch_post_add(int dt, int64_t rows, int32_t dim, float* h, const float* t, const void* w1, const void* scalar,
                    float eps, const void* w2, void* x, hipStream_t st) {
  if (rows == 0) return INL_OK;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  const char *a = (const char*)w1, *s = (const char*)scalar, *b = (const char*)w2;
  char* xo = (char*)x;
  const uintptr_t wal = dt == INL_BF16 ? 7 : 15;
  if (dim % 4 == 0 && dim <= 64 * 4 * 4 && ((uintptr_t)h & 15) == 0 && ((uintptr_t)t & 15) == 0 &&
      ((uintptr_t)x & wal) == 0 && ((uintptr_t)w1 & wal) == 0 && ((uintptr_t)w2 & wal) == 0) {
    if (dt == INL_BF16) hipLaunchKernelGGL((post_add_vec_kernel<bf16, bf16, 4>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
    else hipLaunchKernelGGL((post_add_vec_kernel<float, float, 4>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
    INL_HIP_TRY(hipGetLastError());
    return INL_OK;
  }
  if (dt == INL_BF16) {
    if (dim <= 64 * 16) hipLaunchKernelGGL((post_add_kernel<bf16, bf16, 16>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
    else hipLaunchKernelGGL((post_add_kernel<bf16, bf16, 64>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
  } else {
    if (dim <= 64 * 16) hipLaunchKernelGGL((post_add_kernel<float, float, 16>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
    else hipLaunchKernelGGL((post_add_kernel<float, float, 64>), grid, block, 0, st, rows, dim, h, t, a, s, eps, b, xo);
  }
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

int launch_gelu_gate(int dt, int64_t rows, int32_t n, const void* a, int64_t as, const void* b, int64_t bs, void* y,
                     int64_t ys, hipStream_t st) {
  if (rows == 0 || n == 0) return INL_OK;
  const int grid = grid_for(rows * n);
  if (dt == INL_BF16)
    hipLaunchKernelGGL(gelu_gate_kernel<bf16>, dim3(grid), dim3(256), 0, st, rows, n, (const char*)a, as,
                       (const char*)b, bs, (char*)y, ys);
  else
    hipLaunchKernelGGL(gelu_gate_kernel<float>, dim3(grid), dim3(256), 0, st, rows, n, (const char*)a, as,
                       (const char*)b, bs, (char*)y, ys);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

struct LayerShape {
  int hd, kvh, full;
};
LayerShape shape_of(const inl_gemma2* e, int i) {
  const inl_gemma2_layer_weights& w = e->layers[i];
  return {w.head_dim > 0 ? w.head_dim : e->cfg.head_dim, w.kv_heads > 0 ? w.kv_heads : e->cfg.kv_heads,
          w.full ? 1 : 0};
}

// Distinct attention shapes of the layers: (window, head_dim, kv_heads).
typedef std::tuple<int, int, int> AttnKey;

struct Layout {
  size_t ids, pos, cu, h, x0, x, a, b, t, ple, pooled, pooled_dt, proj, gemm, total;
  int64_t a_w, b_w;
  std::vector<AttnKey> keys;
  std::vector<size_t> sched, sched_bytes;
};

inl_attn_desc attn_desc(const inl_gemma2* e, int32_t n_texts, const int32_t* cu, const AttnKey& k, const Layout& L) {
  const inl_gemma2_config& c = e->cfg;
  inl_attn_desc d{};
  d.n_texts = n_texts;
  d.cu_seqlens_host = cu;
  d.h_q = c.heads;
  d.h_kv = std::get<2>(k);
  d.head_dim = std::get<1>(k);
  d.causal = 0;
  d.window = std::get<0>(k);
  d.scale = 1.0f;
  d.dtype = c.dtype;
  d.out_dtype = c.dtype;
  d.q_row_stride = d.k_row_stride = d.v_row_stride = L.a_w;
  d.o_row_stride = L.b_w;
  d.flags = c.attn_flags;
  return d;
}

int layout(const inl_gemma2* e, int32_t n_texts, const int32_t* cu, Layout* L) {
  const inl_gemma2_config& c = e->cfg;
  const int64_t n = n_texts > 0 ? cu[n_texts] : 0;
  const int es = dtype_size(c.dtype);
  int64_t qkv_w = 0, q_w = 0;
  L->keys.clear();
  for (int i = 0; i < c.layers; ++i) {
    const LayerShape s = shape_of(e, i);
    qkv_w = std::max<int64_t>(qkv_w, (int64_t)(c.heads + 2 * s.kvh) * s.hd);
    q_w = std::max<int64_t>(q_w, (int64_t)c.heads * s.hd);
    const AttnKey k{s.full ? -1 : c.sliding_window, s.hd, s.kvh};
    if (std::find(L->keys.begin(), L->keys.end(), k) == L->keys.end()) L->keys.push_back(k);
  }
  L->a_w = std::max<int64_t>(std::max<int64_t>(qkv_w, 2 * (int64_t)c.intermediate), c.ple_dim);
  L->b_w = std::max<int64_t>(std::max<int64_t>(q_w, c.intermediate), c.ple_dim);
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += up256(bytes); return o; };
  L->ids = take(n * 4);
  L->pos = take(n * 4);
  L->cu = take((size_t)(n_texts + 1) * 4);
  L->h = take((size_t)n * c.hidden * 4);
  L->x0 = take((size_t)n * c.hidden * es);
  L->x = take((size_t)n * c.hidden * es);
  L->a = take((size_t)n * L->a_w * es);
  L->b = take((size_t)n * L->b_w * es);
  L->t = take((size_t)n * std::max(c.hidden, c.ple_dim) * 4);
  L->ple = take((size_t)n * c.ple_dim * es);
  L->pooled = take((size_t)n_texts * c.hidden * 4);
  L->pooled_dt = take((size_t)n_texts * c.hidden * es);
  L->proj = take((size_t)n_texts * c.embedding_dim * 4);
  L->sched.clear();
  L->sched_bytes.clear();
  for (const AttnKey& k : L->keys) {
    const inl_attn_desc d = attn_desc(e, n_texts, cu, k, *L);
    size_t sched = 0;
    const int rc = inl_attn_workspace_size(&d, &sched);
    if (rc) return rc;
    sched = std::max<size_t>(sched, 16);
    L->sched.push_back(take(sched));
    L->sched_bytes.push_back(up256(sched));
  }
  size_t gemm = 0;
  const int rc = inl_linear_workspace_size(&gemm);
  if (rc) return rc;
  L->gemm = take(gemm);
  L->total = off;
  return INL_OK;
}

// Whether every GEMM of an encode goes to the hand-written bf16 kernel.
bool all_own_gemms(const inl_gemma2* e, const Layout& L) {
  const inl_gemma2_config& c = e->cfg;
  if (c.dtype != INL_BF16) return false;
  const int64_t H = c.hidden, I = c.intermediate, E = c.ple_dim;
  bool ok = own_gemm_ok(E, H, H, H, E) && own_gemm_ok(2 * I, H, H, H, L.a_w) && own_gemm_ok(H, I, L.b_w, I, H) &&
            own_gemm_ok(E, H, H, H, L.a_w) && own_gemm_ok(H, E, L.b_w, E, H) &&
            own_gemm_ok(c.embedding_dim, H, H, H, c.embedding_dim);
  for (int i = 0; i < c.layers && ok; ++i) {
    const LayerShape s = shape_of(e, i);
    const int64_t qd = (int64_t)c.heads * s.hd, kvd = (int64_t)s.kvh * s.hd;
    ok = own_gemm_ok(qd + 2 * kvd, H, H, H, L.a_w) && own_gemm_ok(H, qd, L.b_w, qd, H);
  }
  return ok;
}

int check_config(const inl_gemma2_config* c) {
  if (!c) return fail(INL_E_INVALID, "gemma2: config is NULL");
  if (c->vocab <= 0 || c->hidden <= 0 || c->intermediate <= 0 || c->layers <= 0 || c->heads <= 0 ||
      c->kv_heads <= 0 || c->head_dim <= 0 || c->ple_dim <= 0 || c->embedding_dim <= 0 || c->sliding_window < 0 ||
      c->max_positions <= 0 || !(c->eps >= 0.f) || !(c->theta_sliding > 0.0) || !(c->theta_full > 0.0) ||
      !dtype_ok(c->dtype))
    return fail(INL_E_INVALID, "gemma2: bad config");
  if (c->hidden % 8 || c->intermediate % 8 || c->ple_dim % 8 || c->embedding_dim % 4)
    return fail(INL_E_UNSUPPORTED,
                "gemma2: hidden, intermediate and ple_dim must be multiples of 8, embedding_dim of 4");
  if (c->hidden > 64 * 64) return fail(INL_E_UNSUPPORTED, "gemma2: hidden above 4096");
  return INL_OK;
}

int check_shape(const inl_gemma2_config* c, int i, int hd, int kvh) {
  // the attention kernels take head_dim up to 256 (inl_attn_* refuses more)
  const bool pow2 = hd >= 8 && hd <= 256 && hd % 8 == 0 && ((hd / 8) & (hd / 8 - 1)) == 0;
  if (!pow2 || kvh <= 0 || c->heads % kvh)
    return fail(INL_E_UNSUPPORTED, "gemma2: layer " + std::to_string(i) + ": head_dim must be 8 x a power of two "
                                   "up to 256 and the KV heads must divide the heads");
  return INL_OK;
}

}  // namespace

}  // namespace inl

extern "C" int inl_gemma2_create(const inl_gemma2_config* cfg, const void* embed_tokens,
                                 const inl_gemma2_layer_weights* layers, const void* ple_model_projection,
                                 const void* ple_norm, const void* final_norm, const void* embedding_projection,
                                 inl_gemma2** enc) {
  using namespace inl;
  if (!enc) return fail(INL_E_INVALID, "gemma2: encoder out-pointer is NULL");
  *enc = nullptr;
  int rc = check_config(cfg);
  if (rc) return rc;
  if (!embed_tokens || !layers || !ple_model_projection || !ple_norm || !final_norm || !embedding_projection)
    return fail(INL_E_INVALID, "gemma2: NULL weights");
  for (int i = 0; i < cfg->layers; ++i) {
    const inl_gemma2_layer_weights& l = layers[i];
    if (!l.qkv_proj || !l.o_proj || !l.gate_up_proj || !l.down_proj || !l.q_norm || !l.k_norm || !l.input_norm ||
        !l.post_attention_norm || !l.pre_feedforward_norm || !l.post_feedforward_norm || !l.ple_input_gate ||
        !l.ple_projection || !l.ple_post_norm || !l.layer_scalar)
      return fail(INL_E_INVALID, "gemma2: NULL weight in layer " + std::to_string(i));
    rc = check_shape(cfg, i, l.head_dim > 0 ? l.head_dim : cfg->head_dim, l.kv_heads > 0 ? l.kv_heads : cfg->kv_heads);
    if (rc) return rc;
  }
  inl_gemma2* e = new (std::nothrow) inl_gemma2();
  if (!e) return fail(INL_E_NOMEM, "gemma2: host allocation failed");
  e->cfg = *cfg;
  e->embed = embed_tokens;
  e->ple_proj = ple_model_projection;
  e->ple_norm = ple_norm;
  e->final_norm = final_norm;
  e->emb_proj = embedding_projection;
  e->layers.assign(layers, layers + cfg->layers);
  // one table per layer kind, at the head_dim of the first layer of that kind (gemma2.rs:566-573)
  for (int kind = 0; kind < 2 && !rc; ++kind) {
    e->hd_kind[kind] = -1;
    for (int i = 0; i < cfg->layers; ++i) {
      if ((layers[i].full ? 1 : 0) != kind) continue;
      const int hd = layers[i].head_dim > 0 ? layers[i].head_dim : cfg->head_dim;
      if (e->hd_kind[kind] < 0) e->hd_kind[kind] = hd;
      else if (hd != e->hd_kind[kind])   // the kind's one RoPE table must fit every layer of it
        rc = fail(INL_E_UNSUPPORTED, "gemma2: layers of one kind must share a head_dim (one RoPE table per kind)");
    }
    if (e->hd_kind[kind] < 0) e->hd_kind[kind] = cfg->head_dim;
  }
  for (int kind = 0; kind < 2 && !rc; ++kind) {
    const int half = e->hd_kind[kind] / 2;
    std::vector<float> c((size_t)cfg->max_positions * half), s(c.size());
    rc = inl_rope_table_host(e->hd_kind[kind], kind ? cfg->theta_full : cfg->theta_sliding, cfg->max_positions, 0,
                             c.data(), s.data());
    if (rc) break;
    hipError_t err = hipMalloc(&e->cos[kind], c.size() * 4);
    if (err == hipSuccess) err = hipMalloc(&e->sin[kind], s.size() * 4);
    if (err == hipSuccess) err = hipMemcpy(e->cos[kind], c.data(), c.size() * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(e->sin[kind], s.data(), s.size() * 4, hipMemcpyHostToDevice);
    if (err != hipSuccess) rc = hip_fail(err, "gemma2: setting up RoPE tables");
  }
  if (rc) {
    (void)inl_gemma2_destroy(e);
    return rc;
  }
  *enc = e;
  return INL_OK;
}

extern "C" int inl_gemma2_destroy(inl_gemma2* e) {
  if (!e) return INL_OK;
  for (int k = 0; k < 2; ++k)
    for (float* p : {e->cos[k], e->sin[k]})
      if (p) (void)hipFree(p);
  delete e;
  return INL_OK;
}

extern "C" int inl_gemma2_workspace_size(const inl_gemma2* e, int32_t n_texts, const int32_t* cu, size_t* bytes) {
  using namespace inl;
  if (!e || !bytes || n_texts < 0 || (n_texts > 0 && !cu)) return fail(INL_E_INVALID, "gemma2: bad arguments");
  int64_t total = 0;
  int rc = check_cu(n_texts, cu, &total);
  if (rc) return rc;
  Layout L;
  rc = layout(e, n_texts, cu, &L);
  if (rc) return rc;
  *bytes = L.total;
  return INL_OK;
}

extern "C" int inl_gemma2_encode(inl_gemma2* e, int32_t n_texts, const int32_t* cu, const int32_t* ids_host,
                                 int32_t out_dim, float* out, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace inl;
  if (!e || n_texts < 0 || (n_texts > 0 && (!cu || !out))) return fail(INL_E_INVALID, "gemma2: bad arguments");
  const inl_gemma2_config& c = e->cfg;
  if (out_dim <= 0 || out_dim > c.embedding_dim)
    return fail(INL_E_INVALID, "gemma2: out_dim must be in [1, embedding_dim]");
  if (n_texts == 0) return INL_OK;
  int64_t n = 0;
  int rc = check_cu(n_texts, cu, &n);
  if (rc) return rc;
  for (int b = 0; b < n_texts; ++b) {
    const int32_t t = cu[b + 1] - cu[b];
    if (t <= 0) return fail(INL_E_INVALID, "gemma2: text " + std::to_string(b) + " is empty");
    if (t > c.max_positions)
      return fail(INL_E_INVALID, "gemma2: text " + std::to_string(b) + " is longer than max_positions");
  }
  if (!ids_host) return fail(INL_E_INVALID, "gemma2: ids_host is NULL");
  for (int64_t i = 0; i < n; ++i)
    if (ids_host[i] < 0 || ids_host[i] >= c.vocab)
      return fail(INL_E_INVALID, "gemma2: token id " + std::to_string(ids_host[i]) + " at " + std::to_string(i) +
                                     " is outside the vocabulary");
  Layout L;
  rc = layout(e, n_texts, cu, &L);
  if (rc) return rc;
  if (!workspace || workspace_bytes < L.total || ((uintptr_t)workspace & 255))
    return fail(INL_E_INVALID,
                "gemma2: workspace is NULL, unaligned (256 B) or smaller than inl_gemma2_workspace_size()");
  if (n > kLibGemmMaxRows && !all_own_gemms(e, L))
    return fail(INL_E_UNSUPPORTED, "gemma2: " + std::to_string(n) + " tokens: batches above " +
                                       std::to_string(kLibGemmMaxRows) +
                                       " tokens run only when every GEMM is on the library's own bf16 kernel "
                                       "(bf16 weights, widths and strides multiples of 8, inner sizes of 32)");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int32_t* d_ids = (int32_t*)(ws + L.ids);
  int32_t* d_pos = (int32_t*)(ws + L.pos);
  int32_t* d_cu = (int32_t*)(ws + L.cu);
  float* h = (float*)(ws + L.h);
  char* x0 = ws + L.x0;
  char* x = ws + L.x;
  char* A = ws + L.a;
  char* B = ws + L.b;
  float* T = (float*)(ws + L.t);
  char* P = ws + L.ple;
  float* pooled = (float*)(ws + L.pooled);
  char* pooled_dt = ws + L.pooled_dt;
  float* proj = (float*)(ws + L.proj);
  void* gws = ws + L.gemm;
  size_t gws_bytes = 0;
  rc = inl_linear_workspace_size(&gws_bytes);
  if (rc) return rc;

  // Uploads, all from the runner's pinned staging buffer: token ids,
  // text-local positions and offsets (the workspace's first three regions,
  // mirrored byte for byte in the buffer), then each attention plan's
  // schedule (one plan per distinct layer shape, used by every layer of it).
  std::lock_guard<std::mutex> lock(e->mu);
  std::vector<std::vector<char>> blobs(L.keys.size());
  std::vector<inl_attn_plan*> plans(L.keys.size(), nullptr);
  auto destroy_plans = [&]() {
    int r = INL_OK;
    for (inl_attn_plan* p : plans)
      if (p) {
        const int r2 = inl_attn_plan_destroy(p);
        if (!r) r = r2;
      }
    return r;
  };
  for (size_t k = 0; k < L.keys.size() && !rc; ++k) {
    const inl_attn_desc d = attn_desc(e, n_texts, cu, L.keys[k], L);
    rc = attn_plan_prepare(&d, ws + L.sched[k], L.sched_bytes[k], &blobs[k], &plans[k]);
  }
  const size_t head = L.cu + (size_t)(n_texts + 1) * 4;   // L.ids == 0
  size_t need = up256(head);
  for (const std::vector<char>& b : blobs) need += up256(b.size());
  if (!rc) rc = e->stage.reserve(need);
  if (!rc) {
    char* hb = e->stage.buf;
    std::memcpy(hb + L.ids, ids_host, (size_t)n * 4);
    rc = inl_positions_host(n_texts, cu, (int32_t*)(hb + L.pos));
    std::memcpy(hb + L.cu, cu, (size_t)(n_texts + 1) * 4);
    hipError_t err = rc ? hipSuccess : hipMemcpyAsync(ws, hb, head, hipMemcpyHostToDevice, st);
    size_t off = up256(head);
    for (size_t k = 0; k < blobs.size() && !rc && err == hipSuccess; ++k) {
      if (blobs[k].empty()) continue;
      std::memcpy(hb + off, blobs[k].data(), blobs[k].size());
      err = hipMemcpyAsync(ws + L.sched[k], hb + off, blobs[k].size(), hipMemcpyHostToDevice, st);
      off += up256(blobs[k].size());
    }
    if (err != hipSuccess) rc = hip_fail(err, "gemma2: uploads");
    if (!rc) rc = e->stage.record(st);
  }
  if (rc) {
    (void)destroy_plans();
    return rc;
  }

  const int dt = c.dtype, es = dtype_size(dt);
  const int64_t H = c.hidden, I = c.intermediate, E = c.ple_dim;
  // embedding scale: sqrt(hidden), rounded to bf16 in bf16 (gemma2.rs:576-587)
  float scale = (float)std::sqrt((double)c.hidden);
  if (dt == INL_BF16) scale = (float)(bf16)scale;
  if (!rc) {
    if (dt == INL_BF16)
      hipLaunchKernelGGL((embed_scale_kernel<bf16, bf16>), dim3((unsigned)n), dim3(256), 0, st, d_ids,
                         (const char*)e->embed, c.hidden, scale, h, x0);
    else
      hipLaunchKernelGGL((embed_scale_kernel<float, float>), dim3((unsigned)n), dim3(256), 0, st, d_ids,
                         (const char*)e->embed, c.hidden, scale, h, x0);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) rc = hip_fail(err, "gemma2: embedding");
  }

  // layer loop
  inl_norm_rope_desc nr{};
  nr.n_tokens = n;
  nr.x_row_stride = nr.y_row_stride = L.a_w;
  nr.dtype = nr.out_dtype = dt;
  nr.norm = 1;
  nr.eps = c.eps;
  nr.sections = 1;
  nr.table_rows = c.max_positions;
  nr.round_tables = nr.round_norm = dt == INL_BF16;
  for (int i = 0; i < c.layers && !rc; ++i) {
    const inl_gemma2_layer_weights& w = e->layers[i];
    const LayerShape s = shape_of(e, i);
    const int64_t qd = (int64_t)c.heads * s.hd, kvd = (int64_t)s.kvh * s.hd, qkv_w = qd + 2 * kvd;
    const size_t pk = std::find(L.keys.begin(), L.keys.end(), AttnKey{s.full ? -1 : c.sliding_window, s.hd, s.kvh}) -
                      L.keys.begin();
    // this layer's per-layer input
    if (!rc) rc = gemm(dt, n, E, H, x0, H, (const char*)e->ple_proj + (int64_t)i * E * H * es, H, INL_F32, T, E,
                       1.0f / std::sqrt((float)c.hidden), gws, gws_bytes, stream);
    if (!rc) rc = inl_rms_norm_rows_fwd(n, c.ple_dim, T, E, e->ple_norm, dt, c.eps, dt, P, E, stream);
    if (i == 0 && !rc) rc = inl_rms_norm_rows_fwd(n, c.hidden, h, H, w.input_norm, dt, c.eps, dt, x, H, stream);
    if (!rc) rc = gemm(dt, n, qkv_w, H, x, H, w.qkv_proj, H, dt, A, L.a_w, 1.f, gws, gws_bytes, stream);
    // q (q_norm, rope), k (k_norm, rope) and v (weightless, no rope) of the
    // fused row in one launch
    nr.head_dim = s.hd;
    nr.rotary_dim = s.hd;
    nr.heads = c.heads + 2 * s.kvh;
    if (!rc) rc = norm_rope_launch_ex(&nr, A, A, w.q_norm, w.k_norm, c.heads, c.heads + s.kvh, c.heads + s.kvh, d_pos,
                                      e->cos[s.full], e->sin[s.full], nullptr, nullptr, stream);
    if (!rc) rc = inl_attn_fwd(plans[pk], A, A + qd * es, A + (qd + kvd) * es, B, stream);
    if (!rc) rc = gemm(dt, n, H, qd, B, L.b_w, w.o_proj, qd, INL_F32, T, H, 1.f, gws, gws_bytes, stream);
    if (!rc) rc = launch_post_add(dt, n, c.hidden, h, T, w.post_attention_norm, nullptr, c.eps, w.pre_feedforward_norm,
                                  x, st);
    // m = gelu_tanh(x . Wgate^T) * (x . Wup^T): one fused GEMM in bf16
    if (!rc && dt == INL_BF16 && own_gemm_ok(I, H, H, H, L.b_w)) {
      rc = inl_gemm_bf16_gated_fwd(n, I, H, x, H, w.gate_up_proj, H, INL_GATE_GEGLU, nullptr, 0, dt, B, L.b_w, stream);
    } else {
      if (!rc) rc = gemm(dt, n, 2 * I, H, x, H, w.gate_up_proj, H, dt, A, L.a_w, 1.f, gws, gws_bytes, stream);
      if (!rc) rc = launch_gelu_gate(dt, n, c.intermediate, A, L.a_w, A + I * es, L.a_w, B, L.b_w, st);
    }
    if (!rc) rc = gemm(dt, n, H, I, B, L.b_w, w.down_proj, I, INL_F32, T, H, 1.f, gws, gws_bytes, stream);
    if (!rc) rc = launch_post_add(dt, n, c.hidden, h, T, w.post_feedforward_norm, nullptr, c.eps, nullptr, x, st);
    // g = gelu_tanh(h . Wgate_ple^T) * per_layer: one fused GEMM in bf16
    if (!rc && dt == INL_BF16 && own_gemm_ok(E, H, H, H, L.b_w) && E % 4 == 0) {
      rc = inl_gemm_bf16_gated_fwd(n, E, H, x, H, w.ple_input_gate, H, INL_GATE_GELU_MUL, P, E, dt, B, L.b_w, stream);
    } else {
      if (!rc) rc = gemm(dt, n, E, H, x, H, w.ple_input_gate, H, dt, A, L.a_w, 1.f, gws, gws_bytes, stream);
      if (!rc) rc = launch_gelu_gate(dt, n, c.ple_dim, A, L.a_w, P, E, B, L.b_w, st);
    }
    if (!rc) rc = gemm(dt, n, H, E, B, L.b_w, w.ple_projection, E, INL_F32, T, H, 1.f, gws, gws_bytes, stream);
    const void* next_norm = i + 1 < c.layers ? e->layers[i + 1].input_norm : e->final_norm;
    if (!rc) rc = launch_post_add(dt, n, c.hidden, h, T, w.ple_post_norm, w.layer_scalar, c.eps, next_norm, x, st);
  }
  // mean of the normed final rows, projected, L2 (and Matryoshka)
  if (!rc) rc = inl_pool_mean_fwd(n_texts, d_cu, c.hidden, H, dt, x, 0, pooled, stream);
  if (!rc) {
    const int64_t m = (int64_t)n_texts * H;
    if (dt == INL_BF16)
      hipLaunchKernelGGL(cast_kernel<bf16>, dim3(grid_for(m)), dim3(256), 0, st, m, pooled, pooled_dt);
    else
      hipLaunchKernelGGL(cast_kernel<float>, dim3(grid_for(m)), dim3(256), 0, st, m, pooled, pooled_dt);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) rc = hip_fail(err, "gemma2: pooled cast");
  }
  if (!rc) rc = gemm(dt, n_texts, c.embedding_dim, H, pooled_dt, H, e->emb_proj, H, INL_F32, proj, c.embedding_dim, 1.f, gws,
                     gws_bytes, stream);
  if (!rc) {
    if (out_dim == c.embedding_dim) {
      rc = inl_l2_normalize_fwd(n_texts, c.embedding_dim, c.embedding_dim, proj, out_dim, out, 1e-12f, 0, stream);
    } else {
      rc = inl_l2_normalize_fwd(n_texts, c.embedding_dim, c.embedding_dim, proj, c.embedding_dim, proj, 1e-12f, 0,
                                stream);
      if (!rc) rc = inl_l2_normalize_fwd(n_texts, out_dim, c.embedding_dim, proj, out_dim, out, 0.f, 1, stream);
    }
  }
  const int rc2 = destroy_plans();
  return rc ? rc : rc2;
}
