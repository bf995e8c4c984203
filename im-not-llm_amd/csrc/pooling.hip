// Pooling epilogues of the encoder engines on gfx950 (HBM-bound kernels).
//
//   last-token: final RMSNorm of each text's last row + L2 normalisation
//               (crates/inl-text/src/qwen3/mod.rs:339-358, :464-469);
//   mean:       per-text mean of the rows (crates/inl-text/src/gemma2.rs:
//               647-656), optionally L2-normalised (:660-661);
//   l2:         row L2 normalisation, also Matryoshka truncate + renormalise
//               (crates/inl-text/src/native.rs:822-830);
//   SPLADE:     per-text max of the bias-free MLM logits over speaking
//               positions, ln(relu(max + bias - shift) * open + 1), then the
//               max-fold onto canonical terms
//               (crates/inl-sparse/src/modernbert.rs:806-907).
// The SPLADE max and fold are order-independent, so the output - and the
// active-term set {t : w_t > 0} - is bit-exact for given logits.

#include <cmath>

#include "inl_common.hpp"
#include "lanes.hpp"

namespace inl {

namespace {

template <typename T>
__device__ __forceinline__ float ld(const char* p) {
  if constexpr (sizeof(T) == 2) return (float)*reinterpret_cast<const bf16*>(p);
  else return *reinterpret_cast<const float*>(p);
}

// Sum of `v` over the block (blockDim.x <= 1024, multiple of 64).
__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// ---- last-token: one block per text ----
template <typename T>
__global__ __launch_bounds__(256) void pool_last_kernel(const char* hidden, int64_t stride, const int32_t* cu,
                                                        int32_t h, const char* weight, float eps,
                                                        int32_t round_norm, float* out) {
  __shared__ float red[16];
  const int b = blockIdx.x;
  const int32_t s0 = cu[b], s1 = cu[b + 1];
  float* o = out + (int64_t)b * h;
  if (s1 <= s0) {  // empty text: zero row
    for (int i = threadIdx.x; i < h; i += blockDim.x) o[i] = 0.f;
    return;
  }
  const char* row = hidden + (int64_t)(s1 - 1) * stride * (int64_t)sizeof(T);
  float ss = 0.f;
  for (int i = threadIdx.x; i < h; i += blockDim.x) {
    const float x = ld<T>(row + i * (int)sizeof(T));
    ss += x * x;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)h + eps);
  float ss2 = 0.f;
  for (int i = threadIdx.x; i < h; i += blockDim.x) {
    float y = ld<T>(row + i * (int)sizeof(T)) * inv;
    if (weight) y *= ld<T>(weight + i * (int)sizeof(T));
    if (round_norm && sizeof(T) == 2) y = (float)(bf16)y;
    o[i] = y;
    ss2 += y * y;
  }
  const float n = sqrtf(block_sum(ss2, red) + 1e-12f);
  for (int i = threadIdx.x; i < h; i += blockDim.x) o[i] = o[i] / n;
}

// ---- mean, vector form: one block of 1024 lanes per (text, column slice) ----
// 16 lanes cover a slice of 16 * VW columns of a row with one 16-byte load
// each (VW = 16 / sizeof(T)); the 64 lane rows walk the text's rows 64 apart,
// four rows per step, so each lane has four loads in flight. The 64 partial
// sums of a column are then added in a fixed order through LDS: the result
// does not depend on timing (no atomics).
template <typename T>
__global__ __launch_bounds__(1024) void pool_mean_vec_kernel(const char* hidden, int64_t stride, const int32_t* cu,
                                                             int32_t h, float* out) {
  constexpr int VW = 16 / sizeof(T);
  constexpr int COLS = 16 * VW;
  __shared__ float part[64][COLS];
  const int b = blockIdx.y;
  const int l = threadIdx.x & 15;
  const int rg = threadIdx.x >> 4;
  const int c0 = blockIdx.x * COLS + l * VW;
  const int32_t s0 = cu[b], s1 = cu[b + 1];
  float acc[VW];
#pragma unroll
  for (int e = 0; e < VW; ++e) acc[e] = 0.f;
  auto add = [&](const u32x4& w) __attribute__((always_inline)) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += __builtin_bit_cast(float, w[q] << 16);
        acc[2 * q + 1] += __builtin_bit_cast(float, w[q] & 0xffff0000u);
      }
    } else {
      // cast the whole vector: a bit_cast of one element lvalue of a vector
      // type reads element 0 here
      const f32x4 f = __builtin_bit_cast(f32x4, w);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] += f[q];
    }
  };
  if (c0 < h) {
    const char* base = hidden + (int64_t)c0 * (int64_t)sizeof(T);
    const int64_t rstep = stride * (int64_t)sizeof(T);
    int32_t r = s0 + rg;
    for (; r + 3 * 64 < s1; r += 4 * 64) {
      u32x4 w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = *reinterpret_cast<const u32x4*>(base + (int64_t)(r + 64 * k) * rstep);
#pragma unroll
      for (int k = 0; k < 4; ++k) add(w[k]);
    }
    for (; r < s1; r += 64) add(*reinterpret_cast<const u32x4*>(base + (int64_t)r * rstep));
  }
#pragma unroll
  for (int e = 0; e < VW; ++e) part[rg][l * VW + e] = acc[e];
  __syncthreads();
  if (threadIdx.x < COLS) {
    const int c = blockIdx.x * COLS + threadIdx.x;
    float sum = 0.f;
    for (int i = 0; i < 64; ++i) sum += part[i][threadIdx.x];
    const int32_t n = s1 - s0;
    if (c < h) out[(int64_t)b * h + c] = n > 0 ? sum / (float)n : 0.f;
  }
}

// ---- mean, generic form (rows or columns not 16-byte aligned): one block
// per (text, 64-column slice); 4 row phases ----
template <typename T>
__global__ __launch_bounds__(256) void pool_mean_kernel(const char* hidden, int64_t stride, const int32_t* cu,
                                                        int32_t h, float* out) {
  __shared__ float part[4][64];
  const int b = blockIdx.y;
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int phase = threadIdx.x >> 6;
  const int32_t s0 = cu[b], s1 = cu[b + 1];
  float acc = 0.f;
  if (col < h)
    for (int32_t r = s0 + phase; r < s1; r += 4)
      acc += ld<T>(hidden + ((int64_t)r * stride + col) * (int64_t)sizeof(T));
  part[phase][threadIdx.x & 63] = acc;
  __syncthreads();
  if (phase == 0 && col < h) {
    const float sum = (part[0][threadIdx.x] + part[1][threadIdx.x]) + (part[2][threadIdx.x] + part[3][threadIdx.x]);
    const int32_t n = s1 - s0;
    out[(int64_t)b * h + col] = n > 0 ? sum / (float)n : 0.f;
  }
}

// ---- row L2 normalisation: one block per row ----
__global__ __launch_bounds__(256) void l2_kernel(const float* x, int64_t xs, float* y, int64_t ys, int32_t dim,
                                                 float eps, int32_t skip_zero) {
  __shared__ float red[16];
  const float* xr = x + (int64_t)blockIdx.x * xs;
  float* yr = y + (int64_t)blockIdx.x * ys;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) ss += xr[i] * xr[i];
  const float n = sqrtf(block_sum(ss, red) + eps);
  const bool keep = skip_zero && !(n > 0.f);
  for (int i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = keep ? xr[i] : xr[i] / n;
}

// ---- SPLADE ----
constexpr int kMaxMasked = 16;
struct SpladeParams {
  const float* logits;
  int64_t stride;
  const int32_t* offs;     // [rows + 1] speaking-position offsets (device)
  const float* bias;       // [vocab] or null
  const int32_t* canonical;  // [vocab] or null
  float* out;
  int32_t direct;          // 1: logits already hold each row's maximum (offs unused)
  int32_t vocab, out_dim, n_masked;
  float shift;
  int32_t masked[kMaxMasked];
};

__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

__global__ __launch_bounds__(256) void splade_kernel(SpladeParams p) {
  const int r = blockIdx.y;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= p.vocab) return;
  const int32_t a = p.direct ? r : p.offs[r], e = p.direct ? r + 1 : p.offs[r + 1];
  // running max over the row's speaking positions (4 independent chains)
  float m0 = -INFINITY, m1 = -INFINITY, m2 = -INFINITY, m3 = -INFINITY;
  const float* col = p.logits + t;
  int32_t i = a;
  for (; i + 4 <= e; i += 4) {
    m0 = fmaxf(m0, col[(int64_t)i * p.stride]);
    m1 = fmaxf(m1, col[(int64_t)(i + 1) * p.stride]);
    m2 = fmaxf(m2, col[(int64_t)(i + 2) * p.stride]);
    m3 = fmaxf(m3, col[(int64_t)(i + 3) * p.stride]);
  }
  for (; i < e; ++i) m0 = fmaxf(m0, col[(int64_t)i * p.stride]);
  const float m = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
  // finish: relu before the 0/1 vocabulary mask, so -inf never meets a zero
  float x = p.bias ? m + p.bias[t] : m;
  x = x - p.shift;
  x = x > 0.f ? x : 0.f;
  bool open = true;
  for (int k = 0; k < p.n_masked; ++k) open = open && p.masked[k] != t;
  x = open ? x : 0.f;
  const float w = logf(x + 1.0f);
  if (p.canonical) {
    // w >= 0: unsigned order of the bits is the float order. An id outside
    // [0, out_dim) is skipped rather than written out of bounds.
    const uint32_t c = (uint32_t)p.canonical[t];
    if (c < (uint32_t)p.out_dim)
      atomicMax(reinterpret_cast<unsigned int*>(p.out + (int64_t)r * p.out_dim + c), __float_as_uint(w));
  } else {
    p.out[(int64_t)r * p.out_dim + t] = w;
  }
}

bool aligned_to(const void* ptr, int n) { return ((uintptr_t)ptr % n) == 0; }

}  // namespace

}  // namespace inl

extern "C" int inl_pool_last_fwd(int32_t n_texts, const int32_t* cu, int32_t hidden_dim, int64_t row_stride,
                                 int32_t dtype, const void* hidden, const void* weight, float eps,
                                 int32_t round_norm, float* pooled, void* stream) {
  using namespace inl;
  if (n_texts < 0 || hidden_dim <= 0 || !dtype_ok(dtype)) return fail(INL_E_INVALID, "pool_last: bad arguments");
  if (n_texts == 0) return INL_OK;
  const int64_t rs = row_stride ? row_stride : hidden_dim;
  if (!cu || !hidden || !pooled || rs < hidden_dim) return fail(INL_E_INVALID, "pool_last: NULL pointer or bad stride");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == INL_BF16)
    hipLaunchKernelGGL(pool_last_kernel<bf16>, dim3(n_texts), dim3(256), 0, st, (const char*)hidden, rs, cu,
                       hidden_dim, (const char*)weight, eps, round_norm, pooled);
  else
    hipLaunchKernelGGL(pool_last_kernel<float>, dim3(n_texts), dim3(256), 0, st, (const char*)hidden, rs, cu,
                       hidden_dim, (const char*)weight, eps, round_norm, pooled);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_pool_mean_fwd(int32_t n_texts, const int32_t* cu, int32_t hidden_dim, int64_t row_stride,
                                 int32_t dtype, const void* hidden, int32_t normalize, float* pooled,
                                 void* stream) {
  using namespace inl;
  if (n_texts < 0 || hidden_dim <= 0 || !dtype_ok(dtype)) return fail(INL_E_INVALID, "pool_mean: bad arguments");
  if (n_texts == 0) return INL_OK;
  const int64_t rs = row_stride ? row_stride : hidden_dim;
  if (!cu || !hidden || !pooled || rs < hidden_dim) return fail(INL_E_INVALID, "pool_mean: NULL pointer or bad stride");
  if (n_texts > 65535) return fail(INL_E_UNSUPPORTED, "pool_mean: more than 65535 texts in one call");
  hipStream_t st = (hipStream_t)stream;
  const int es = dtype_size(dtype);
  const bool vec = ((uintptr_t)hidden % 16 == 0) && (rs * es) % 16 == 0 && (hidden_dim * es) % 16 == 0;
  if (vec) {
    dim3 grid((hidden_dim + 16 * (16 / es) - 1) / (16 * (16 / es)), n_texts);
    if (dtype == INL_BF16)
      hipLaunchKernelGGL(pool_mean_vec_kernel<bf16>, grid, dim3(1024), 0, st, (const char*)hidden, rs, cu,
                         hidden_dim, pooled);
    else
      hipLaunchKernelGGL(pool_mean_vec_kernel<float>, grid, dim3(1024), 0, st, (const char*)hidden, rs, cu,
                         hidden_dim, pooled);
  } else {
    dim3 grid((hidden_dim + 63) / 64, n_texts);
    if (dtype == INL_BF16)
      hipLaunchKernelGGL(pool_mean_kernel<bf16>, grid, dim3(256), 0, st, (const char*)hidden, rs, cu, hidden_dim,
                         pooled);
    else
      hipLaunchKernelGGL(pool_mean_kernel<float>, grid, dim3(256), 0, st, (const char*)hidden, rs, cu, hidden_dim,
                         pooled);
  }
  INL_HIP_TRY(hipGetLastError());
  if (normalize) {
    hipLaunchKernelGGL(l2_kernel, dim3(n_texts), dim3(256), 0, st, pooled, (int64_t)hidden_dim, pooled,
                       (int64_t)hidden_dim, hidden_dim, 1e-12f, 0);
    INL_HIP_TRY(hipGetLastError());
  }
  return INL_OK;
}

extern "C" int inl_l2_normalize_fwd(int32_t rows, int32_t dim, int64_t in_stride, const float* x,
                                    int64_t out_stride, float* y, float eps_inside, int32_t skip_zero,
                                    void* stream) {
  using namespace inl;
  if (rows < 0 || dim <= 0 || in_stride < dim || out_stride < dim || !(eps_inside >= 0.f))
    return fail(INL_E_INVALID, "l2_normalize: bad arguments");
  if (rows == 0) return INL_OK;
  if (!x || !y) return fail(INL_E_INVALID, "l2_normalize: NULL pointer");
  hipLaunchKernelGGL(l2_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, in_stride, y, out_stride, dim,
                     eps_inside, skip_zero);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

namespace inl {
namespace {

int splade_launch(int32_t rows, const int32_t* offs, int32_t vocab, const float* logits, int64_t logits_stride,
                  const float* bias, float shift, const int32_t* masked_ids_host, int32_t n_masked,
                  const int32_t* canonical, int32_t out_dim, float* out, void* stream, bool direct);

}  // namespace
}  // namespace inl

extern "C" int inl_pool_splade_fwd(int32_t rows, const int32_t* offs, int32_t vocab, const float* logits,
                                   int64_t logits_stride, const float* bias, float shift,
                                   const int32_t* masked_ids_host, int32_t n_masked, const int32_t* canonical,
                                   int32_t out_dim, float* out, void* stream) {
  if (rows > 0 && !offs) return inl::fail(INL_E_INVALID, "pool_splade: NULL pointer or bad stride");
  return inl::splade_launch(rows, offs, vocab, logits, logits_stride, bias, shift, masked_ids_host, n_masked,
                            canonical, out_dim, out, stream, false);
}

extern "C" int inl_splade_finish_fwd(int32_t rows, int32_t vocab, const float* maxima, int64_t maxima_stride,
                                     const float* bias, float shift, const int32_t* masked_ids_host,
                                     int32_t n_masked, const int32_t* canonical, int32_t out_dim, float* out,
                                     void* stream) {
  return inl::splade_launch(rows, nullptr, vocab, maxima, maxima_stride, bias, shift, masked_ids_host, n_masked,
                            canonical, out_dim, out, stream, true);
}

namespace inl {
namespace {

int splade_launch(int32_t rows, const int32_t* offs, int32_t vocab, const float* logits, int64_t logits_stride,
                  const float* bias, float shift, const int32_t* masked_ids_host, int32_t n_masked,
                  const int32_t* canonical, int32_t out_dim, float* out, void* stream, bool direct) {
  if (rows < 0 || vocab <= 0 || n_masked < 0 || out_dim <= 0) return fail(INL_E_INVALID, "pool_splade: bad arguments");
  if (n_masked > kMaxMasked) return fail(INL_E_UNSUPPORTED, "pool_splade: more than 16 masked vocabulary ids");
  if (!canonical && out_dim != vocab) return fail(INL_E_INVALID, "pool_splade: out_dim must equal vocab without canonical ids");
  if (rows == 0) return INL_OK;
  const int64_t ls = logits_stride ? logits_stride : vocab;
  if (!logits || !out || ls < vocab || (n_masked && !masked_ids_host))
    return fail(INL_E_INVALID, "pool_splade: NULL pointer or bad stride");
  if (rows > 65535) return fail(INL_E_UNSUPPORTED, "pool_splade: more than 65535 rows in one call");
  SpladeParams p{};
  p.logits = logits;
  p.stride = ls;
  p.offs = offs;
  p.bias = bias;
  p.canonical = canonical;
  p.out = out;
  p.vocab = vocab;
  p.out_dim = out_dim;
  p.shift = shift;
  p.n_masked = n_masked;
  p.direct = direct;
  for (int k = 0; k < n_masked; ++k) {
    if (masked_ids_host[k] < 0 || masked_ids_host[k] >= vocab)
      return fail(INL_E_INVALID, "pool_splade: masked id outside the vocabulary");
    p.masked[k] = masked_ids_host[k];
  }
  hipStream_t st = (hipStream_t)stream;
  if (canonical) {
    const int64_t n = (int64_t)rows * out_dim;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n);
    INL_HIP_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(splade_kernel, dim3((vocab + 255) / 256, rows), dim3(256), 0, st, p);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

}  // namespace
}  // namespace inl
