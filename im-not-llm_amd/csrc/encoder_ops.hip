// The element-wise ops of an encoder layer around its GEMMs (gfx950,
// HBM-bound): the token-embedding gather into the f32 residual stream, the
// pre-norm RMSNorm of that stream into the next GEMM's input dtype, and the
// SwiGLU gate of the MLP. Reference: crates/inl-text/src/qwen3/mod.rs
// (Embedding :322-323,350; RmsNorm :72-90 applied at :287-295 and :357;
// Mlp :109-116).
//
// All three move whole rows with 16-byte vector accesses when the rows and
// pointers allow it (one lane per 8 bf16 or 4 f32 values).

#include <cmath>
#include <type_traits>

#include "inl_common.hpp"
#include "lanes.hpp"

namespace inl {

namespace {

template <typename T>
__device__ __forceinline__ float ldf(const char* p) {
  if constexpr (sizeof(T) == 2) return (float)*reinterpret_cast<const bf16*>(p);
  else return *reinterpret_cast<const float*>(p);
}

template <typename T>
__device__ __forceinline__ void stf(char* p, float v) {
  if constexpr (sizeof(T) == 2) *reinterpret_cast<bf16*>(p) = (bf16)v;
  else *reinterpret_cast<float*>(p) = v;
}

// ---- embedding gather: out[t, :] = f32(table[ids[t], :]); an id outside
// [0, vocab) gives a NaN row (the host checks ids before it calls) ----
template <typename T>
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* ids, const char* table, int64_t vocab,
                                                    int32_t hidden, float* out, int64_t out_stride) {
  const int64_t t = blockIdx.x;
  const int32_t id = ids[t];
  const bool ok = id >= 0 && id < vocab;
  const char* row = table + (int64_t)(ok ? id : 0) * hidden * (int64_t)sizeof(T);
  float* o = out + t * out_stride;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x)
    o[i] = ok ? ldf<T>(row + i * (int)sizeof(T)) : __builtin_nanf("");
}

// 4 consecutive values at byte address p of a T array, as f32. VEC: one
// vector access (p aligned to 4 * sizeof(T)); otherwise four scalar ones.
template <typename T, bool VEC>
__device__ __forceinline__ f32x4 ld4(const char* p) {
  if constexpr (VEC && sizeof(T) == 2) {
    const u32x2 b = *reinterpret_cast<const u32x2*>(p);
    return (f32x4){__builtin_bit_cast(float, b[0] << 16), __builtin_bit_cast(float, b[0] & 0xffff0000u),
                   __builtin_bit_cast(float, b[1] << 16), __builtin_bit_cast(float, b[1] & 0xffff0000u)};
  } else if constexpr (VEC) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    return (f32x4){ldf<T>(p), ldf<T>(p + sizeof(T)), ldf<T>(p + 2 * sizeof(T)), ldf<T>(p + 3 * sizeof(T))};
  }
}
template <typename T, bool VEC>
__device__ __forceinline__ void st4(char* p, const f32x4& v) {
  if constexpr (VEC && sizeof(T) == 2) {
    const bf16x2 lo = __builtin_convertvector((f32x2){v[0], v[1]}, bf16x2);
    const bf16x2 hi = __builtin_convertvector((f32x2){v[2], v[3]}, bf16x2);
    *reinterpret_cast<u32x2*>(p) = (u32x2){__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  } else if constexpr (VEC) {
    *reinterpret_cast<f32x4*>(p) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) stf<T>(p + e * sizeof(T), v[e]);
  }
}

// ---- RMSNorm of f32 rows into TO: one wave per row ----
// y = x / sqrt(mean(x^2) + eps) * w (w in TW, the model dtype). Each lane
// holds 4-value chunks of the row; the sum of squares is a wave_sum. With
// K > 0 the row (at most K * 256 values) and its weights stay in registers
// between the two passes: every load is issued first, at a clamped address
// (masked after, so no load waits behind a branch). K = 0 reads a longer row
// twice. VEC: the weights and the output are read and written 4 values at a
// time (the host checks their alignment).
template <typename TW, typename TO, int K, bool VEC>
__global__ __launch_bounds__(256) void rms_rows_kernel(const float* x, int64_t xs, int64_t rows, int32_t dim,
                                                       const char* w, float eps, char* y, int64_t ys) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* xr = x + r * xs;
  char* yr = y + r * ys * (int64_t)sizeof(TO);
  const f32x4 one = {1.f, 1.f, 1.f, 1.f};
  float ss = 0.f;
  if constexpr (K > 0) {
    f32x4 held[K], wv[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int i = lane * 4 + 256 * k;
      const int ic = i < dim ? i : dim - 4;
      held[k] = *reinterpret_cast<const f32x4*>(xr + ic);
      wv[k] = w ? ld4<TW, VEC>(w + ic * (int)sizeof(TW)) : one;
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (lane * 4 + 256 * k >= dim) held[k] = (f32x4){0.f, 0.f, 0.f, 0.f};
      ss += (held[k][0] * held[k][0] + held[k][1] * held[k][1]) + (held[k][2] * held[k][2] + held[k][3] * held[k][3]);
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int i = lane * 4 + 256 * k;
      if (i < dim) st4<TO, VEC>(yr + i * (int)sizeof(TO), held[k] * inv * wv[k]);
    }
  } else {
    for (int i = lane * 4; i < dim; i += 256) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
      ss += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)dim + eps);
    for (int i = lane * 4; i < dim; i += 256) {
      const f32x4 wq = w ? ld4<TW, VEC>(w + i * (int)sizeof(TW)) : one;
      st4<TO, VEC>(yr + i * (int)sizeof(TO), *reinterpret_cast<const f32x4*>(xr + i) * inv * wq);
    }
  }
}

// ---- SwiGLU: out[t, i] = silu(gu[t, i]) * gu[t, inter + i] ----
// silu(g) = g / (1 + exp(-g)) in f32, as candle's Activation::Silu.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const char* gu, int64_t gs, int64_t rows, int32_t inter,
                                                     char* out, int64_t os) {
  constexpr int VW = 16 / sizeof(T);
  const int64_t vecs = (int64_t)inter / VW;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * vecs) return;
  const int64_t r = i / vecs;
  const int64_t c = (i - r * vecs) * VW;
  const char* g = gu + (r * gs + c) * (int64_t)sizeof(T);
  const char* u = gu + (r * gs + inter + c) * (int64_t)sizeof(T);
  const u32x4 gv = *reinterpret_cast<const u32x4*>(g);
  const u32x4 uv = *reinterpret_cast<const u32x4*>(u);
  float gf[VW], uf[VW];
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gf[2 * q] = __builtin_bit_cast(float, gv[q] << 16);
      gf[2 * q + 1] = __builtin_bit_cast(float, gv[q] & 0xffff0000u);
      uf[2 * q] = __builtin_bit_cast(float, uv[q] << 16);
      uf[2 * q + 1] = __builtin_bit_cast(float, uv[q] & 0xffff0000u);
    }
  } else {
    const f32x4 g4 = __builtin_bit_cast(f32x4, gv), u4 = __builtin_bit_cast(f32x4, uv);
#pragma unroll
    for (int q = 0; q < 4; ++q) { gf[q] = g4[q]; uf[q] = u4[q]; }
  }
  char* o = out + (r * os + c) * (int64_t)sizeof(T);
  if constexpr (sizeof(T) == 2) {
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = (bf16)(gf[e] / (1.0f + expf(-gf[e])) * uf[e]);
    *reinterpret_cast<bf16x8*>(o) = ov;
  } else {
    f32x4 ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = gf[e] / (1.0f + expf(-gf[e])) * uf[e];
    *reinterpret_cast<f32x4*>(o) = ov;
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

}  // namespace inl

extern "C" int inl_embed_fwd(int64_t n_tokens, const int32_t* ids, const void* table, int64_t vocab,
                             int32_t hidden, int32_t dtype, float* out, int64_t out_stride, void* stream) {
  using namespace inl;
  if (n_tokens < 0 || vocab <= 0 || hidden <= 0 || !dtype_ok(dtype))
    return fail(INL_E_INVALID, "embed: bad arguments");
  const int64_t os = out_stride ? out_stride : hidden;
  if (os < hidden) return fail(INL_E_INVALID, "embed: out_stride < hidden");
  if (n_tokens == 0) return INL_OK;
  if (!ids || !table || !out) return fail(INL_E_INVALID, "embed: NULL pointer");
  if (n_tokens > 0x7fffffff) return fail(INL_E_UNSUPPORTED, "embed: more than 2^31 tokens");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == INL_BF16)
    hipLaunchKernelGGL(embed_kernel<bf16>, dim3((unsigned)n_tokens), dim3(256), 0, st, ids, (const char*)table,
                       vocab, hidden, out, os);
  else
    hipLaunchKernelGGL(embed_kernel<float>, dim3((unsigned)n_tokens), dim3(256), 0, st, ids, (const char*)table,
                       vocab, hidden, out, os);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_rms_norm_rows_fwd(int64_t rows, int32_t dim, const float* x, int64_t x_stride,
                                     const void* weight, int32_t weight_dtype, float eps, int32_t out_dtype,
                                     void* y, int64_t y_stride, void* stream) {
  using namespace inl;
  if (rows < 0 || dim <= 0 || !dtype_ok(weight_dtype) || !dtype_ok(out_dtype) || !(eps >= 0.f))
    return fail(INL_E_INVALID, "rms_norm_rows: bad arguments");
  const int64_t xs = x_stride ? x_stride : dim, ys = y_stride ? y_stride : dim;
  if (dim % 4 || xs % 4 || xs < dim || ys < dim)
    return fail(INL_E_INVALID, "rms_norm_rows: dim and x_stride must be multiples of 4; strides >= dim");
  if (rows == 0) return INL_OK;
  if (!x || !y || !al16(x)) return fail(INL_E_INVALID, "rms_norm_rows: NULL x/y or x not 16-byte aligned");
  if ((rows + 3) / 4 > 0x7fffffff) return fail(INL_E_UNSUPPORTED, "rms_norm_rows: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + 3) / 4));
  const char* w = (const char*)weight;
  // chunks of 256 values a lane holds: the smallest of 1, 2, 4, 8 that covers
  // the row, 0 (two passes) beyond 2048
  const int K = dim <= 256 ? 1 : dim <= 512 ? 2 : dim <= 1024 ? 4 : dim <= 2048 ? 8 : 0;
  // Vector weight and output accesses when every 4-value group is aligned
  // to 4 elements: the pointers and the output row stride.
  const int wsz = dtype_size(weight_dtype), osz = dtype_size(out_dtype);
  const bool vec = ((uintptr_t)w % (4 * wsz)) == 0 && ((uintptr_t)y % (4 * osz)) == 0 && ys % 4 == 0;
  auto launch = [&](auto tw, auto to, auto vtag) {
    using TW = decltype(tw);
    using TO = decltype(to);
    constexpr bool V = decltype(vtag)::value;
    switch (K) {
      case 1: hipLaunchKernelGGL((rms_rows_kernel<TW, TO, 1, V>), grid, dim3(256), 0, st, x, xs, rows, dim, w, eps, (char*)y, ys); break;
      case 2: hipLaunchKernelGGL((rms_rows_kernel<TW, TO, 2, V>), grid, dim3(256), 0, st, x, xs, rows, dim, w, eps, (char*)y, ys); break;
      case 4: hipLaunchKernelGGL((rms_rows_kernel<TW, TO, 4, V>), grid, dim3(256), 0, st, x, xs, rows, dim, w, eps, (char*)y, ys); break;
      case 8: hipLaunchKernelGGL((rms_rows_kernel<TW, TO, 8, V>), grid, dim3(256), 0, st, x, xs, rows, dim, w, eps, (char*)y, ys); break;
      default: hipLaunchKernelGGL((rms_rows_kernel<TW, TO, 0, V>), grid, dim3(256), 0, st, x, xs, rows, dim, w, eps, (char*)y, ys);
    }
  };
  auto launch_v = [&](auto tw, auto to) {
    if (vec) launch(tw, to, std::true_type{});
    else launch(tw, to, std::false_type{});
  };
  if (weight_dtype == INL_BF16 && out_dtype == INL_BF16) launch_v(bf16{}, bf16{});
  else if (weight_dtype == INL_BF16) launch_v(bf16{}, float{});
  else if (out_dtype == INL_BF16) launch_v(float{}, bf16{});
  else launch_v(float{}, float{});
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_swiglu_fwd(int64_t rows, int32_t intermediate, int32_t dtype, const void* gate_up,
                              int64_t gu_stride, void* out, int64_t out_stride, void* stream) {
  using namespace inl;
  if (rows < 0 || intermediate <= 0 || !dtype_ok(dtype)) return fail(INL_E_INVALID, "swiglu: bad arguments");
  const int es = dtype_size(dtype), vw = 16 / es;
  const int64_t gs = gu_stride ? gu_stride : 2 * (int64_t)intermediate;
  const int64_t os = out_stride ? out_stride : intermediate;
  if (intermediate % vw || gs % vw || os % vw || gs < 2 * (int64_t)intermediate || os < intermediate)
    return fail(INL_E_INVALID, "swiglu: sizes and strides must be 16-byte multiples, strides covering the rows");
  if (rows == 0) return INL_OK;
  if (!gate_up || !out || !al16(gate_up) || !al16(out))
    return fail(INL_E_INVALID, "swiglu: NULL or unaligned pointer");
  const int64_t n = rows * (intermediate / vw);
  if ((n + 255) / 256 > 0x7fffffff) return fail(INL_E_UNSUPPORTED, "swiglu: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == INL_BF16)
    hipLaunchKernelGGL(swiglu_kernel<bf16>, grid, dim3(256), 0, st, (const char*)gate_up, gs, rows, intermediate,
                       (char*)out, os);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, grid, dim3(256), 0, st, (const char*)gate_up, gs, rows, intermediate,
                       (char*)out, os);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}
