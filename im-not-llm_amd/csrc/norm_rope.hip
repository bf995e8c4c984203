// Fused per-head RMSNorm + RoPE prologue for packed encoder rows (gfx950).
//
// One (token, head) row of head_dim elements is handled by G = head_dim / 8
// lanes, each owning 8 contiguous elements (one 16-byte bf16 chunk): the
// sum of squares is reduced over the G lanes with shuffles, and a rotation
// partner (element i + half of a half-split pair) lives in lane j +/- half/8
// and is exchanged with one shuffle per element. HBM-bound: one read of x,
// one write of y; weights and cos/sin tables are shared by every row and
// stay in cache.
//
// Replaces, per layer, the reference's q/k(/v) RMSNorm and RoPE kernels
// (crates/inl-text/src/qwen3/mod.rs:236-249, gemma2.rs:389-410,
// crates/inl-sparse/src/modernbert.rs:264-269, crates/inl-late/src/qwen3_5.rs:
// 289-300, crates/inl-vision/src/vision.rs:792-800).

#include <cmath>
#include <vector>

#include "inl_common.hpp"

namespace inl {

namespace {

struct NormRopeParams {
  const char* x;
  char* y;
  const char* w;            // [head_dim] in x dtype, or null
  const int32_t* rows;      // table row per token
  const float* cos;
  const float* sin;
  const float* cos2;
  const float* sin2;
  int64_t n_rows;           // tokens * heads
  int32_t heads;
  int32_t head_dim;
  int64_t x_stride, y_stride;  // elements between token rows
  int32_t norm;
  float eps;
  int32_t rotary_dim;
  int32_t sections;
  int32_t table_rows;
  int32_t round_tables;
  int32_t round_norm;
};

__device__ __forceinline__ float round_bf16(float v) { return (float)(bf16)v; }

template <typename TI>
__device__ __forceinline__ void load8(const char* p, float (&v)[8]) {
  if constexpr (sizeof(TI) == 2) {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __builtin_bit_cast(float, w[j] << 16);
      v[2 * j + 1] = __builtin_bit_cast(float, w[j] & 0xffff0000u);
    }
  } else {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
  }
}

template <typename TO>
__device__ __forceinline__ void store8(char* p, const float (&v)[8]) {
  if constexpr (sizeof(TO) == 2) {
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (bf16)v[j];
    *reinterpret_cast<bf16x8*>(p) = o;
  } else {
    f32x4 a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 16) = b;
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void norm_rope_kernel(NormRopeParams p) {
  const int G = p.head_dim >> 3;                 // lanes per row (power of two <= 64)
  const int lane = threadIdx.x & 63;
  const int j = lane & (G - 1);                  // chunk of the row this lane owns
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / G;
  const bool valid = row < p.n_rows;             // whole groups are valid or not
  const int64_t tok = valid ? row / p.heads : 0;
  const int head = valid ? (int)(row - tok * p.heads) : 0;

  float v[8];
  if (valid) load8<TI>(p.x + (tok * p.x_stride + (int64_t)head * p.head_dim + 8 * j) * (int64_t)sizeof(TI), v);
  else
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;

  if (p.norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    for (int m = G >> 1; m > 0; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float inv = 1.0f / sqrtf(ss / (float)p.head_dim + p.eps);
    float w[8];
    if (p.w) load8<TI>(p.w + 8 * j * (int)sizeof(TI), w);
    else
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = 1.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = v[e] * inv * w[e];
      if (p.round_norm && sizeof(TO) == 2) v[e] = round_bf16(v[e]);
    }
  }

  if (p.rotary_dim == 8 && p.sections == 1) {
    // Both halves of the rotated section sit in chunk 0: pairs (e, e + 4)
    // rotate inside the lane, by table column e (4 columns).
    if (j == 0 && valid) {
      const int32_t pos = p.rows[tok];
      if (pos < 0 || pos >= p.table_rows) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __builtin_nanf("");
      } else {
        const f32x4 c = *reinterpret_cast<const f32x4*>(p.cos + (int64_t)pos * 4);
        const f32x4 s = *reinterpret_cast<const f32x4*>(p.sin + (int64_t)pos * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float ce = c[e], se = s[e];
          if (p.round_tables) { ce = round_bf16(ce); se = round_bf16(se); }
          const float a = v[e], b = v[e + 4];
          v[e] = a * ce - b * se;
          v[e + 4] = b * ce + a * se;
        }
      }
    }
  } else if (p.rotary_dim > 0) {
    // Geometry of the half-split this lane belongs to.
    int sec_lanes, sec0;  // lanes per rotated section, first lane of it
    if (p.sections == 2) {
      sec_lanes = G >> 1;
      sec0 = j < sec_lanes ? 0 : sec_lanes;
    } else {
      sec_lanes = p.rotary_dim >> 3;
      sec0 = 0;
    }
    const int half_lanes = sec_lanes >> 1;
    const int jj = j - sec0;                         // chunk inside the section
    const bool rotated = jj >= 0 && jj < sec_lanes;  // pass-through chunks are not
    const bool first = jj < half_lanes;
    const int partner = lane + (first ? half_lanes : -half_lanes);
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = __shfl(v[e], rotated ? partner : lane, 64);
    if (rotated && valid) {
      const int32_t pos = p.rows[tok];
      const int width = half_lanes * 8;              // table columns
      const float* ct = (p.sections == 2 && !(j < (G >> 1))) ? p.cos2 : p.cos;
      const float* st = (p.sections == 2 && !(j < (G >> 1))) ? p.sin2 : p.sin;
      if (pos < 0 || pos >= p.table_rows) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __builtin_nanf("");
      } else {
        const int col = 8 * (first ? jj : jj - half_lanes);
        float c[8], s[8];
        load8<float>(reinterpret_cast<const char*>(ct + (int64_t)pos * width + col), c);
        load8<float>(reinterpret_cast<const char*>(st + (int64_t)pos * width + col), s);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float ce = c[e], se = s[e];
          if (p.round_tables) { ce = round_bf16(ce); se = round_bf16(se); }
          v[e] = first ? (v[e] * ce - pv[e] * se) : (v[e] * ce + pv[e] * se);
        }
      }
    }
  }

  if (valid) store8<TO>(p.y + (tok * p.y_stride + (int64_t)head * p.head_dim + 8 * j) * (int64_t)sizeof(TO), v);
}

}  // namespace

}  // namespace inl

extern "C" int inl_norm_rope_fwd(const inl_norm_rope_desc* d, const void* x, void* y,
                                 const void* weight, const int32_t* rows, const float* cos,
                                 const float* sin, const float* cos2, const float* sin2,
                                 void* stream) {
  using namespace inl;
  if (!d) return fail(INL_E_INVALID, "norm_rope: desc is NULL");
  if (!dtype_ok(d->dtype) || !dtype_ok(d->out_dtype))
    return fail(INL_E_INVALID, "norm_rope: dtype must be INL_F32 or INL_BF16");
  if (d->n_tokens < 0 || d->heads <= 0) return fail(INL_E_INVALID, "norm_rope: bad n_tokens/heads");
  const int hd = d->head_dim;
  if (hd < 8 || hd > 512 || (hd & 7) || ((hd >> 3) & ((hd >> 3) - 1)))
    return fail(INL_E_UNSUPPORTED, "norm_rope: head_dim must be 8 x a power of two, <= 512");
  if (d->norm != 0 && d->norm != 1) return fail(INL_E_INVALID, "norm_rope: norm must be 0 or 1");
  if (d->norm && !(d->eps >= 0.f)) return fail(INL_E_INVALID, "norm_rope: eps must be >= 0");
  if (d->rotary_dim < 0) return fail(INL_E_INVALID, "norm_rope: rotary_dim < 0");
  if (d->rotary_dim > 0) {
    if (d->sections == 1) {
      if (d->rotary_dim > hd || (d->rotary_dim % 16 && d->rotary_dim != 8))
        return fail(INL_E_UNSUPPORTED, "norm_rope: rotary_dim must be 8 or a multiple of 16, <= head_dim");
    } else if (d->sections == 2) {
      if (d->rotary_dim != hd || hd % 32)
        return fail(INL_E_UNSUPPORTED, "norm_rope: axial rope needs rotary_dim == head_dim, a multiple of 32");
      if (!cos2 || !sin2) return fail(INL_E_INVALID, "norm_rope: axial rope needs cos2/sin2");
    } else {
      return fail(INL_E_INVALID, "norm_rope: sections must be 1 or 2");
    }
    if (!rows || !cos || !sin || d->table_rows <= 0)
      return fail(INL_E_INVALID, "norm_rope: rope needs rows, cos, sin and table_rows > 0");
  }
  const int64_t xs = d->x_row_stride ? d->x_row_stride : (int64_t)d->heads * hd;
  const int64_t ys = d->y_row_stride ? d->y_row_stride : (int64_t)d->heads * hd;
  if (xs < (int64_t)d->heads * hd || ys < (int64_t)d->heads * hd || (xs * dtype_size(d->dtype)) % 16 ||
      (ys * dtype_size(d->out_dtype)) % 16)
    return fail(INL_E_INVALID, "norm_rope: row strides must cover all heads, in 16-byte multiples");
  if (d->n_tokens == 0) return INL_OK;
  if (!x || !y || ((uintptr_t)x & 15) || ((uintptr_t)y & 15) || (weight && ((uintptr_t)weight & 15)))
    return fail(INL_E_INVALID, "norm_rope: x, y and weight must be non-null and 16-byte aligned");

  NormRopeParams p{};
  p.x = (const char*)x;
  p.y = (char*)y;
  p.w = d->norm ? (const char*)weight : nullptr;
  p.rows = rows;
  p.cos = cos;
  p.sin = sin;
  p.cos2 = cos2;
  p.sin2 = sin2;
  p.n_rows = d->n_tokens * d->heads;
  p.heads = d->heads;
  p.head_dim = hd;
  p.x_stride = xs;
  p.y_stride = ys;
  p.norm = d->norm;
  p.eps = d->eps;
  p.rotary_dim = d->rotary_dim;
  p.sections = d->sections;
  p.table_rows = d->table_rows;
  p.round_tables = d->round_tables;
  p.round_norm = d->round_norm;

  const int G = hd >> 3;
  const int64_t threads = p.n_rows * G;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return fail(INL_E_UNSUPPORTED, "norm_rope: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (d->dtype == INL_BF16 && d->out_dtype == INL_BF16)
    hipLaunchKernelGGL((norm_rope_kernel<bf16, bf16>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  else if (d->dtype == INL_BF16)
    hipLaunchKernelGGL((norm_rope_kernel<bf16, float>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  else if (d->out_dtype == INL_BF16)
    hipLaunchKernelGGL((norm_rope_kernel<float, bf16>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((norm_rope_kernel<float, float>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_rope_table_host(int32_t rotary_dim, double theta, int32_t positions,
                                   int32_t mode, float* cos_out, float* sin_out) {
  using namespace inl;
  if (rotary_dim <= 0 || rotary_dim % 2 || positions < 0 || !(theta > 0.0) || !cos_out || !sin_out)
    return fail(INL_E_INVALID, "rope_table: bad arguments");
  const int half = rotary_dim / 2;
  if (mode == 0) {
    // f64 inverse frequencies and angles, stored as f32
    // (crates/inl-text/src/qwen3/mod.rs:131-153).
    std::vector<double> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0 / std::pow(theta, (double)(2 * i) / (double)rotary_dim);
    for (int64_t pos = 0; pos < positions; ++pos)
      for (int i = 0; i < half; ++i) {
        const double a = (double)pos * inv[i];
        cos_out[pos * half + i] = (float)std::cos(a);
        sin_out[pos * half + i] = (float)std::sin(a);
      }
  } else if (mode == 1) {
    // f32 inverse frequencies and angle products (crates/inl-late/src/qwen3_5.rs:940-957).
    std::vector<float> inv(half);
    const float th = (float)theta;
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / std::pow(th, (float)(2 * i) / (float)rotary_dim);
    for (int64_t pos = 0; pos < positions; ++pos)
      for (int i = 0; i < half; ++i) {
        const float a = (float)pos * inv[i];
        cos_out[pos * half + i] = std::cos(a);
        sin_out[pos * half + i] = std::sin(a);
      }
  } else {
    return fail(INL_E_INVALID, "rope_table: mode must be 0 (f64) or 1 (f32)");
  }
  return INL_OK;
}

extern "C" int inl_positions_host(int32_t n_texts, const int32_t* cu, int32_t* positions) {
  using namespace inl;
  int64_t total = 0;
  if (n_texts < 0 || (n_texts > 0 && (!cu || !positions))) return fail(INL_E_INVALID, "positions: bad arguments");
  int rc = check_cu(n_texts, cu, &total);
  if (rc) return rc;
  for (int32_t b = 0; b < n_texts; ++b)
    for (int32_t i = cu[b]; i < cu[b + 1]; ++i) positions[i] = i - cu[b];
  return INL_OK;
}
