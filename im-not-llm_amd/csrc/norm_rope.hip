// Fused per-head RMSNorm + RoPE prologue for packed encoder rows (gfx950).
//
// A token is handled by G = head_dim / 8 lanes, each owning 8 contiguous
// elements (one 16-byte bf16 chunk) of every head row of that token: the
// sum of squares is reduced over the G lanes with shuffles, and a rotation
// partner (element i + half of a half-split pair) lives in lane j +/- half/8
// and is exchanged with one shuffle per element. The weight and the token's
// cos/sin are loaded once per token, not once per head. HBM-bound: one read
// of x, one write of y.
//
// Replaces, per layer, the reference's q/k(/v) RMSNorm and RoPE kernels
// (crates/inl-text/src/qwen3/mod.rs:236-249, gemma2.rs:389-410,
// crates/inl-sparse/src/modernbert.rs:264-269, crates/inl-late/src/qwen3_5.rs:
// 289-300, crates/inl-vision/src/vision.rs:792-800).

#include <cmath>
#include <type_traits>
#include <vector>

#include "inl_common.hpp"
#include "lanes.hpp"

namespace inl {

namespace {

struct NormRopeParams {
  const char* x;
  char* y;
  const char* w;            // [head_dim] in x dtype, or null
  const char* w2;           // heads >= w2_heads use this weight instead (null: none)
  int32_t w2_heads;
  int32_t w3_heads;         // heads >= w3_heads are normalised without a weight
  int32_t rope_heads;       // heads >= rope_heads are not rotated
  const int32_t* rows;      // table row per token
  const float* cos;
  const float* sin;
  const float* cos2;
  const float* sin2;
  int64_t n_tokens;
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

// A lane's 8 input values kept as loaded (bf16: one 16-byte vector, f32:
// two) until the head step that uses them, so that the HB heads in flight
// cost half the registers in bf16.
struct Raw8 {
  u32x4 a, b;
};
template <typename TI>
__device__ __forceinline__ void load_raw(const char* p, Raw8& r) {
  r.a = *reinterpret_cast<const u32x4*>(p);
  if constexpr (sizeof(TI) != 2) r.b = *reinterpret_cast<const u32x4*>(p + 16);
}
template <typename TI>
__device__ __forceinline__ void unpack8(const Raw8& r, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = r.a[j];
    if constexpr (sizeof(TI) == 2) {
      v[2 * j] = __builtin_bit_cast(float, a << 16);
      v[2 * j + 1] = __builtin_bit_cast(float, a & 0xffff0000u);
    } else {
      const uint32_t b = r.b[j];
      v[j] = __builtin_bit_cast(float, a);
      v[4 + j] = __builtin_bit_cast(float, b);
    }
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

// out[e] = in[e] of lane (lane ^ m), for m a power of two below 64
// (uniform): one switch for the 8 values. Called with every lane of the
// wave active (a DPP read of a lane outside exec returns 0).
__device__ __forceinline__ void xor_lanes8(const float (&in)[8], float (&out)[8], int m, int lane) {
  switch (m) {
    case 1:
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = dpp<0xB1>(in[e]);      // quad_perm [1, 0, 3, 2]
      break;
    case 2:
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = dpp<0x4E>(in[e]);      // quad_perm [2, 3, 0, 1]
      break;
    case 4: {
      const bool hi = lane & 4;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float down = dpp<0x114>(in[e]);   // row_shr:4: lane i - 4
        const float up = dpp<0x104>(in[e]);     // row_shl:4: lane i + 4
        out[e] = hi ? down : up;
      }
      break;
    }
    case 8:
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = dpp<0x128>(in[e]);     // row_ror:8
      break;
    case 16: {
      const bool odd = lane & 16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = in[e], b = in[e];   // a: rows (0, 0, 2, 2), b: rows (1, 1, 3, 3)
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        out[e] = odd ? a : b;
      }
      break;
    }
    default: {
      const bool upper = lane & 32;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = in[e], b = in[e];   // a: halves (0, 0), b: halves (1, 1)
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        out[e] = upper ? a : b;
      }
    }
  }
}
// A group of G = head_dim / 8 lanes owns one token: each lane holds 8
// elements of a head row. The token's norm weights, table row and the lane's
// cos/sin columns are loaded once per group of HB (4, 5 or 8) heads of the token
// (each lane group owns one (token, head chunk)), so per (token, head) x is
// read and y written and the tables cost 1/HB of that in cache reads; the
// HB loads of a lane go out together. Heads [0, w2_heads) take weight w,
// [w2_heads, w3_heads) weight w2 and the rest none; heads from rope_heads on
// are normalised only (a fused q/k/v row: q and k rotated, v not). Every
// lane of a wave runs the head step the same number of times (the shuffles
// need all of them).
template <typename TI, typename TO, int G, int HB>
__global__ __launch_bounds__(256) void norm_rope_kernel(NormRopeParams p) {
  // G = head_dim / 8 lanes per row (a power of two <= 64)
  const int lane = threadIdx.x & 63;
  const int j = lane & (G - 1);                  // chunk of the row this lane owns
  // lane group -> (token, chunk of HB heads)
  const uint32_t chunks = ((uint32_t)p.heads + HB - 1) / HB;
  const uint32_t grp = blockIdx.x * (256u / (uint32_t)G) + threadIdx.x / (uint32_t)G;
  const uint32_t tok = grp / chunks;
  const int hfirst = (int)(grp - tok * chunks) * HB;
  const bool valid = tok < (uint32_t)p.n_tokens;
  const int heads = min(p.heads, hfirst + HB);

  // Every load below is issued unconditionally from a valid address and
  // masked afterwards: a load under a per-lane condition becomes a branch
  // that waits for it, which would put the x rows, the position and the
  // table row one after another instead of in flight together. x goes first.
  const uint32_t tokc = valid ? tok : 0u;   // launches have n_tokens >= 1
  const char* xt = p.x + ((int64_t)tokc * p.x_stride + 8 * j) * (int64_t)sizeof(TI);
  char* yt = p.y + ((int64_t)tok * p.y_stride + 8 * j) * (int64_t)sizeof(TO);
  const int64_t hstep_x = (int64_t)p.head_dim * (int64_t)sizeof(TI);
  const int64_t hstep_y = (int64_t)p.head_dim * (int64_t)sizeof(TO);
  Raw8 raw[HB];
#pragma unroll
  for (int i = 0; i < HB; ++i) load_raw<TI>(xt + min(hfirst + i, heads - 1) * hstep_x, raw[i]);

  // ---- per-token constants ----
  // the weights stay packed as loaded (ones when absent) until used
  Raw8 wr, w2r;
  {
    const uint32_t one = sizeof(TI) == 2 ? 0x3f803f80u : 0x3f800000u;
    wr.a = wr.b = w2r.a = w2r.b = (u32x4){one, one, one, one};
  }
  if (p.norm && p.w && hfirst < p.w2_heads) load_raw<TI>(p.w + 8 * j * (int)sizeof(TI), wr);
  if (p.norm && p.w2 && hfirst + HB > p.w2_heads && hfirst < p.w3_heads) load_raw<TI>(p.w2 + 8 * j * (int)sizeof(TI), w2r);

  // rope geometry: `mode` 0 = none for this lane, 1 = pairs (e, e + 4) inside
  // the lane (rotary_dim 8), 2 = half-split with the partner lane
  int mode = 0, partner = lane;
  bool first = true;
  float c[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { c[e] = 1.f; sn[e] = 0.f; }
  bool bad_pos = false;
  int sec_lanes = 0, sec0 = 0;
  // Partner distance of the half-split lanes. A power of two puts every
  // partner at lane ^ half_lanes (sections start at multiples of sec_lanes),
  // so the exchange runs on DPP / permlane instead of an LDS shuffle.
  int half_lanes = 0;
  bool xor_partner = false;
  if (p.rotary_dim == 8 && p.sections == 1) {
    mode = j == 0 ? 1 : 0;
  } else if (p.rotary_dim > 0) {
    if (p.sections == 2) {
      sec_lanes = G >> 1;
      sec0 = j < sec_lanes ? 0 : sec_lanes;
    } else {
      sec_lanes = p.rotary_dim >> 3;
      sec0 = 0;
    }
    half_lanes = sec_lanes >> 1;
    xor_partner = half_lanes > 0 && (half_lanes & (half_lanes - 1)) == 0;
    const int jj = j - sec0;                         // chunk inside the section
    if (jj >= 0 && jj < sec_lanes) {
      mode = 2;
      first = jj < half_lanes;
      partner = lane + (first ? half_lanes : -half_lanes);
    }
  }
  if (p.rotary_dim > 0) {   // uniform: the tables exist
    const int32_t pos = p.rows[tokc];
    bad_pos = mode != 0 && valid && (pos < 0 || pos >= p.table_rows);
    const int64_t posc = pos < 0 ? 0 : (pos >= p.table_rows ? p.table_rows - 1 : pos);
    float tc[8], ts[8];
    if (p.rotary_dim == 8 && p.sections == 1) {
      const f32x4 c4 = *reinterpret_cast<const f32x4*>(p.cos + posc * 4);
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(p.sin + posc * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) { tc[e] = c4[e]; ts[e] = s4[e]; tc[e + 4] = 1.f; ts[e + 4] = 0.f; }
    } else {
      const int half_lanes = sec_lanes >> 1;
      const int width = half_lanes * 8;              // table columns
      const bool second_sec = p.sections == 2 && !(j < (G >> 1));
      const float* ct = second_sec ? p.cos2 : p.cos;
      const float* st = second_sec ? p.sin2 : p.sin;
      const int jj = j - (second_sec ? (G >> 1) : 0);
      const int col = mode == 2 ? 8 * (first ? jj : jj - half_lanes) : 0;
      load8<float>(reinterpret_cast<const char*>(ct + posc * width + col), tc);
      load8<float>(reinterpret_cast<const char*>(st + posc * width + col), ts);
    }
    if (mode != 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) { c[e] = tc[e]; sn[e] = ts[e]; }
      if (p.round_tables)
#pragma unroll
        for (int e = 0; e < 8; ++e) { c[e] = round_bf16(c[e]); sn[e] = round_bf16(sn[e]); }
    }
  }

  {
    const int h0 = hfirst;   // this lane group's one step of HB heads
#pragma unroll
    for (int i = 0; i < HB; ++i) {
      float v[1][8];
      unpack8<TI>(raw[i], v[0]);
      if (!(valid && hfirst + i < heads))
#pragma unroll
        for (int e = 0; e < 8; ++e) v[0][e] = 0.f;
      if (p.norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[0][e] * v[0][e];
        ss = group_sum<G>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)p.head_dim + p.eps);
        const int h = h0 + i;
        const int wk = h < p.w2_heads ? 0 : (h < p.w3_heads ? 1 : 2);   // uniform in the lane group
        float wv[8];
        unpack8<TI>(wk == 0 ? wr : w2r, wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float we = wk == 2 ? 1.f : wv[e];
          v[0][e] = v[0][e] * inv * we;
          if (p.round_norm && sizeof(TO) == 2) v[0][e] = round_bf16(v[0][e]);
        }
      }
      const bool rot = h0 + i < p.rope_heads;
      if (mode == 1 && rot) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = v[0][e], b = v[0][e + 4];
          v[0][e] = a * c[e] - b * sn[e];
          v[0][e + 4] = b * c[e] + a * sn[e];
        }
      }
      if (p.rotary_dim > 0 && !(p.rotary_dim == 8 && p.sections == 1)) {
        float pv[8];
        if (xor_partner)
          xor_lanes8(v[0], pv, half_lanes, lane);
        else
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[e] = __shfl(v[0][e], partner, 64);
        if (mode == 2 && rot)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            v[0][e] = first ? (v[0][e] * c[e] - pv[e] * sn[e]) : (v[0][e] * c[e] + pv[e] * sn[e]);
      }
      if (bad_pos && rot)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[0][e] = __builtin_nanf("");
      if (valid && h0 + i < heads) store8<TO>(yt + (h0 + i) * hstep_y, v[0]);
    }
  }
}

}  // namespace

}  // namespace inl

namespace inl {

// inl_norm_rope_fwd with per-head ranges: heads [0, w2_heads) normalised
// with weight, [w2_heads, w3_heads) with weight2, the rest without a weight;
// heads from rope_heads on are not rotated.
int norm_rope_launch_ex(const inl_norm_rope_desc* d, const void* x, void* y, const void* weight,
                        const void* weight2, int32_t w2_heads, int32_t w3_heads, int32_t rope_heads,
                        const int32_t* rows, const float* cos, const float* sin, const float* cos2,
                        const float* sin2, void* stream) {
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
  if (!x || !y || ((uintptr_t)x & 15) || ((uintptr_t)y & 15) || (weight && ((uintptr_t)weight & 15)) ||
      (weight2 && ((uintptr_t)weight2 & 15)))
    return fail(INL_E_INVALID, "norm_rope: x, y and weight must be non-null and 16-byte aligned");
  if (w2_heads < 0 || w2_heads > w3_heads || w3_heads > d->heads || rope_heads < 0 || rope_heads > d->heads ||
      (weight2 && w2_heads == w3_heads))
    return fail(INL_E_INVALID, "norm_rope: head ranges must satisfy 0 <= w2_heads <= w3_heads <= heads");

  NormRopeParams p{};
  p.x = (const char*)x;
  p.y = (char*)y;
  p.w = d->norm ? (const char*)weight : nullptr;
  p.w2 = d->norm ? (const char*)weight2 : nullptr;
  p.w2_heads = w2_heads;
  p.w3_heads = w3_heads;
  p.rope_heads = rope_heads;
  p.rows = rows;
  p.cos = cos;
  p.sin = sin;
  p.cos2 = cos2;
  p.sin2 = sin2;
  p.n_tokens = d->n_tokens;
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
  // heads per lane group: 8 for 5-7 heads (a fused q/k/v row: one group per
  // token), else 4 (8 was slower on 8 and 16 heads of head_dim 128). The
  // fused row of EmbeddingGemma (3 q + 1 k + 1 v heads of 256) takes exactly
  // 5: no repeated loads of its last head, and 16 fewer registers.
  const int HB = d->heads == 5 && G == 32 ? 5 : (d->heads > 4 && d->heads < 8 ? 8 : 4);
  const int64_t groups_per_block = 256 / G;
  const int64_t groups = d->n_tokens * ((d->heads + HB - 1) / HB);   // (token, HB-head chunk)
  if (groups + groups_per_block >= ((int64_t)1 << 31))
    return fail(INL_E_UNSUPPORTED, "norm_rope: tokens x head chunks must stay below 2^31");
  const int64_t blocks = (groups + groups_per_block - 1) / groups_per_block;
  hipStream_t st = (hipStream_t)stream;
  auto launch = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    const dim3 grid((unsigned)blocks), block(256);
    auto go = [&](auto hb) {
      constexpr int H = decltype(hb)::value;
      switch (G) {
        case 1: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 1, H>), grid, block, 0, st, p); break;
        case 2: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 2, H>), grid, block, 0, st, p); break;
        case 4: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 4, H>), grid, block, 0, st, p); break;
        case 8: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 8, H>), grid, block, 0, st, p); break;
        case 16: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 16, H>), grid, block, 0, st, p); break;
        case 32: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 32, H>), grid, block, 0, st, p); break;
        default: hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 64, H>), grid, block, 0, st, p);
      }
    };
    if (HB == 5) hipLaunchKernelGGL((norm_rope_kernel<TI, TO, 32, 5>), grid, block, 0, st, p);
    else if (HB == 8) go(std::integral_constant<int, 8>{});
    else go(std::integral_constant<int, 4>{});
  };
  if (d->dtype == INL_BF16 && d->out_dtype == INL_BF16) launch(bf16{}, bf16{});
  else if (d->dtype == INL_BF16) launch(bf16{}, float{});
  else if (d->out_dtype == INL_BF16) launch(float{}, bf16{});
  else launch(float{}, float{});
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

int norm_rope_launch(const inl_norm_rope_desc* d, const void* x, void* y, const void* weight,
                     const void* weight2, int32_t w2_heads, const int32_t* rows, const float* cos,
                     const float* sin, const float* cos2, const float* sin2, void* stream) {
  if (!d) return fail(INL_E_INVALID, "norm_rope: desc is NULL");
  if (weight2 && (w2_heads <= 0 || w2_heads >= d->heads))
    return fail(INL_E_INVALID, "norm_rope: the second weight's first head must lie inside the heads");
  return norm_rope_launch_ex(d, x, y, weight, weight2, weight2 ? w2_heads : d->heads, d->heads, d->heads, rows, cos,
                             sin, cos2, sin2, stream);
}

}  // namespace inl

extern "C" int inl_norm_rope_fwd(const inl_norm_rope_desc* d, const void* x, void* y,
                                 const void* weight, const int32_t* rows, const float* cos,
                                 const float* sin, const float* cos2, const float* sin2,
                                 void* stream) {
  return inl::norm_rope_launch(d, x, y, weight, nullptr, 0, rows, cos, sin, cos2, sin2, stream);
}

extern "C" int inl_norm_rope_qk_fwd(const inl_norm_rope_desc* d, int32_t q_heads, const void* x, void* y,
                                    const void* q_weight, const void* k_weight, const int32_t* rows,
                                    const float* cos, const float* sin, const float* cos2, const float* sin2,
                                    void* stream) {
  using namespace inl;
  if (!d) return fail(INL_E_INVALID, "norm_rope_qk: desc is NULL");
  if (q_heads <= 0 || q_heads >= d->heads)
    return fail(INL_E_INVALID, "norm_rope_qk: need 0 < q_heads < heads");
  // heads >= q_heads take k_weight (ones when NULL: the kernel's default)
  return norm_rope_launch_ex(d, x, y, q_weight, k_weight, q_heads, d->heads, d->heads, rows, cos, sin, cos2, sin2,
                             stream);
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
