// Kernel-side definitions shared by the attention kernels.
#pragma once

#include "inl_common.hpp"

namespace inl {

struct AttnParams {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  int64_t q_stride, k_stride, v_stride, o_stride;  // elements between token rows
  const int4* items;  // {seg_start, seg_len, q0, (lo_tile << 16) | hi_tile}
  // Persistent kernels only: items[] holds work units (item, head group),
  // unit_hg[u] the head group of unit u, and workgroup b runs units
  // wg_start[b] .. wg_start[b + 1] - 1 in order.
  const int32_t* unit_hg;
  const int32_t* wg_start;
  int32_t n_hg;       // head groups per item (workgroups per item unless persistent)
  int32_t groups_per_kv;  // (h_q / h_kv) / hpw
  int32_t group;      // h_q / h_kv
  int32_t hpw;        // query heads per workgroup
  int32_t rb;         // waves per head per workgroup (NW / hpw), 32 rows each
  int32_t head_dim;
  int32_t causal;
  int32_t window;
  float scale_log2;   // scale * log2(e)
  int32_t out_bf16;
  // Generic kernel with a split key range (all null otherwise): an item i
  // with item_part[i] >= 0 covers part of its query block's key tiles and
  // writes partial slot item_part[i] (per head group and wave: 32 rows of
  // unnormalised O, row max and row sum) instead of the output;
  // attn_merge_kernel combines each block's slots into the output.
  const int32_t* item_part;
  float* part_o;      // [slot][32 rows][D] f32 (D: the kernel's compiled head dim)
  float2* part_ml;    // [slot][32 rows] {max (log2 domain, scaled), sum}
};

constexpr float kLog2e = 1.4426950408889634f;

// Max / sum of x over lanes l and l ^ 32, without an LDS round trip:
// v_permlane32_swap exchanges one half of the first register with the other
// half of the second, so with both holding x, lane l sees x[l] in one and
// x[l ^ 32] in the other (max and sum do not need to know which).
__device__ __forceinline__ void swap_halves(float x, float* a, float* b) {
  float u = x, v = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  *a = u;
  *b = v;
}
// Lanes 32-63 of a trade places with lanes 0-31 of b.
__device__ __forceinline__ void swap_lanes_32(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float half_max(float x) {
  float a, b;
  swap_halves(x, &a, &b);
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  swap_halves(x, &a, &b);
  return a + b;
}

// Byte offset of 16-byte chunk `c` of row `r` in a row-major tile whose rows
// are `row_bytes` long. The XOR keeps the 8 rows a group of lanes reads at
// one logical chunk in 8 distinct chunk columns (bank-conflict free).
__device__ __forceinline__ int swz(int r, int c, int row_bytes) {
  return r * row_bytes + ((c ^ (r & 7)) << 4);
}

// Launch of the bf16 fast path (attn_fwd_bf16.hip): returns the kernel entry
// and its dynamic LDS size for head dims 64/128/256.
typedef void (*AttnKernelFn)(AttnParams);
bool bf16_fast_kernel(int head_dim_padded, AttnKernelFn* fn, int* bn, int* nw, int* lds);

// Ping-pong bf16 kernel (attn_pp.hip): 8 waves in two groups that alternate
// MFMA and softmax phases; head dim 128. Persistent: one workgroup per CU,
// each running a host-assigned list of at most PP_MAX_UNITS work units.
constexpr int PP_MAX_UNITS = 1024;
bool bf16_pp_kernel(int head_dim, AttnKernelFn* fn, int* bn, int* nw, int* lds);

// Persistent bf16 kernel for head_dim 256 (attn_wide.hip): 4 waves, one per
// SIMD, each overlapping its softmax with its own MFMAs; same unit lists.
bool bf16_wide_kernel(int head_dim, AttnKernelFn* fn, int* bn, int* nw, int* lds);

// Persistent ping-pong kernel for head_dim 64 without grouped queries: each
// unit serves two query heads, one per wave group (attn_pp64.hip).
bool bf16_pp64_kernel(int head_dim, AttnKernelFn* fn, int* bn, int* nw, int* lds);

}  // namespace inl
