// Packed variable-length encoder attention for MI355X (gfx950).
//
// One kernel template serves every attention form of the encoder engines
// (causal GQA, bidirectional full, sliding window): a query i of a text sees
// key j of the same text iff (!causal || j <= i) && (window < 0 ||
// |i - j| <= window). It replaces the reference's padded attention calls
// (crates/inl-core/src/attention.rs:215-315, crates/inl-text/src/gemma2.rs:
// 414-441, crates/inl-sparse/src/modernbert.rs:366-401,
// crates/inl-late/src/qwen3_5.rs:364-407, crates/inl-vision/src/vision.rs:
// 226-259) with one launch per layer over packed texts.
//
// Work decomposition. The host builds a tile schedule: one item per
// (text, block of BLOCK_M query rows) holding the range of BLOCK_N-key tiles
// the rows can see (tiles above the causal diagonal, outside the window or in
// other texts are never visited), sorted by cost, longest first. A workgroup
// takes one item for `hpw` query heads that share one KV head, so every K/V
// tile staged in LDS serves hpw * BLOCK_M query rows. Each 64-lane wave owns
// 32 query rows of one head.
//
// Per wave and key tile (32x32 MFMA tiles, fp32 accumulation):
//   S^T[key, query] = K . Q^T      A = K rows from LDS, B = Q^T in registers
//   online softmax on S^T columns  (each lane owns one query; the max needs a
//                                   single cross-half exchange, the row sum is
//                                   combined once at the end)
//   O^T[d, query] += V^T . P^T     A = V^T from LDS, B = P^T from registers
// Computing the transposed products keeps every query's scores and output in
// its own lane, so softmax rescaling is lane-local. V is transposed while it
// is staged into LDS (register transposes of 4-key groups), and its key
// columns are stored in the order the S^T accumulator hands P to the PV
// product, so P never moves between lanes.
//
// bf16 inputs: QK^T on v_mfma_f32_32x32x16_bf16. For PV, V is converted to
// fp16 while it is staged (exact for every bf16 value of magnitude below
// 65504) and P is rounded to fp16, so PV runs on v_mfma_f32_32x32x16_f16 with
// 8x the P precision of bf16: a causal row that sees two keys of comparable
// weight would otherwise carry up to ~4e-3 of P rounding error. The flag
// INL_ATTN_PV_BF16 keeps V and P in bf16 instead (any V range, coarser P).
// f32 inputs use v_mfma_f32_32x32x2_f32 throughout.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <mutex>
#include <new>
#include <queue>
#include <set>
#include <unordered_map>
#include <vector>

#include "attn_kernels.hpp"

namespace inl {

namespace {

// Element type of V^T in LDS and of P for the PV product.
template <typename E, bool PV16>
struct PvType { typedef float T; };
template <> struct PvType<bf16, true> { typedef f16 T; };
template <> struct PvType<bf16, false> { typedef bf16 T; };

// Column of a 4-key group inside a V^T row. bf16: within 16 keys, swap key
// bits 2 and 3, so lane-half h of the PV product reads its 8 keys
// {8a + 4h + b} (a, b the S^T accumulator's row split) as one 16-byte chunk.
// f32: within 32 keys, key 8a + 4h + b goes to 16h + 4a + b.
template <typename E>
__device__ __forceinline__ int vcol(int key4) {
  if constexpr (sizeof(E) == 2) {
    return (key4 & ~15) | ((key4 & 4) << 1) | ((key4 & 8) >> 1);
  } else {
    return (key4 & ~31) | ((key4 & 4) << 2) | ((key4 & 24) >> 1);
  }
}

template <typename E, int D, int BN, int NW, bool PV16>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(AttnParams p) {
  typedef typename PvType<E, PV16>::T PT;
  constexpr int NT = NW * 64;
  constexpr int ES = (int)sizeof(E);
  constexpr int VEC = 16 / ES;          // elements per 16-byte chunk
  constexpr int CHK = D / VEC;          // chunks per K row
  constexpr int KROW = D * ES;          // bytes per K row in LDS
  constexpr int VROW = BN * ES;         // bytes per V^T row in LDS
  constexpr int KT_BYTES = BN * D * ES; // one K (or V^T) tile
  constexpr int NKC = BN * CHK;         // K chunks per tile
  constexpr int NVU = (BN / 4) * CHK;   // V units (4 keys x 1 chunk) per tile
  constexpr int KPT = (NKC + NT - 1) / NT;
  constexpr int VPT = (NVU + NT - 1) / NT;
  constexpr int NKB = BN / 32;          // 32-key blocks per tile
  constexpr int NDB = D / 32;           // 32-wide d blocks of the output
  static_assert(CHK >= 8 && (VROW / 16) >= 8, "swizzle needs 8 chunks per row");
  static_assert(BN % 32 == 0 && D % 32 == 0, "tile shape");

  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lq = lane & 31;   // query column this lane owns
  const int hf = lane >> 5;   // lane half

  const int item_idx = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item_idx * p.n_hg;
  const int4 it = p.items[item_idx];
  const int seg = it.x;
  const int T = it.y;
  const int q0 = it.z;
  const int lo_t = (int)((uint32_t)it.w >> 16);
  const int hi_t = it.w & 0xffff;
  const int kvh = hg / p.groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * p.groups_per_kv) * p.hpw + wave / p.rb;
  const int r0 = q0 + (wave % p.rb) * 32;  // first query row of this wave
  const int hd = p.head_dim;
  const bool active = r0 < T;

  // Key range this wave can see (text-local, [klo, khi)).
  const int rlast = min(r0 + 31, T - 1);
  int klo = 0, khi = p.causal ? min(T, r0 + 32) : T;
  if (p.window >= 0) {
    klo = max(0, r0 - p.window);
    khi = min(khi, rlast + p.window + 1);
  }

  // ---- Q^T operand, resident in registers for the whole item ----
  const int qrow = r0 + lq;
  const bool qvalid = qrow < T;
  const char* qptr = p.q + ((int64_t)(seg + (qvalid ? qrow : 0)) * p.q_stride + (int64_t)head * hd) * ES;
  constexpr int QC = D / VEC / 2;  // chunks of Q per lane
  u32x4 qreg[QC];
#pragma unroll
  for (int i = 0; i < QC; ++i) {
    const int c = 2 * i + hf;  // 16-byte chunk of the row
    u32x4 z = {0u, 0u, 0u, 0u};
    if (qvalid && c * VEC < hd) z = *reinterpret_cast<const u32x4*>(qptr + c * 16);
    qreg[i] = z;
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;

  // ---- staging of one K/V tile: global -> registers -> LDS ----
  u32x4 kst[KPT];
  u32x4 vst[VPT][4];
  const char* kbase = p.k + ((int64_t)seg * p.k_stride + (int64_t)kvh * hd) * ES;
  const char* vbase = p.v + ((int64_t)seg * p.v_stride + (int64_t)kvh * hd) * ES;

  auto load_tile = [&](int t) {
    const int kt0 = t * BN;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int id = tid + i * NT;
      u32x4 z = {0u, 0u, 0u, 0u};
      if (NKC % NT == 0 || id < NKC) {
        const int row = id / CHK, c = id % CHK;
        const int key = kt0 + row;
        if (key < T && c * VEC < hd)
          z = *reinterpret_cast<const u32x4*>(kbase + ((int64_t)key * p.k_stride) * ES + c * 16);
      }
      kst[i] = z;
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int id = tid + i * NT;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4 z = {0u, 0u, 0u, 0u};
        if (NVU % NT == 0 || id < NVU) {
          const int g = id / CHK, c = id % CHK;
          const int key = kt0 + 4 * g + j;
          if (key < T && c * VEC < hd)
            z = *reinterpret_cast<const u32x4*>(vbase + ((int64_t)key * p.v_stride) * ES + c * 16);
        }
        vst[i][j] = z;
      }
    }
  };

  auto store_tile = [&](int buf) {
    char* sK = smem + buf * 2 * KT_BYTES;
    char* sV = sK + KT_BYTES;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int id = tid + i * NT;
      if (NKC % NT == 0 || id < NKC) {
        const int row = id / CHK, c = id % CHK;
        *reinterpret_cast<u32x4*>(sK + swz(row, c, KROW)) = kst[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int id = tid + i * NT;
      if (NVU % NT == 0 || id < NVU) {
        const int g = id / CHK, c = id % CHK;
        const int col = vcol<E>(4 * g);  // key column of this 4-key group
        if constexpr (ES == 2) {
          // 4 keys x 8 d (bf16) -> for each d, 4 consecutive keys (8 bytes)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int w = e >> 1;
            uint32_t a0 = vst[i][0][w], a1 = vst[i][1][w], a2 = vst[i][2][w], a3 = vst[i][3][w];
            uint32_t lo, hi;
            if constexpr (PV16) {
              // bf16 -> f32 (bit shift) -> fp16 (RNE; exact below 65504)
              auto f = [&](uint32_t x) { return __builtin_bit_cast(float, (e & 1) ? (x & 0xffff0000u) : (x << 16)); };
              f32x2 x01 = {f(a0), f(a1)}, x23 = {f(a2), f(a3)};
              lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(x01, f16x2));
              hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(x23, f16x2));
            } else if (e & 1) {
              lo = (a0 >> 16) | (a1 & 0xffff0000u);
              hi = (a2 >> 16) | (a3 & 0xffff0000u);
            } else {
              lo = (a0 & 0xffffu) | (a1 << 16);
              hi = (a2 & 0xffffu) | (a3 << 16);
            }
            const int dd = c * 8 + e;
            u32x2 val = {lo, hi};
            *reinterpret_cast<u32x2*>(sV + swz(dd, col >> 3, VROW) + (col & 7) * 2) = val;
          }
        } else {
          // 4 keys x 4 d (f32) -> for each d, 4 consecutive keys (16 bytes)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int dd = c * 4 + e;
            u32x4 val = {vst[i][0][e], vst[i][1][e], vst[i][2][e], vst[i][3][e]};
            *reinterpret_cast<u32x4*>(sV + swz(dd, col >> 2, VROW)) = val;
          }
        }
      }
    }
  };

  if (lo_t < hi_t) {
    load_tile(lo_t);
    store_tile(0);
  }
  __syncthreads();

  const float c2 = p.scale_log2;

  for (int t = lo_t; t < hi_t; ++t) {
    const int buf = (t - lo_t) & 1;
    const bool more = t + 1 < hi_t;
    if (more) load_tile(t + 1);

    const int kt0 = t * BN;
    if (active && kt0 < khi && kt0 + BN > klo) {
      const char* sK = smem + buf * 2 * KT_BYTES;
      const char* sV = sK + KT_BYTES;

      // ---- S^T = K . Q^T ----
      f32x16 sacc[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
        const int krow = kb * 32 + lq;
        if constexpr (ES == 2) {
#pragma unroll
          for (int st = 0; st < D / 16; ++st) {
            if (st * 16 < hd) {
              bf16x8 a = *reinterpret_cast<const bf16x8*>(sK + swz(krow, 2 * st + hf, KROW));
              bf16x8 b = __builtin_bit_cast(bf16x8, qreg[st]);
              sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, sacc[kb], 0, 0, 0);
            }
          }
        } else {
#pragma unroll
          for (int g = 0; g < D / 8; ++g) {
            if (g * 8 < hd) {
              f32x4 a = *reinterpret_cast<const f32x4*>(sK + swz(krow, 2 * g + hf, KROW));
              f32x4 b = __builtin_bit_cast(f32x4, qreg[g]);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], sacc[kb], 0, 0, 0);
            }
          }
        }
      }

      // ---- mask (only tiles that cross an edge of the visible region) ----
      const bool need_mask =
          (kt0 + BN > T) || (p.causal && kt0 + BN - 1 > r0) ||
          (p.window >= 0 && (rlast - kt0 > p.window || kt0 + BN - 1 - r0 > p.window));
      if (need_mask) {
        const int qi = r0 + lq;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kj = kt0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            bool ok = kj < T;
            if (p.causal) ok = ok && kj <= qi;
            if (p.window >= 0) ok = ok && abs(qi - kj) <= p.window;
            if (!ok) sacc[kb][r] = -INFINITY;
          }
      }

      // ---- online softmax (log2 domain, f32) ----
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
      mx = half_max(mx);
      const float m_new = fmaxf(m_i, mx * c2);
      const float base = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_i - base);
      m_i = m_new;
      l_i *= alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sacc[kb][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], c2, -base));

      // ---- O^T += V^T . P^T ----
      if constexpr (ES == 2) {
        // P is rounded (fp16, or bf16 with INL_ATTN_PV_BF16) for the product;
        // the row sum is taken over the same rounded values (in f32; the dot2
        // instructions would wait for the matrix core), so the weights that
        // multiply V sum exactly to the normaliser.
        typedef PT pt8 __attribute__((ext_vector_type(8)));
        typedef PT pt2 __attribute__((ext_vector_type(2)));
        pt8 pk[BN / 16];
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) {
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            f32x2 pr = {sacc[ks >> 1][8 * (ks & 1) + e], sacc[ks >> 1][8 * (ks & 1) + e + 1]};
            pt2 pair = __builtin_convertvector(pr, pt2);
            pk[ks][e] = pair[0];
            pk[ks][e + 1] = pair[1];
            l_i += (float)pair[0] + (float)pair[1];
          }
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          if (db * 32 < hd) {
            const int vrow = db * 32 + lq;
#pragma unroll
            for (int ks = 0; ks < BN / 16; ++ks) {
              pt8 a = *reinterpret_cast<const pt8*>(sV + swz(vrow, 2 * ks + hf, VROW));
              if constexpr (PV16)
                oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk[ks], oacc[db], 0, 0, 0);
              else
                oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pk[ks], oacc[db], 0, 0, 0);
            }
          }
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) l_i += sacc[kb][r];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          if (db * 32 < hd) {
            const int vrow = db * 32 + lq;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
              for (int q4 = 0; q4 < 4; ++q4) {
                f32x4 a = *reinterpret_cast<const f32x4*>(sV + swz(vrow, 8 * kb + 4 * hf + q4, VROW));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], sacc[kb][4 * q4 + e], oacc[db], 0, 0, 0);
              }
            }
          }
        }
      }
    }

    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, one query row per lane column ----
  if (!active || !qvalid) return;
  const float l_tot = half_sum(l_i);
  const int part = p.item_part ? p.item_part[item_idx] : -1;
  if (part >= 0) {
    // Part of the block's key range: unnormalised O with its row max and
    // sum, 32 rows of D floats per wave and head group.
    const int64_t slot = ((int64_t)part * p.n_hg + hg) * NW + wave;
    float* prow = p.part_o + (slot * 32 + lq) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hf;
        if (d0 < hd) {
          f32x4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = oacc[db][4 * g + e];
          *reinterpret_cast<f32x4*>(prow + d0) = val;
        }
      }
    if (hf == 0) p.part_ml[slot * 32 + lq] = make_float2(m_i, l_tot);
    return;
  }
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  char* orow = p.o + ((int64_t)(seg + qrow) * p.o_stride + (int64_t)head * hd) * (p.out_bf16 ? 2 : 4);
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = db * 32 + 8 * g + 4 * hf;
      if (d0 < hd) {
        if (p.out_bf16) {
          bf16x4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = (bf16)(oacc[db][4 * g + e] * inv);
          *reinterpret_cast<bf16x4*>(orow + d0 * 2) = val;
        } else {
          f32x4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = oacc[db][4 * g + e] * inv;
          *reinterpret_cast<f32x4*>(orow + d0 * 4) = val;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Merge of a split key range. A query block whose key tiles were split over
// several items has one partial slot per part (consecutive, from `first`);
// row r's output is sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M the
// largest m_s (parts in which the row saw no key have m_s = -inf, weight 0).
// One workgroup per (block, head group, wave of the attention kernel, half):
// 16 rows of 16 threads, each thread up to 4 chunks of 4 dims (head_dim <=
// 256). Parts are taken 4 at a time, all their loads issued before any is
// used, with a running max and rescale between groups.
// ---------------------------------------------------------------------------

struct MergeParams {
  const int4* blocks;     // {seg_start, seg_len, q0, first partial slot}
  const int32_t* n_parts; // parts per block
  const float* part_o;
  const float2* part_ml;
  char* o;
  int64_t o_stride;
  int32_t n_hg, nw, rb, hpw, group, groups_per_kv, head_dim, dpad, out_bf16;
};

constexpr int kMergeThreads = 256;
constexpr int kMergeTpr = 16;                           // threads per row
constexpr int kMergeRows = kMergeThreads / kMergeTpr;   // rows per workgroup
constexpr int kMergeWgPerWave = 32 / kMergeRows;

__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(MergeParams p) {
  constexpr int CPT = 256 / 4 / kMergeTpr;  // chunks per thread at head_dim 256
  constexpr int G = 4;                      // parts per group
  const int half = blockIdx.x % kMergeWgPerWave;
  const int w = (blockIdx.x / kMergeWgPerWave) % p.nw;
  const int bh = blockIdx.x / kMergeWgPerWave / p.nw;
  const int bi = bh / p.n_hg;
  const int hg = bh - bi * p.n_hg;
  const int4 blk = p.blocks[bi];
  const int ns = p.n_parts[bi];
  const int kvh = hg / p.groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * p.groups_per_kv) * p.hpw + w / p.rb;
  const int r = half * kMergeRows + threadIdx.x / kMergeTpr;  // row within the wave's 32
  const int sub = threadIdx.x % kMergeTpr;
  const int row = blk.z + (w % p.rb) * 32 + r;
  if (row >= blk.y) return;
  const int chunks = p.head_dim / 4;
  // part s of this wave's rows: slot (first + s) * n_hg * nw + hg * nw + w
  const int64_t slot0 = ((int64_t)blk.w * p.n_hg + hg) * p.nw + w;
  const int64_t sstep = (int64_t)p.n_hg * p.nw * 32;  // rows between parts
  const float2* ml = p.part_ml + slot0 * 32 + r;
  const float* po = p.part_o + (slot0 * 32 + r) * p.dpad;
  float mx = -INFINITY, l = 0.f;
  f32x4 acc[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < ns; s0 += G) {
    float2 m[G];
    f32x4 v[G][CPT];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int s = min(s0 + g, ns - 1);  // past the end: re-read the last part, weight 0
      m[g] = ml[s * sstep];
      const float* ps = po + s * sstep * p.dpad;
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int c = min(sub + kMergeTpr * j, chunks - 1);
        v[g][j] = *reinterpret_cast<const f32x4*>(ps + 4 * c);
      }
    }
    float gm = mx;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (s0 + g < ns) gm = fmaxf(gm, m[g].x);
    const float a = mx == -INFINITY ? 0.f : exp2f(mx - gm);  // rescale of the groups before
    l *= a;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j][e] *= a;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float wt = (s0 + g < ns && m[g].x != -INFINITY) ? exp2f(m[g].x - gm) : 0.f;
      l += m[g].y * wt;
#pragma unroll
      for (int j = 0; j < CPT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][e] += v[g][j][e] * wt;
    }
    mx = gm;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  char* orow = p.o + ((int64_t)(blk.x + row) * p.o_stride + (int64_t)head * p.head_dim) * (p.out_bf16 ? 2 : 4);
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = sub + kMergeTpr * j;
    if (c < chunks) {
      if (p.out_bf16) {
        bf16x4 val;
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = (bf16)(acc[j][e] * inv);
        *reinterpret_cast<bf16x4*>(orow + 8 * c) = val;
      } else {
        f32x4 val;
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = acc[j][e] * inv;
        *reinterpret_cast<f32x4*>(orow + 16 * c) = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: kernel selection, schedule, launch
// ---------------------------------------------------------------------------

typedef void (*KernelFn)(AttnParams);

struct KernelCfg {
  KernelFn fn;
  int d;        // compiled head dim (>= real head_dim)
  int bn;       // keys per tile
  int nw;       // waves per workgroup
  int lds;      // dynamic LDS bytes
  int rows;     // query rows per wave (32 or 64)
  bool persistent = false;  // one workgroup per CU over a host-assigned unit list
  bool head_pairs = false;  // a unit serves two query heads with their own K/V (group 1)
  const char* name = "";    // kernel name, for reporting
};

int unit_weight(const KernelCfg& cfg, const inl_attn_desc* d, int T, int q0, int BM, int lo_t, int hi_t) {
  const int tiles = hi_t - lo_t;
  if (!cfg.persistent) return 8 * tiles + 18;
  const int BN = cfg.bn;
  const int rows = std::min(T, q0 + BM) - q0;
  // Tiles on which some 32-row chunk of the unit needs a mask: those outside
  // the intersection of the chunks' unmasked tile ranges [f_lo, f_hi) (the
  // kernel's per-wave test); all of them when a chunk lies past the text.
  int a = lo_t, b = hi_t;
  bool all = false;
  for (int r0 = q0; r0 < q0 + BM && !all; r0 += 32) {
    if (r0 >= T) {
      all = true;
      break;
    }
    const int rlast = std::min(r0 + 31, T - 1);
    int e = T;
    if (d->causal) e = std::min(e, r0 + 1);
    if (d->window >= 0) e = std::min(e, r0 + d->window + 1);
    a = std::max(a, d->window >= 0 ? (std::max(0, rlast - d->window) + BN - 1) / BN : 0);
    b = std::min(b, e / BN);
  }
  const int masked = all ? tiles : tiles - std::max(0, b - a);
  if (cfg.d == 256) return 8 * tiles + 46 + masked + (rows * 7 + 32) / 64;
  return 8 * tiles + 17 + 3 * masked + (rows * 35 + 512) / 1024;
}

template <typename E, int D, int BN, int NW, bool PV16>
KernelCfg make_cfg(const char* name) {
  return KernelCfg{attn_fwd_kernel<E, D, BN, NW, PV16>, D, BN, NW, 4 * BN * D * (int)sizeof(E), 32, false, false,
                   name};
}

// `fits32`: every text's q/k/v rows span < 4 GiB, as the fast kernel's
// 32-bit buffer offsets need.
int select_kernel(int32_t dtype, int32_t head_dim, int32_t flags, bool fits32, int h_q, int group,
                  KernelCfg* cfg) {
  const bool pv16 = !(flags & INL_ATTN_PV_BF16);
  if (dtype == INL_BF16 && pv16 && fits32) {
    AttnKernelFn fn;
    int bn, nw, lds;
    if (group == 1 && h_q % 2 == 0 && bf16_pp64_kernel(head_dim, &fn, &bn, &nw, &lds)) {
      *cfg = KernelCfg{fn, head_dim, bn, nw, lds, 32, true, true, "attn_pp64_kernel<64, 64>"};
      return INL_OK;
    }
    if (bf16_pp_kernel(head_dim, &fn, &bn, &nw, &lds)) {
      *cfg = KernelCfg{fn, head_dim, bn, nw, lds, 32, true, false, "attn_pp_kernel<128, 64>"};
      return INL_OK;
    }
    if (bf16_wide_kernel(head_dim, &fn, &bn, &nw, &lds)) {
      *cfg = KernelCfg{fn, head_dim, bn, nw, lds, 32, true, false, "attn_wide_kernel<256, 32>"};
      return INL_OK;
    }
    if (bf16_fast_kernel(head_dim, &fn, &bn, &nw, &lds)) {
      *cfg = KernelCfg{fn, head_dim, bn, nw, lds, 32, false, false, "attn_bf16_kernel<64, 64, 4>"};
      return INL_OK;
    }
  }
  if (dtype == INL_BF16) {
    if (head_dim <= 64)
      *cfg = pv16 ? make_cfg<bf16, 64, 64, 4, true>("attn_fwd_kernel<bf16, 64, 64, 4, pv16>")
                  : make_cfg<bf16, 64, 64, 4, false>("attn_fwd_kernel<bf16, 64, 64, 4, pv_bf16>");
    else if (head_dim <= 128)
      *cfg = pv16 ? make_cfg<bf16, 128, 64, 4, true>("attn_fwd_kernel<bf16, 128, 64, 4, pv16>")
                  : make_cfg<bf16, 128, 64, 4, false>("attn_fwd_kernel<bf16, 128, 64, 4, pv_bf16>");
    else if (head_dim <= 256)
      *cfg = pv16 ? make_cfg<bf16, 256, 64, 4, true>("attn_fwd_kernel<bf16, 256, 64, 4, pv16>")
                  : make_cfg<bf16, 256, 64, 4, false>("attn_fwd_kernel<bf16, 256, 64, 4, pv_bf16>");
    else return fail(INL_E_UNSUPPORTED, "attention: head_dim > 256 is not supported");
  } else {
    if (head_dim <= 64) *cfg = make_cfg<float, 64, 64, 4, false>("attn_fwd_kernel<f32, 64, 64, 4>");
    else if (head_dim <= 128) *cfg = make_cfg<float, 128, 64, 4, false>("attn_fwd_kernel<f32, 128, 64, 4>");
    else if (head_dim <= 256) *cfg = make_cfg<float, 256, 32, 4, false>("attn_fwd_kernel<f32, 256, 32, 4>");
    else return fail(INL_E_UNSUPPORTED, "attention: head_dim > 256 is not supported");
  }
  return INL_OK;
}

// Largest divisor of `group` that also divides the wave count.
int heads_per_wg(int group, int nw) {
  for (int h = std::min(group, nw); h >= 1; --h)
    if (group % h == 0 && nw % h == 0) return h;
  return 1;
}

int validate_desc(const inl_attn_desc* d, int64_t* total_tokens) {
  if (!d) return fail(INL_E_INVALID, "attention: desc is NULL");
  if (!dtype_ok(d->dtype) || !dtype_ok(d->out_dtype))
    return fail(INL_E_INVALID, "attention: dtype must be INL_F32 or INL_BF16");
  if (d->h_q <= 0 || d->h_kv <= 0 || d->h_q % d->h_kv != 0)
    return fail(INL_E_INVALID, "attention: h_q must be a positive multiple of h_kv");
  if (d->head_dim < 8 || d->head_dim > 256 || d->head_dim % 8 != 0)
    return fail(INL_E_UNSUPPORTED, "attention: head_dim must be a multiple of 8 in [8, 256]");
  if (d->causal != 0 && d->causal != 1) return fail(INL_E_INVALID, "attention: causal must be 0 or 1");
  if (d->window < -1) return fail(INL_E_INVALID, "attention: window must be -1 or >= 0");
  if (d->flags & ~(INL_ATTN_PV_BF16 | INL_ATTN_NO_SPLIT)) return fail(INL_E_INVALID, "attention: unknown flags");
  if (!(d->scale > 0.f) || !std::isfinite(d->scale))
    return fail(INL_E_INVALID, "attention: scale must be finite and > 0");
  const int es = dtype_size(d->dtype);
  const int vec = 16 / es;
  auto stride_ok = [&](int64_t s, int64_t minimum, int esz) {
    return s >= minimum && (s * esz) % 16 == 0;
  };
  const int64_t qs = d->q_row_stride ? d->q_row_stride : (int64_t)d->h_q * d->head_dim;
  const int64_t ks = d->k_row_stride ? d->k_row_stride : (int64_t)d->h_kv * d->head_dim;
  const int64_t vs = d->v_row_stride ? d->v_row_stride : (int64_t)d->h_kv * d->head_dim;
  const int64_t os = d->o_row_stride ? d->o_row_stride : (int64_t)d->h_q * d->head_dim;
  (void)vec;
  if (!stride_ok(qs, (int64_t)d->h_q * d->head_dim, es) ||
      !stride_ok(ks, (int64_t)d->h_kv * d->head_dim, es) ||
      !stride_ok(vs, (int64_t)d->h_kv * d->head_dim, es) ||
      !stride_ok(os, (int64_t)d->h_q * d->head_dim, dtype_size(d->out_dtype)))
    return fail(INL_E_INVALID,
                "attention: row strides must cover all heads and be multiples of 16 bytes");
  if (d->n_texts < 0) return fail(INL_E_INVALID, "attention: n_texts < 0");
  if (d->n_texts > 0 && !d->cu_seqlens_host)
    return fail(INL_E_INVALID, "attention: cu_seqlens_host is NULL");
  int rc = check_cu(d->n_texts, d->cu_seqlens_host, total_tokens);
  if (rc) return rc;
  for (int b = 0; b < d->n_texts; ++b)
    if (d->cu_seqlens_host[b + 1] - d->cu_seqlens_host[b] >= (1 << 16) * 32)
      return fail(INL_E_UNSUPPORTED, "attention: a text longer than 2^21 tokens");
  if (d->seq_starts_host) {
    int64_t rows = 0;
    for (int b = 0; b < d->n_texts; ++b) {
      const int64_t st = d->seq_starts_host[b];
      const int64_t end = st + (d->cu_seqlens_host[b + 1] - d->cu_seqlens_host[b]);
      if (st < 0 || end > INT32_MAX)
        return fail(INL_E_INVALID, "attention: seq_starts_host[b] must be >= 0 and the text must end "
                                   "below row 2^31");
      rows = std::max(rows, end);
    }
    *total_tokens = rows;
  }
  return INL_OK;
}

size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

struct Schedule {
  // Work items (text, block of query rows, key-tile range), longest first.
  // For a persistent kernel: work units (item, head group) in workgroup order.
  std::vector<int4> items;
  std::vector<int32_t> unit_hg;   // persistent: head group of each unit
  std::vector<int32_t> wg_start;  // persistent: workgroup b runs units [wg_start[b], wg_start[b + 1])
  // Generic kernel with a split key range (empty otherwise): partial slot of
  // each item (-1: writes the output), and per split query block its
  // {seg_start, seg_len, q0, first slot} and number of parts.
  std::vector<int32_t> item_part;
  std::vector<int4> merge_blocks;
  std::vector<int32_t> merge_parts;
  int64_t n_slots = 0;            // partial slots (parts), each n_hg * nw * 32 rows
  int block_m = 0;
  int hpw = 1;
  int n_hg = 1;
  KernelCfg cfg{};

  // Device copy, one buffer: items, unit_hg, wg_start, item_part,
  // merge_blocks, merge_parts (the uploaded part, 16-byte aligned pieces),
  // then the partial (max, sum) and O areas, which the kernels fill.
  size_t hg_offset() const { return items.size() * sizeof(int4); }
  size_t wg_offset() const { return hg_offset() + align16(unit_hg.size() * sizeof(int32_t)); }
  size_t part_offset() const { return wg_offset() + align16(wg_start.size() * sizeof(int32_t)); }
  size_t mblk_offset() const { return part_offset() + align16(item_part.size() * sizeof(int32_t)); }
  size_t mparts_offset() const { return mblk_offset() + merge_blocks.size() * sizeof(int4); }
  size_t upload_bytes() const {
    return items.empty() ? 0 : align16(mparts_offset() + merge_parts.size() * sizeof(int32_t));
  }
  int64_t slot_rows() const { return n_slots * n_hg * cfg.nw * 32; }
  size_t ml_offset() const { return upload_bytes(); }
  size_t po_offset() const { return ml_offset() + align16((size_t)slot_rows() * sizeof(float2)); }
  size_t bytes() const {
    return n_slots == 0 ? upload_bytes() : po_offset() + (size_t)slot_rows() * cfg.d * sizeof(float);
  }
  std::vector<char> pack() const {
    std::vector<char> b(upload_bytes(), 0);
    if (b.empty()) return b;
    memcpy(b.data(), items.data(), hg_offset());
    if (!unit_hg.empty()) memcpy(b.data() + hg_offset(), unit_hg.data(), unit_hg.size() * sizeof(int32_t));
    if (!wg_start.empty()) memcpy(b.data() + wg_offset(), wg_start.data(), wg_start.size() * sizeof(int32_t));
    if (!item_part.empty())
      memcpy(b.data() + part_offset(), item_part.data(), item_part.size() * sizeof(int32_t));
    if (!merge_blocks.empty())
      memcpy(b.data() + mblk_offset(), merge_blocks.data(), merge_blocks.size() * sizeof(int4));
    if (!merge_parts.empty())
      memcpy(b.data() + mparts_offset(), merge_parts.data(), merge_parts.size() * sizeof(int32_t));
    return b;
  }
  int64_t n_units() const { return cfg.persistent ? (int64_t)items.size() : (int64_t)items.size() * n_hg; }
  int64_t grid() const { return cfg.persistent ? (int64_t)wg_start.size() - 1 : n_units(); }
};

int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  return n;
}

// Expected time of one persistent unit (text of T rows, query rows q0 ..
// q0 + BM - 1, key tiles lo_t .. hi_t - 1), in eighths of a key tile: a
// tile, 2.1 tiles per unit (Q in, O out, the switch), 0.4 per tile on which
// some 32-row wave needs a mask, and 0.55 per 128 query rows inside the
// text. Fitted (least squares, 2.8 % rms) to per-workgroup cycle counts of
// attn_pp over mixed-length causal and windowed batches; attn_pp64's own fit
// (1.4 % rms) is close to them. attn_wide (head_dim 256, 32-key tiles) has
// its own: 5.75 tiles per unit, 0.17 per masked tile and 1.75 per 128 rows
// (2.5 % rms).
struct KernelCfg;
int unit_weight(const KernelCfg& cfg, const inl_attn_desc* d, int T, int q0, int BM, int lo_t, int hi_t);

struct CostedItem {
  int4 it;
  int cost;        // key tiles
  int weight = 0;  // persistent kernels: expected time of one unit, in eighths of a tile
};

// Persistent schedule (`gpk`: head groups per KV head, consecutive in hg):
// every (item, head group) unit goes to the workgroup
// with the least work so far (longest units first, LPT), by the units'
// weights (unit_weight: tiles plus per-unit overhead).
// Workgroups are dispatched to the 8 XCDs round-robin (b % 8), and each XCD
// has its own L2; when the head groups split evenly over the XCDs, units of
// head group h run only on workgroups b with b % 8 == h % 8, so the K/V rows
// a head group reads are fetched into one L2.
// Placement refinement. The longest-first placement leaves the most loaded
// workgroup of an XCD class a few percent above the class mean, because a
// unit is large next to a workgroup's share (config 2: ~5.6 units per
// workgroup, predicted maximum 1.035x the mean). Up to 32 times per class,
// the most loaded workgroup trades one unit for a lighter one of a workgroup
// of its class (among the 16 least loaded), the trade that lowers the pair's
// maximum the most (config 2: predicted 1.015x). A trade keeps both lists'
// order, each unit taking the other's place, and is made only between units
// whose start times overlap: the units after them shift by the difference of
// the two weights alone, so every unit still runs beside the other q-blocks
// of its text and finds their K/V rows in L2. (Moving units between lists
// instead shifted whole list tails: 1.010x predicted, but 9-65 % more K/V
// reads from L2 misses. The trades cost config 2 1.010x -> 1.036x the
// algorithmic bytes for a 1.2 % faster step.)
void rebalance(const std::vector<CostedItem>& items, int n_hg, int classes,
               std::vector<std::vector<int64_t>>* lists_p) {
  std::vector<std::vector<int64_t>>& lists = *lists_p;
  const int64_t n_wg = (int64_t)lists.size();
  // unit weights, parallel to the lists
  std::vector<std::vector<int32_t>> wl(n_wg);
  std::vector<int64_t> load(n_wg, 0);
  for (int64_t b = 0; b < n_wg; ++b) {
    wl[b].reserve(lists[b].size());
    for (int64_t u : lists[b]) {
      wl[b].push_back(items[u / n_hg].weight);
      load[b] += wl[b].back();
    }
  }
  auto starts = [&](int64_t b, std::vector<int64_t>* st) {
    st->resize(wl[b].size());
    int64_t acc = 0;
    for (size_t k = 0; k < wl[b].size(); ++k) {
      (*st)[k] = acc;
      acc += wl[b][k];
    }
  };
  std::vector<int64_t> wgs, dst_c, ss, sd;
  for (int c = 0; c < classes; ++c) {
    wgs.clear();
    int64_t total = 0;
    for (int64_t b = c; b < n_wg; b += classes) {
      wgs.push_back(b);
      total += load[b];
    }
    if (wgs.size() < 2) continue;
    for (int iter = 0; iter < 32; ++iter) {
      int64_t src = wgs[0];
      for (int64_t b : wgs)
        if (load[b] > load[src]) src = b;
      const int64_t cur = load[src];
      // within 0.5 % of the class mean: done
      if (cur * 200 * (int64_t)wgs.size() <= total * 201) break;
      dst_c.assign(wgs.begin(), wgs.end());
      if (dst_c.size() > 16) {
        std::nth_element(dst_c.begin(), dst_c.begin() + 16, dst_c.end(),
                         [&](int64_t a, int64_t b) { return load[a] < load[b]; });
        dst_c.resize(16);
      }
      starts(src, &ss);
      int64_t best = cur, bd = -1;
      size_t bi = 0, bj = 0;
      const std::vector<int32_t>& ws = wl[src];
      for (int64_t d : dst_c) {
        if (d == src) continue;
        const int64_t ld = load[d];
        const std::vector<int32_t>& wdv = wl[d];
        starts(d, &sd);
        for (size_t i = 0; i < ws.size(); ++i) {
          const int64_t wa = ws[i];
          for (size_t j = 0; j < wdv.size(); ++j) {
            const int64_t diff = wa - wdv[j];
            if (diff <= 0) continue;
            if (std::abs(ss[i] - sd[j]) > std::max<int64_t>(wa, wdv[j])) continue;
            const int64_t nm = std::max(cur - diff, ld + diff);
            if (nm < best) { best = nm; bd = d; bi = i; bj = j; }
          }
        }
      }
      if (bd < 0) break;
      std::swap(lists[src][bi], lists[bd][bj]);
      const int64_t diff = (int64_t)wl[src][bi] - wl[bd][bj];
      std::swap(wl[src][bi], wl[bd][bj]);
      load[src] -= diff;
      load[bd] += diff;
    }
  }
}

void assign_units(const std::vector<CostedItem>& items, int n_hg, int gpk, Schedule* s) {
  const int64_t U = (int64_t)items.size() * n_hg;
  s->items.clear();
  s->unit_hg.clear();
  s->wg_start.assign(1, 0);
  if (U == 0) return;
  const int n_cu = device_cus();
  const bool affinity = n_hg % 8 == 0;
  int64_t n_wg = std::min<int64_t>(n_cu, U);
  n_wg = std::max<int64_t>(n_wg, (U + PP_MAX_UNITS - 1) / PP_MAX_UNITS);
  n_wg = (n_wg + 7) / 8 * 8;
  // Stream affinity: without head-group affinity, each (text, KV head)
  // stream, or each piece of a long one, goes to one XCD class (longest
  // first to the class with the least work), so the q-blocks that re-read
  // its K/V rows share one L2. Used when there are enough streams, the
  // classes balance, and no class outgrows its workgroups' unit tables.
  const int n_kv = n_hg / gpk;
  std::vector<int> text_of(items.size());
  std::unordered_map<int, int> text_id;   // text start row -> text number, in first-seen order
  for (size_t i = 0; i < items.size(); ++i)
    text_of[i] = text_id.emplace(items[i].it.x, (int)text_id.size()).first->second;
  const int n_texts = (int)text_id.size();
  std::vector<int> stream_class;
  bool streams = false;
  if (!affinity && n_wg >= 8 && (int64_t)items.size() * n_kv >= 32) {
    const int64_t n_streams = (int64_t)n_texts * n_kv;
    if (n_streams >= 32) {
      // Streams in pieces of contiguous query blocks, each at most half a
      // class's share of the work: one long text then spreads over several
      // XCDs instead of overloading one (its K/V rows are re-read per piece,
      // which a sliding window mostly confines to the piece's own rows).
      std::vector<std::vector<size_t>> text_items(n_texts);
      int64_t total = 0;
      for (size_t i = 0; i < items.size(); ++i) {
        text_items[text_of[i]].push_back(i);
        total += (int64_t)n_kv * gpk * items[i].weight;
      }
      const int64_t cap = std::max<int64_t>(1, total / 16);
      std::vector<int64_t> piece_cost, piece_units;
      std::vector<int64_t> piece_of(items.size() * n_kv);
      for (int t = 0; t < n_texts; ++t) {
        std::vector<size_t>& ti = text_items[t];
        std::stable_sort(ti.begin(), ti.end(), [&](size_t a, size_t b) { return items[a].it.z < items[b].it.z; });
        for (int kv = 0; kv < n_kv; ++kv) {
          int64_t acc = 0;
          for (size_t i : ti) {
            const int64_t c = (int64_t)gpk * items[i].weight;
            if (acc == 0 || acc + c > cap) {
              piece_cost.push_back(0);
              piece_units.push_back(0);
              acc = 0;
            }
            acc += c;
            piece_cost.back() += c;
            piece_units.back() += gpk;
            piece_of[i * n_kv + kv] = (int64_t)piece_cost.size() - 1;
          }
        }
      }
      const int64_t n_pieces = (int64_t)piece_cost.size();
      std::vector<int64_t> order(n_pieces);
      for (int64_t k = 0; k < n_pieces; ++k) order[k] = k;
      std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return piece_cost[a] > piece_cost[b]; });
      std::vector<int> cls(n_pieces);
      std::vector<int64_t> cls_units(8, 0), cls_cost(8, 0);
      std::priority_queue<std::pair<int64_t, int>, std::vector<std::pair<int64_t, int>>, std::greater<std::pair<int64_t, int>>> ch;
      for (int c = 0; c < 8; ++c) ch.push({0, c});
      for (int64_t k : order) {
        auto top = ch.top();
        ch.pop();
        cls[k] = top.second;
        cls_units[top.second] += piece_units[k];
        cls_cost[top.second] = top.first + piece_cost[k];
        ch.push({top.first + piece_cost[k], top.second});
      }
      // Classes must fit their workgroups' unit tables and balance within
      // 10 %; otherwise no stream affinity.
      const int64_t cmax = *std::max_element(cls_cost.begin(), cls_cost.end());
      streams = *std::max_element(cls_units.begin(), cls_units.end()) <= (n_wg / 8) * (int64_t)PP_MAX_UNITS &&
                cmax * 8 * 10 <= total * 11;
      if (streams) {
        stream_class.resize(items.size() * n_kv);
        for (size_t i = 0; i < items.size(); ++i)
          for (int kv = 0; kv < n_kv; ++kv) stream_class[i * n_kv + kv] = cls[piece_of[i * n_kv + kv]];
      }
    }
  }
  const int classes = affinity || streams ? 8 : 1;
  std::vector<std::vector<int64_t>> lists(n_wg);  // unit = item * n_hg + hg
  typedef std::pair<int64_t, int64_t> Load;       // (cost so far, workgroup)
  std::vector<std::priority_queue<Load, std::vector<Load>, std::greater<Load>>> heaps(classes);
  for (int64_t b = 0; b < n_wg; ++b) heaps[b % classes].push(Load(0, b));
  auto place = [&](size_t i, int hg) {
    auto& h = heaps[streams ? stream_class[i * n_kv + hg / gpk] : hg % classes];
    Load top = h.top();
    h.pop();
    lists[top.second].push_back((int64_t)i * n_hg + hg);
    if ((int)lists[top.second].size() < PP_MAX_UNITS) h.push(Load(top.first + items[i].weight, top.second));
  };
  // Texts in groups of about one unit per workgroup (texts by total cost,
  // longest first), each group longest unit first. The q-blocks of a text
  // then run at about the same time, while its K/V rows are in L2 (a plain
  // longest-first order spreads a causal text's q-blocks over the whole
  // launch), and within a group the longest-first order keeps the balance.
  // Among units of equal cost: KV head major, then item, then the head
  // groups that share the KV head, so that neighbours read the same rows.
  std::vector<int64_t> text_cost(n_texts, 0);
  std::vector<std::vector<size_t>> text_items(n_texts);
  for (size_t i = 0; i < items.size(); ++i) {
    text_cost[text_of[i]] += items[i].weight;
    text_items[text_of[i]].push_back(i);
  }
  std::vector<int> text_order(n_texts);
  for (int t = 0; t < n_texts; ++t) text_order[t] = t;
  std::stable_sort(text_order.begin(), text_order.end(),
                   [&](int a, int b) { return text_cost[a] > text_cost[b]; });
  std::vector<size_t> grp;
  for (size_t t = 0; t < text_order.size();) {
    grp.clear();
    int64_t units = 0;
    while (t < text_order.size() && units < n_wg) {
      for (size_t i : text_items[text_order[t]]) grp.push_back(i);
      units += (int64_t)text_items[text_order[t]].size() * n_hg;
      ++t;
    }
    std::stable_sort(grp.begin(), grp.end(), [&](size_t a, size_t b) { return items[a].cost > items[b].cost; });
    for (size_t j0 = 0; j0 < grp.size();) {
      size_t j1 = j0 + 1;
      while (j1 < grp.size() && items[grp[j1]].cost == items[grp[j0]].cost) ++j1;
      for (int kv = 0; kv < n_hg / gpk; ++kv)
        for (size_t j = j0; j < j1; ++j)
          for (int g = 0; g < gpk; ++g) place(grp[j], kv * gpk + g);
      j0 = j1;
    }
  }
  // Only with head-group affinity: under stream affinity (one K/V stream per
  // XCD, long texts re-read in rounds) the trades cost more K/V traffic than
  // they save time (EmbeddingGemma full attention: 1.1 % faster, 2.23x ->
  // 2.62x the algorithmic bytes).
  if (affinity) rebalance(items, n_hg, classes, &lists);
  s->items.reserve(U);
  s->unit_hg.reserve(U);
  // Without head-group affinity, equal-cost units (the q-blocks of one text,
  // and the head groups of one item, in order) go round-robin to logical
  // workgroups 0, 1, 2, ...; workgroup b = 8 j + x runs logical list
  // x * (n_wg / 8) + j, so each run of n_wg / 8 consecutive lists shares one
  // XCD and its L2 holds the K/V rows that neighbouring q-blocks re-read.
  const bool spread = classes == 1 && n_wg % 8 == 0;
  const int64_t per_xcd = n_wg / 8;
  for (int64_t pb = 0; pb < n_wg; ++pb) {
    const int64_t b = spread ? (pb % 8) * per_xcd + pb / 8 : pb;
    for (int64_t u : lists[b]) {
      s->items.push_back(items[u / n_hg].it);
      s->unit_hg.push_back((int32_t)(u % n_hg));
    }
    s->wg_start.push_back((int32_t)s->items.size());
  }
}

// Key-range split for the generic f32 kernel. Its workgroups hold one query
// block each and walk the block's key tiles in order, so a small batch
// (fewer workgroups than the GPU holds at once) takes as long as its longest
// block: 4 tiles of about 7 us each for a 256-token causal text at head_dim
// 128. Cutting blocks into parts of at most `c` tiles, each part a workgroup
// of its own, and merging the parts afterwards shortens that. `c` minimises
// an estimate in tile times: the workgroups, longest first, dispatched to
// the first free slot of the GPU (each costs its tiles plus half a tile of
// loads and stores), plus one tile for the merge launch if anything is
// split. Batches with many more workgroups than slots are not split.
// bf16 descs take the persistent kernels or run unsplit.
constexpr int kLdsPerCu = 160 * 1024;
constexpr size_t kMaxPartialBytes = (size_t)256 << 20;

void split_key_ranges(const inl_attn_desc* d, std::vector<CostedItem>& tmp, Schedule* s) {
  if (d->dtype != INL_F32 || (d->flags & INL_ATTN_NO_SPLIT) || tmp.empty()) return;
  const int max_tiles = tmp.front().cost;  // sorted longest first
  if (max_tiles < 2) return;
  const int64_t resident = (int64_t)device_cus() * std::max(1, kLdsPerCu / std::max(1, s->cfg.lds));
  if ((int64_t)tmp.size() * s->n_hg > 16 * resident) return;
  auto est = [&](int c) {
    std::vector<int> parts;
    for (const CostedItem& it : tmp)
      for (int t = 0; t < it.cost; t += c) parts.push_back(std::min(c, it.cost - t));
    std::stable_sort(parts.begin(), parts.end(), [](int a, int b) { return a > b; });
    std::priority_queue<double, std::vector<double>, std::greater<double>> free_at;
    for (int64_t i = 0; i < resident; ++i) free_at.push(0.0);
    double end = 0.0;
    for (int cost : parts)
      for (int h = 0; h < s->n_hg; ++h) {
        const double t = free_at.top() + cost + 0.5;
        free_at.pop();
        free_at.push(t);
        end = std::max(end, t);
      }
    return end + (c < max_tiles ? 1.0 : 0.0);
  };
  int c_best = max_tiles;
  double e_best = est(max_tiles);
  int c = 1;
  while (2 * c < max_tiles) c *= 2;
  for (; c >= 1; c /= 2) {
    const double e = est(c);
    if (e < e_best - 0.01) { e_best = e; c_best = c; }
  }
  if (c_best >= max_tiles) return;
  int64_t slots = 0;
  for (const CostedItem& it : tmp)
    if (it.cost > c_best) slots += (it.cost + c_best - 1) / c_best;
  const size_t row_bytes = sizeof(float2) + (size_t)s->cfg.d * sizeof(float);
  if ((size_t)slots * s->n_hg * s->cfg.nw * 32 * row_bytes > kMaxPartialBytes) return;
  std::vector<CostedItem> out;
  std::vector<int32_t> part;
  int32_t next = 0;
  for (const CostedItem& it : tmp) {
    if (it.cost <= c_best) {
      out.push_back(it);
      part.push_back(-1);
      continue;
    }
    const int lo_t = (int)((uint32_t)it.it.w >> 16), hi_t = it.it.w & 0xffff;
    s->merge_blocks.push_back(make_int4(it.it.x, it.it.y, it.it.z, next));
    s->merge_parts.push_back((hi_t - lo_t + c_best - 1) / c_best);
    for (int t = lo_t; t < hi_t; t += c_best) {
      const int t1 = std::min(t + c_best, hi_t);
      out.push_back({make_int4(it.it.x, it.it.y, it.it.z, (t << 16) | t1), t1 - t});
      part.push_back(next++);
    }
  }
  // longest parts first, as for unsplit items
  std::vector<size_t> order(out.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return out[a].cost > out[b].cost; });
  tmp.clear();
  s->item_part.clear();
  for (size_t i : order) {
    tmp.push_back(out[i]);
    s->item_part.push_back(part[i]);
  }
  s->n_slots = next;
}

// `allow_split`: false for the allocation-free entry, whose static buffer
// holds schedules, not partial outputs.
int build_schedule(const inl_attn_desc* d, Schedule* s, bool allow_split = true) {
  int64_t max_t = 0;
  for (int b = 0; b < d->n_texts; ++b)
    max_t = std::max<int64_t>(max_t, d->cu_seqlens_host[b + 1] - d->cu_seqlens_host[b]);
  const int es = dtype_size(d->dtype);
  const int64_t qs = d->q_row_stride ? d->q_row_stride : (int64_t)d->h_q * d->head_dim;
  const int64_t ks = d->k_row_stride ? d->k_row_stride : (int64_t)d->h_kv * d->head_dim;
  const int64_t vs = d->v_row_stride ? d->v_row_stride : (int64_t)d->h_kv * d->head_dim;
  const int64_t os = d->o_row_stride ? d->o_row_stride : (int64_t)d->h_q * d->head_dim;
  // The persistent kernels address each text's q, k, v and out rows with
  // 32-bit buffer offsets; the output row (f32 out is twice a bf16 input
  // row, and a caller stride may be wider) counts like the input rows.
  const int64_t widest = std::max(std::max(qs, std::max(ks, vs)) * es, os * dtype_size(d->out_dtype));
  const bool fits32 = (max_t + 256) * widest < ((int64_t)1 << 32);
  int rc = select_kernel(d->dtype, d->head_dim, d->flags, fits32, d->h_q, d->h_q / d->h_kv, &s->cfg);
  if (rc) return rc;
  const int group = d->h_q / d->h_kv;
  if (s->cfg.head_pairs) {
    // two heads per unit, one per wave group: 4 waves x 32 rows
    s->hpw = 2;
    s->n_hg = d->h_q / 2;
    s->block_m = s->cfg.rows * (s->cfg.nw / 2);
  } else {
    s->hpw = heads_per_wg(group, s->cfg.nw);
    s->n_hg = d->h_kv * (group / s->hpw);
    s->block_m = s->cfg.rows * (s->cfg.nw / s->hpw);
  }
  const int BM = s->block_m, BN = s->cfg.bn;
  std::vector<CostedItem> tmp;
  for (int b = 0; b < d->n_texts; ++b) {
    const int seg = d->seq_starts_host ? d->seq_starts_host[b] : d->cu_seqlens_host[b];
    const int T = d->cu_seqlens_host[b + 1] - d->cu_seqlens_host[b];
    for (int q0 = 0; q0 < T; q0 += BM) {
      const int qlast = std::min(q0 + BM, T) - 1;
      int lo = 0, hi = d->causal ? qlast + 1 : T;
      if (d->window >= 0) {
        lo = std::max(0, q0 - d->window);
        hi = std::min(hi, qlast + d->window + 1);
      }
      const int lo_t = lo / BN, hi_t = (hi + BN - 1) / BN;
      if (hi_t > 0xffff)
        return fail(INL_E_UNSUPPORTED, "attention: a text spans more than 65535 key tiles");
      tmp.push_back({make_int4(seg, T, q0, (lo_t << 16) | hi_t), hi_t - lo_t,
                     unit_weight(s->cfg, d, T, q0, BM, lo_t, hi_t)});
    }
  }
  std::stable_sort(tmp.begin(), tmp.end(),
                   [](const CostedItem& a, const CostedItem& b) { return a.cost > b.cost; });
  if (s->cfg.persistent) {
    if ((int64_t)tmp.size() * s->n_hg > INT32_MAX)
      return fail(INL_E_UNSUPPORTED, "attention: too many tiles for one launch");
    assign_units(tmp, s->n_hg, s->cfg.head_pairs ? 1 : group / s->hpw, s);
    return INL_OK;
  }
  if (allow_split) split_key_ranges(d, tmp, s);
  if ((int64_t)tmp.size() * s->n_hg > INT32_MAX)
    return fail(INL_E_UNSUPPORTED, "attention: too many tiles for one launch");
  s->items.resize(tmp.size());
  for (size_t i = 0; i < tmp.size(); ++i) s->items[i] = tmp[i].it;
  return INL_OK;
}

// `dev_sched`: the device copy of s.pack().
AttnParams make_params(const inl_attn_desc* d, const Schedule& s, const void* dev_sched,
                       const void* q, const void* k, const void* v, void* out) {
  AttnParams p{};
  p.q = (const char*)q;
  p.k = (const char*)k;
  p.v = (const char*)v;
  p.o = (char*)out;
  p.q_stride = d->q_row_stride ? d->q_row_stride : (int64_t)d->h_q * d->head_dim;
  p.k_stride = d->k_row_stride ? d->k_row_stride : (int64_t)d->h_kv * d->head_dim;
  p.v_stride = d->v_row_stride ? d->v_row_stride : (int64_t)d->h_kv * d->head_dim;
  p.o_stride = d->o_row_stride ? d->o_row_stride : (int64_t)d->h_q * d->head_dim;
  p.items = (const int4*)dev_sched;
  p.unit_hg = (const int32_t*)((const char*)dev_sched + s.hg_offset());
  p.wg_start = (const int32_t*)((const char*)dev_sched + s.wg_offset());
  p.group = d->h_q / d->h_kv;
  p.hpw = s.hpw;
  p.groups_per_kv = s.cfg.head_pairs ? 1 : p.group / s.hpw;
  p.n_hg = s.n_hg;
  p.rb = s.cfg.nw / s.hpw;
  p.head_dim = d->head_dim;
  p.causal = d->causal;
  p.window = d->window;
  p.scale_log2 = d->scale * kLog2e;
  p.out_bf16 = d->out_dtype == INL_BF16;
  if (s.n_slots) {
    char* base = (char*)dev_sched;
    p.item_part = (const int32_t*)(base + s.part_offset());
    p.part_ml = (float2*)(base + s.ml_offset());
    p.part_o = (float*)(base + s.po_offset());
  }
  return p;
}

// The dynamic LDS limit of a kernel is raised once per (kernel, device):
// plans do it when they are created, the one-shot forms before their first
// launch on a device. Launches then take no lock.
std::mutex g_attr_mu;
std::set<std::pair<const void*, int>> g_attr_done;

int ensure_lds_attr(const KernelCfg& cfg) {
  int dev = 0;
  INL_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_attr_mu);
  if (g_attr_done.count({(const void*)cfg.fn, dev})) return INL_OK;
  INL_HIP_TRY(hipFuncSetAttribute((const void*)cfg.fn, hipFuncAttributeMaxDynamicSharedMemorySize, cfg.lds));
  g_attr_done.insert({(const void*)cfg.fn, dev});
  return INL_OK;
}

int launch(const Schedule& s, const AttnParams& p, hipStream_t stream) {
  const KernelCfg& cfg = s.cfg;
  const int64_t blocks = s.grid();
  if (blocks <= 0) return INL_OK;
  if (blocks > 0x7fffffff) return fail(INL_E_UNSUPPORTED, "attention: too many tiles for one launch");
  hipLaunchKernelGGL(cfg.fn, dim3((unsigned)blocks), dim3(cfg.nw * 64), cfg.lds, stream, p);
  INL_HIP_TRY(hipGetLastError());
  if (!s.merge_blocks.empty()) {
    MergeParams m{};
    const char* base = (const char*)p.items;
    m.blocks = (const int4*)(base + s.mblk_offset());
    m.n_parts = (const int32_t*)(base + s.mparts_offset());
    m.part_o = p.part_o;
    m.part_ml = p.part_ml;
    m.o = p.o;
    m.o_stride = p.o_stride;
    m.n_hg = p.n_hg;
    m.nw = cfg.nw;
    m.rb = p.rb;
    m.hpw = p.hpw;
    m.group = p.group;
    m.groups_per_kv = p.groups_per_kv;
    m.head_dim = p.head_dim;
    m.dpad = cfg.d;
    m.out_bf16 = p.out_bf16;
    const int64_t mgrid = (int64_t)s.merge_blocks.size() * s.n_hg * cfg.nw * kMergeWgPerWave;
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)mgrid), dim3(kMergeThreads), 0, stream, m);
    INL_HIP_TRY(hipGetLastError());
  }
  return INL_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

int check_ptrs(const void* q, const void* k, const void* v, const void* out, int64_t total) {
  if (total == 0) return INL_OK;
  if (!q || !k || !v || !out) return fail(INL_E_INVALID, "attention: NULL tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(INL_E_INVALID, "attention: q, k, v and out must be 16-byte aligned");
  return INL_OK;
}

}  // namespace

}  // namespace inl

namespace inl {
namespace {

// Upload a schedule into device memory `buf` (a caller workspace or the
// static scratch) and launch. The schedule is copied from ordinary (pageable)
// host memory: hipMemcpyAsync takes the data before it returns, so nothing
// pinned is allocated; the copy orders behind the stream's earlier work.
int launch_one_shot(const inl_attn_desc* desc, const Schedule& s, void* buf, const void* q, const void* k,
                    const void* v, void* out, hipStream_t stream) {
  int rc = ensure_lds_attr(s.cfg);
  if (rc) return rc;
  const std::vector<char> blob = s.pack();
  INL_HIP_TRY(hipMemcpyAsync(buf, blob.data(), blob.size(), hipMemcpyHostToDevice, stream));
  AttnParams p = make_params(desc, s, buf, q, k, v, out);
  return launch(s, p, stream);
}

}  // namespace
}  // namespace inl

struct inl_attn_plan {
  inl_attn_desc desc;     // cu_seqlens_host and seq_starts_host are not kept
  inl::Schedule sched;    // also kept on the host for inspection
  std::vector<char> host_blob;   // the uploaded schedule bytes (inl_attn_plan_create_in), kept with the plan
  void* d_sched = nullptr;
  bool owns_sched = true; // false: d_sched is the caller's workspace
  int64_t total_tokens = 0;
};

extern "C" int inl_attn_plan_create(const inl_attn_desc* desc, inl_attn_plan** plan) {
  using namespace inl;
  if (!plan) return fail(INL_E_INVALID, "attention: plan out-pointer is NULL");
  *plan = nullptr;
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  inl_attn_plan* pl = new (std::nothrow) inl_attn_plan();
  if (!pl) return fail(INL_E_NOMEM, "attention: host allocation failed");
  pl->desc = *desc;
  pl->desc.cu_seqlens_host = nullptr;
  pl->desc.seq_starts_host = nullptr;
  pl->total_tokens = total;
  rc = build_schedule(desc, &pl->sched);
  if (rc) { delete pl; return rc; }
  rc = ensure_lds_attr(pl->sched.cfg);
  if (rc) { delete pl; return rc; }
  const std::vector<char> blob = pl->sched.pack();
  if (!blob.empty()) {
    hipError_t e = hipMalloc(&pl->d_sched, pl->sched.bytes());
    if (e != hipSuccess) { delete pl; return hip_fail(e, "hipMalloc(plan)"); }
    e = hipMemcpy(pl->d_sched, blob.data(), blob.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) { (void)hipFree(pl->d_sched); delete pl; return hip_fail(e, "hipMemcpy(plan)"); }
  }
  *plan = pl;
  return INL_OK;
}

namespace inl {

int attn_plan_prepare(const inl_attn_desc* desc, void* dev_sched, size_t workspace_bytes, std::vector<char>* blob,
                      inl_attn_plan** plan) {
  if (!plan || !blob) return fail(INL_E_INVALID, "attention: plan out-pointer is NULL");
  *plan = nullptr;
  blob->clear();
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  inl_attn_plan* pl = new (std::nothrow) inl_attn_plan();
  if (!pl) return fail(INL_E_NOMEM, "attention: host allocation failed");
  pl->desc = *desc;
  pl->desc.cu_seqlens_host = nullptr;
  pl->desc.seq_starts_host = nullptr;
  pl->total_tokens = total;
  pl->owns_sched = false;
  rc = build_schedule(desc, &pl->sched);
  if (!rc) rc = ensure_lds_attr(pl->sched.cfg);
  if (!rc) *blob = pl->sched.pack();
  if (!rc && !blob->empty()) {
    if (!dev_sched || workspace_bytes < pl->sched.bytes())
      rc = fail(INL_E_INVALID, "attention: workspace is NULL or smaller than inl_attn_workspace_size()");
    else if (!aligned16(dev_sched))
      rc = fail(INL_E_INVALID, "attention: workspace must be 16-byte aligned");
    else
      pl->d_sched = dev_sched;
  }
  if (rc) {
    delete pl;
    blob->clear();
    return rc;
  }
  *plan = pl;
  return INL_OK;
}

}  // namespace inl

extern "C" int inl_attn_plan_create_in(const inl_attn_desc* desc, void* workspace, size_t workspace_bytes,
                                       void* stream, inl_attn_plan** plan) {
  using namespace inl;
  std::vector<char> blob;
  int rc = attn_plan_prepare(desc, workspace, workspace_bytes, &blob, plan);
  if (rc || blob.empty()) return rc;
  // the plan keeps the host copy of its schedule until it is destroyed
  (*plan)->host_blob = std::move(blob);
  const hipError_t e = hipMemcpyAsync(workspace, (*plan)->host_blob.data(), (*plan)->host_blob.size(),
                                      hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e != hipSuccess) {
    delete *plan;
    *plan = nullptr;
    return hip_fail(e, "hipMemcpyAsync(plan)");
  }
  return INL_OK;
}

extern "C" int inl_attn_plan_destroy(inl_attn_plan* plan) {
  if (!plan) return INL_OK;
  int rc = INL_OK;
  if (plan->d_sched && plan->owns_sched) {
    hipError_t e = hipFree(plan->d_sched);
    if (e != hipSuccess) rc = inl::hip_fail(e, "hipFree(plan)");
  }
  delete plan;
  return rc;
}

extern "C" int inl_attn_plan_info(const inl_attn_plan* plan, int64_t* n_tiles,
                                  int32_t* block_m, int32_t* block_n) {
  if (!plan) return inl::fail(INL_E_INVALID, "attention: plan is NULL");
  if (n_tiles) *n_tiles = plan->sched.n_units();
  if (block_m) *block_m = plan->sched.block_m;
  if (block_n) *block_n = plan->sched.cfg.bn;
  return INL_OK;
}

extern "C" int inl_attn_fwd(const inl_attn_plan* plan, const void* q, const void* k,
                            const void* v, void* out, void* stream) {
  using namespace inl;
  if (!plan) return fail(INL_E_INVALID, "attention: plan is NULL");
  int rc = check_ptrs(q, k, v, out, plan->total_tokens);
  if (rc) return rc;
  AttnParams p = make_params(&plan->desc, plan->sched, plan->d_sched, q, k, v, out);
  return launch(plan->sched, p, (hipStream_t)stream);
}

extern "C" int inl_attn_workspace_size(const inl_attn_desc* desc, size_t* bytes) {
  using namespace inl;
  if (!bytes) return fail(INL_E_INVALID, "attention: bytes out-pointer is NULL");
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  Schedule s;
  rc = build_schedule(desc, &s);
  if (rc) return rc;
  *bytes = s.bytes();
  return INL_OK;
}

extern "C" int inl_attn_varlen_fwd(const inl_attn_desc* desc, const void* q, const void* k,
                                   const void* v, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  using namespace inl;
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  rc = check_ptrs(q, k, v, out, total);
  if (rc) return rc;
  Schedule s;
  rc = build_schedule(desc, &s);
  if (rc) return rc;
  const size_t need = s.bytes();
  if (need == 0) return INL_OK;
  if (!workspace || workspace_bytes < need)
    return fail(INL_E_INVALID, "attention: workspace is NULL or smaller than inl_attn_workspace_size()");
  if (!aligned16(workspace)) return fail(INL_E_INVALID, "attention: workspace must be 16-byte aligned");
  return launch_one_shot(desc, s, workspace, q, k, v, out, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Allocation-free one-shot form: the schedule goes into `scratch`, a static
// device array of the library, instead of a caller workspace.
// ---------------------------------------------------------------------------

namespace inl {
namespace {

// Each GPU the library runs on holds its own copy until the process ends.
// Host code never uses this name as an address: it is a host-side stand-in.
// The device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[INL_ATTN_STATIC_SCHEDULE_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The calling thread's current device's copy of `scratch`, looked up on the
// first call on that device (with that device current).
int scratch_on_current_device(void** ptr) {
  int dev = 0;
  INL_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(INL_E_UNSUPPORTED, "attention: device ordinal beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    INL_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(INL_E_HIP, "attention: hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return INL_OK;
}

}  // namespace
}  // namespace inl

extern "C" int inl_attn_varlen_fwd_static(const inl_attn_desc* desc, const void* q, const void* k,
                                          const void* v, void* out, void* stream) {
  using namespace inl;
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  rc = check_ptrs(q, k, v, out, total);
  if (rc) return rc;
  Schedule s;
  rc = build_schedule(desc, &s, /*allow_split=*/false);
  if (rc) return rc;
  const size_t need = s.bytes();
  if (need == 0) return INL_OK;
  if (need > INL_ATTN_STATIC_SCHEDULE_BYTES)
    return fail(INL_E_INVALID, "attention: the batch's schedule needs " + std::to_string(need) +
                                   " bytes, more than the static buffer's " +
                                   std::to_string((size_t)INL_ATTN_STATIC_SCHEDULE_BYTES) +
                                   "; split the batch or use inl_attn_varlen_fwd with a workspace");
  void* buf = nullptr;
  rc = scratch_on_current_device(&buf);
  if (rc) return rc;
  return launch_one_shot(desc, s, buf, q, k, v, out, (hipStream_t)stream);
}

extern "C" int inl_attn_kernel_name(const inl_attn_desc* desc, const char** name) {
  using namespace inl;
  if (!name) return fail(INL_E_INVALID, "attention: name out-pointer is NULL");
  *name = nullptr;
  int64_t total = 0;
  int rc = validate_desc(desc, &total);
  if (rc) return rc;
  Schedule s;
  rc = build_schedule(desc, &s);
  if (rc) return rc;
  *name = s.cfg.name;
  return INL_OK;
}
