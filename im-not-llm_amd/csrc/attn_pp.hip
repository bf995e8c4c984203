// Ping-pong bf16 attention for head_dim 128 on gfx950.
//
// Same schedule, masks and results as the other attention kernels (see
// attn_fwd.hip for the per-wave math: S^T = K.Q^T on bf16 MFMA, lane-local
// softmax on query columns, O^T += V^T.P^T on fp16 MFMA with P rounded to
// fp16 and the row sum taken over the rounded values), arranged so that the
// matrix cores never wait for the softmax:
//
//   - A workgroup is 8 waves in two groups of 4 (waves 0-3, 4-7). The two
//     waves of one SIMD belong to different groups. Each wave owns 32 query
//     rows of one head; both groups share every K/V tile staged in LDS.
//   - Execution alternates between two half-slots separated by barriers. In
//     one half-slot group 0 runs its MFMA phase while group 1 runs its
//     softmax phase; in the next the roles swap. One SIMD therefore always
//     has one wave issuing MFMAs and one issuing VALU work, and the hardware
//     interleaves the two.
//   - MFMA phase of tile j: O^T += V_{j-1}^T P_{j-1}^T, S^T = K_j Q^T, and the
//     in-place bf16 -> fp16 conversion of the wave's own slice of V_j (VALU
//     work that fits between its MFMAs).
//   - Softmax phase of tile j: row max, then P = exp2(s * c - m) against a
//     reference max m that moves only when a row's max exceeds it by more
//     than 8 (log2 units), so O and l are rarely rescaled and P <= 256.
//   - K and V tiles go global -> LDS with direct loads issued two tiles ahead
//     into 4 stages each; every wave loads (and converts) the same 1/8 slice
//     of every tile, so a wave's conversion waits only on its own loads.
//
// LDS layout (per stage, rows of D bf16 / fp16 = 256 bytes):
//   K: 16-byte chunk c of key row r at r * 256 + ((c ^ (r & 15)) * 16);
//      a QK^T fragment read (16 rows at one logical chunk per 16 lanes)
//      touches 16 distinct chunk columns.
//   V: fp16, chunk c of row r at r * 256 + ((c ^ ((r & 3) << 2)) * 16); a
//      transposed PV fragment read (8 rows x 64 bytes) spreads the 8 rows
//      over all four 64-byte column groups.
// Both swizzles are applied by choosing which global chunk each lane loads,
// so the direct loads write 1 KB contiguous blocks and V is converted in place.

#include <type_traits>

#include "attn_kernels.hpp"

namespace inl {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

#define PP_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pp_rsrc(const void* base, uint32_t bytes) {
  // word3 0x00020000: raw (untyped) 32-bit data, the gfx9 buffer format.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same buffer descriptor as four SGPR words, for inline asm.
__device__ __forceinline__ i32x4 pp_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// Direct global -> LDS load of 16 bytes per lane: lane l's bytes land at LDS
// address lds + 16 * l; the global address is the descriptor base + voff
// (bytes past the descriptor's range read as zero). Issued from inline asm so
// that the compiler does not treat every later LDS read as a possible alias
// of the load and wait for all loads in flight; the kernel waits for these
// loads itself (vmcnt) before their data is used.
__device__ __forceinline__ void dma_b128(i32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(size_t)PP_LDS_PTR(p));
}

// Workgroup barrier that orders LDS only. __syncthreads() would also wait
// for every outstanding global -> LDS load (vmcnt(0)), which the pipeline
// keeps in flight across barriers on purpose.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int D, int BN>
struct PPShape {
  static constexpr int NT = 512;            // 8 waves
  static constexpr int CH = D / 8;          // 16-byte chunks per row
  static constexpr int ROW = D * 2;         // bytes per K or V row in LDS
  static constexpr int TILE = BN * ROW;     // bytes per stage
  static constexpr int STAGES = 4;
  static constexpr int LDS = 2 * STAGES * TILE;
  static constexpr int KPW = TILE / 1024 / 8;  // 1 KB direct loads per wave per tile (K and V each)
  static constexpr int RPB = 1024 / ROW;       // rows per 1 KB block
  static_assert(D == 128, "swizzles are laid out for 16 chunks per row");
  static_assert(KPW >= 1, "tile too small for 8 waves");
};

template <int D, int BN>
__global__ __launch_bounds__(512, 1) void attn_pp_kernel(AttnParams p) {
  using S = PPShape<D, BN>;
  constexpr int NKB = BN / 32;   // 32-key blocks of S^T
  constexpr int NDB = D / 32;    // 32-wide d blocks of O^T
  constexpr int KST = D / 16;    // k-steps of the QK^T product
  constexpr int PKS = BN / 16;   // k-steps of the PV product

  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const sKb = smem;
  char* const sVb = smem + S::STAGES * S::TILE;
  const uint32_t lds0 = lds_addr(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int lq = lane & 31;
  const int hf = lane >> 5;

  const int item_idx = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item_idx * p.n_hg;
  const int4 it = p.items[item_idx];
  const int seg = it.x;
  const int T = it.y;
  const int q0 = it.z;
  const int lo_t = it.w >> 16;
  const int hi_t = it.w & 0xffff;
  const int kvh = hg / p.groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * p.groups_per_kv) * p.hpw + wave / p.rb;
  const int r0 = q0 + (wave % p.rb) * 32;
  const bool active = r0 < T;
  const int causal = p.causal;
  const int window = p.window;

  const int rlast = min(r0 + 31, T - 1);
  int klo = 0, khi = causal ? min(T, r0 + 32) : T;
  if (window >= 0) {
    klo = max(0, r0 - window);
    khi = min(khi, rlast + window + 1);
  }

  const uint32_t kst_b = (uint32_t)(p.k_stride * 2);
  const uint32_t vst_b = (uint32_t)(p.v_stride * 2);
  const uint32_t qst_b = (uint32_t)(p.q_stride * 2);
  const i32x4 krs = pp_rsrc_words(p.k + ((int64_t)seg * p.k_stride + (int64_t)kvh * D) * 2, (uint32_t)T * kst_b);
  const i32x4 vrs = pp_rsrc_words(p.v + ((int64_t)seg * p.v_stride + (int64_t)kvh * D) * 2, (uint32_t)T * vst_b);
  const __amdgpu_buffer_rsrc_t qrs =
      pp_rsrc(p.q + ((int64_t)seg * p.q_stride + (int64_t)head * D) * 2, (uint32_t)T * qst_b);

  // ---- per-lane constant offsets ----
  // This wave's slice of every tile: 1 KB blocks i * 8 + wave. Lane l of a
  // block fills LDS slot l: row blk * RPB + l / CH, physical chunk l % CH,
  // and so loads the logical chunk the swizzle puts there.
  uint32_t kg_off[S::KPW], vg_off[S::KPW];   // global byte offsets within a tile
  int cv_off[S::KPW];                         // LDS byte offset of the V chunk this lane converts
#pragma unroll
  for (int i = 0; i < S::KPW; ++i) {
    const int blk = i * 8 + wave;
    const int row = blk * S::RPB + lane / S::CH;
    const int pc = lane % S::CH;
    kg_off[i] = (uint32_t)row * kst_b + ((pc ^ (row & 15)) << 4);
    vg_off[i] = (uint32_t)row * vst_b + ((pc ^ ((row & 3) << 2)) << 4);
    cv_off[i] = blk * 1024 + lane * 16;
  }
  // QK^T fragment of step st (rows lq, lq + 32): logical chunk 2 st + hf.
  int koff[KST];
#pragma unroll
  for (int st = 0; st < KST; ++st) koff[st] = lq * S::ROW + (((2 * st + hf) ^ (lq & 15)) << 4);
  // PV fragment (db, ks, half): rows ks*16 + 8*half + vrow, logical columns
  // db*32 + vcol .. +3. The swizzle of those rows depends on vrow & 3 only,
  // so each db has one per-lane base and ks / half are immediate offsets.
  const int g16 = lane >> 4;
  const int j16 = lane & 15;
  const int vcol = 16 * (g16 & 1) + 4 * (j16 & 3);
  const int vrow = 4 * hf + (j16 >> 2);
  int voff[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    voff[db] = vrow * S::ROW + ((((4 * db + (vcol >> 3)) ^ ((vrow & 3) << 2)) << 4) | ((vcol * 2) & 15));

  // ---- loads ----
  auto stage_of = [&](int t) __attribute__((always_inline)) { return (uint32_t)((t - lo_t) & (S::STAGES - 1)); };
  auto issue_tile = [&](int t) __attribute__((always_inline)) {
    const uint32_t st = stage_of(t) * S::TILE;
    const uint32_t kbase = (uint32_t)(t * BN) * kst_b;
    const uint32_t vbase = (uint32_t)(t * BN) * vst_b;
#pragma unroll
    for (int i = 0; i < S::KPW; ++i)
      dma_b128(krs, lds0 + st + (i * 8 + wave) * 1024, kbase + kg_off[i]);
#pragma unroll
    for (int i = 0; i < S::KPW; ++i)
      dma_b128(vrs, lds0 + S::STAGES * S::TILE + st + (i * 8 + wave) * 1024, vbase + vg_off[i]);
  };

  // ---- prologue: tile lo in flight, Q^T operand into registers ----
  // Q rows past the text load as zero. The compiler-visible wait for the Q
  // loads also retires tile lo's loads; after it the compiler tracks no
  // outstanding global loads, so it never inserts waits of its own later.
  const int qrow = r0 + lq;
  u32x4 qreg[KST];
  if (lo_t < hi_t) issue_tile(lo_t);
#pragma unroll
  for (int i = 0; i < KST; ++i)
    qreg[i] = __builtin_amdgcn_raw_buffer_load_b128(qrs, (uint32_t)qrow * qst_b + (2 * i + hf) * 16, 0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  if (lo_t + 1 < hi_t) issue_tile(lo_t + 1);
  lds_barrier();

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  // Row sum of the rounded fp16 P, in f32 adds: v_dot2_f32_f16 would add a
  // pair per instruction but waits for the matrix core, which the other wave
  // of the SIMD keeps busy.
  float l_i = 0.f;
  f32x16 sacc[NKB];
  u32x4 pk[PKS];   // P^T operand per PV k-step: four packed fp16 pairs
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
  for (int ks = 0; ks < PKS; ++ks)
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[ks][e] = 0u;

  const float c2 = p.scale_log2;

  auto tile_on = [&](int t) __attribute__((always_inline)) { return active && t * BN < khi && t * BN + BN > klo; };

  // LDS fragments are read two MFMA groups ahead of their use (V^T in two
  // register sets, K in a ring of three); sched_barriers keep the compiler
  // from sinking the reads next to their MFMAs.
  auto vfrag = [&](const char* sV, int ks, f16x8* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const char* vp = sV + voff[db] + ks * 16 * S::ROW;
      s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp));
      s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(vp + 8 * S::ROW));
      f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
      dst[db] = (f16x8){h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
    }
  };
  auto kfrag = [&](const char* sK, int st, bf16x8* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) dst[kb] = *reinterpret_cast<const bf16x8*>(sK + kb * 32 * S::ROW + koff[st]);
  };
  // S^T = K Q^T with kr[0], kr[1] already holding the fragments of steps 0, 1.
  auto qk_body = [&](const char* sK, bf16x8 (*kr)[NKB]) __attribute__((always_inline)) {
    const f32x16 zero = {};
#pragma unroll
    for (int st = 0; st < KST; ++st) {
      if (st + 2 < KST) kfrag(sK, st + 2, kr[(st + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[st % 3][kb], __builtin_bit_cast(bf16x8, qreg[st]),
                                                           st == 0 ? zero : sacc[kb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // In-place bf16 -> fp16 of this wave's slice of V stage (exact below 65504
  // in magnitude): the reads are issued early, the conversion later.
  auto conv_read = [&](const char* sV, u32x4* w) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) w[i] = *reinterpret_cast<const u32x4*>(sV + cv_off[i]);
  };
  auto conv_write = [&](char* sV, const u32x4* w) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f32x2 x = {__builtin_bit_cast(float, w[i][e] << 16), __builtin_bit_cast(float, w[i][e] & 0xffff0000u)};
        o[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
      }
      *reinterpret_cast<u32x4*>(sV + cv_off[i]) = o;
    }
  };

  // ---- MFMA phase of tile j ----
  // Fragment reads for the first MFMAs go out first, then the reads of the V
  // slice to convert; the conversion itself sits between PV k-steps.
  auto mphase = [&](int j) __attribute__((always_inline)) {
    const bool do_pv = j > lo_t && tile_on(j - 1);
    const bool do_qk = j < hi_t && tile_on(j);
    const bool do_cv = j < hi_t;
    const char* sK = sKb + stage_of(j) * S::TILE;
    char* sVc = sVb + stage_of(j) * S::TILE;
    u32x4 w[S::KPW];
    bf16x8 kr[3][NKB];
    if (do_pv) {
      const char* sV = sVb + stage_of(j - 1) * S::TILE;
      f16x8 vs[2][NDB];
      vfrag(sV, 0, vs[0]);
      vfrag(sV, 1, vs[1]);
      if (do_cv) conv_read(sVc, w);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vs[ks & 1][db], __builtin_bit_cast(f16x8, pk[ks]),
                                                            oacc[db], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 2 < PKS) vfrag(sV, ks + 2, vs[ks & 1]);
        if (ks + 2 >= PKS && do_qk) kfrag(sK, ks + 2 - PKS, kr[ks + 2 - PKS]);
        __builtin_amdgcn_sched_barrier(0);
        if (ks == 1 && do_cv) conv_write(sVc, w);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if (do_qk) {
        kfrag(sK, 0, kr[0]);
        kfrag(sK, 1, kr[1]);
      }
      if (do_cv) conv_read(sVc, w);
      __builtin_amdgcn_sched_barrier(0);
      if (do_cv) conv_write(sVc, w);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (do_qk) qk_body(sK, kr);
  };

  // P (fp16) and its per-lane sum over this tile, with reference max `base`.
  auto make_p = [&](float base) __attribute__((always_inline)) {
    float lt = 0.f;
#pragma unroll
    for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = sacc[ks >> 1][8 * (ks & 1) + e];
        const float x1 = sacc[ks >> 1][8 * (ks & 1) + e + 1];
        f32x2 pr = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c2, -base)),
                    __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c2, -base))};
        f16x2 pair = __builtin_convertvector(pr, f16x2);
        pk[ks][e / 2] = __builtin_bit_cast(uint32_t, pair);
        lt += (float)pair[0] + (float)pair[1];
      }
    }
    return lt;
  };
  auto apply_mask = [&](int j) __attribute__((always_inline)) {
    const int kt0 = j * BN;
    // Key of element (kb, r) is kbase + c with c a compile-time offset, so
    // every test compares c against one per-lane difference.
    const int kbase = kt0 + 4 * hf;
    const int dT = T - kbase;                     // key < T     <=> c < dT
    const int dq = r0 + lq - kbase;               // key <= qi   <=> c <= dq
    const int whi = window >= 0 ? dq + window : 0x7fffffff;            // c <= whi
    const int wlo = window >= 0 ? dq - window : -0x7fffffff;           // c >= wlo
    const int chi = min(causal ? dq : 0x7fffffff, min(dT - 1, whi));   // c <= chi
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = kb * 32 + 8 * (r >> 2) + (r & 3);
        sacc[kb][r] = (c <= chi && c >= wlo) ? sacc[kb][r] : -INFINITY;
      }
  };

  // ---- softmax of tile j (S^T in sacc) ----
  auto softmax = [&](int j) __attribute__((always_inline)) {
    const int kt0 = j * BN;
    const bool need_mask =
        (kt0 + BN > T) || (causal && kt0 + BN - 1 > r0) ||
        (window >= 0 && (rlast - kt0 > window || kt0 + BN - 1 - r0 > window));
    if (need_mask) apply_mask(j);
    // Row max (v_maximum3: no NaN canonicalisation), across the two halves.
    float mx4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2)
        mx4[(kb * 8 + r / 2) & 3] = __builtin_elementwise_maximum(
            mx4[(kb * 8 + r / 2) & 3], __builtin_elementwise_maximum(sacc[kb][r], sacc[kb][r + 1]));
    float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx4[0], mx4[1]),
                                             __builtin_elementwise_maximum(mx4[2], mx4[3]));
    mx = half_max(mx) * c2;
    // Lazy rescaling: the reference max moves only when a row's max grows by
    // more than 2^8 (P then stays <= 256, well inside fp16's range).
    if (__builtin_amdgcn_ballot_w64(mx > m_i + 8.0f)) {
      const float m_new = __builtin_elementwise_maximum(m_i, mx);
      // m_i == -inf: nothing accumulated yet (alpha 0, and no -inf - -inf).
      const float alpha = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m_new);
      m_i = m_new;
      l_i *= alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
    }
    l_i += make_p(m_i == -INFINITY ? 0.f : m_i);
  };

  // ---- softmax phase of tile j for this wave's group ----
  // Loads of tile j + grp + 2 go out first; at the end the wave waits for the
  // loads it issued one phase earlier (tile j + grp + 1), which the next MFMA
  // phases read.
  auto vphase = [&](int j) __attribute__((always_inline)) {
    const int x = j + grp + 2;
    const bool more = x < hi_t;
    if (more) issue_tile(x);
    __builtin_amdgcn_sched_barrier(0);
    if (j >= lo_t && j < hi_t && tile_on(j)) softmax(j);
    if (more) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * S::KPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };

  // Half-slots, barrier-separated. Group 0: M(lo) V(lo) ... M(hi-1) V(hi-1)
  // M(hi) [PV of the last tile] and one empty half-slot; group 1 starts one
  // half-slot earlier with V(lo-1) (loads only) and ends with M(hi).
  if (grp) {
    vphase(lo_t - 1);
    lds_barrier();
  }
  for (int j = lo_t; j < hi_t; ++j) {
    mphase(j);
    lds_barrier();
    vphase(j);
    lds_barrier();
  }
  mphase(hi_t);
  lds_barrier();
  if (!grp) lds_barrier();

  if (!active || qrow >= T) return;
  const float l_tot = half_sum(l_i);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  char* orow = p.o + ((int64_t)(seg + qrow) * p.o_stride + (int64_t)head * D) * (p.out_bf16 ? 2 : 4);
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = db * 32 + 8 * g + 4 * hf;
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

}  // namespace

bool bf16_pp_kernel(int d, AttnKernelFn* fn, int* bn, int* nw, int* lds) {
  switch (d) {
    case 128: *fn = attn_pp_kernel<128, 64>; *bn = 64; *nw = 8; *lds = PPShape<128, 64>::LDS; return true;
    default: return false;
  }
}

}  // namespace inl
