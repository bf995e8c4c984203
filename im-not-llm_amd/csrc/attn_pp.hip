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
//     one half-slot group 0 runs its MFMA phase (PV of tile j-1, then QK^T
//     of tile j) while group 1 runs its VALU phase (softmax of tile j-1,
//     V conversion, loads); in the next half-slot the roles swap. One SIMD
//     therefore always has one wave issuing MFMAs and one wave issuing VALU
//     work, and the hardware interleaves them.
//   - Lazy rescaling: P = exp2(s * c - m) against a reference max m that
//     moves only when a row's tile max exceeds it by more than 8 (log2
//     units), so O and l are rarely rescaled and P stays <= 256.
//   - K and V tiles go global -> LDS with direct loads (3 stages each, issued
//     two tiles ahead); V is then converted to fp16 into its own LDS stages
//     (2) by the lanes that loaded it. Each group loads and converts half of
//     every tile during its own VALU phases.
//
// Tile stages, by tile index t counted from the item's first tile lo:
//   K_t in K stage (t - lo) % 3, raw V_t in raw stage (t - lo) % 3, fp16 V_t
//   in V stage (t - lo) % 2.
// Group g in its VALU phase of tile j converts V_{j+g} and issues the loads
// of K_{j+g+2} and V_{j+g+2}; group 0's MFMA phase of tile j reads K_j and
// V_{j-1} one half-slot before group 1's. Every stage is rewritten only
// after the half-slot of its last reader.

#include <type_traits>

#include "attn_kernels.hpp"

namespace inl {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

#define PP_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

typedef int i32x4 __attribute__((ext_vector_type(4)));

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
// loads itself (vmcnt) before the barrier that publishes them.
__device__ __forceinline__ void dma_b128(i32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(size_t)PP_LDS_PTR(p));
}

// Workgroup barrier that orders LDS only. __syncthreads() would also wait
// for every outstanding global -> LDS load (vmcnt(0)), which the pipeline
// keeps in flight across barriers on purpose; each wave waits for its own
// loads explicitly before the barrier that publishes them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Max / sum of x over lanes l and l ^ 32. v_permlane32_swap exchanges one
// half of the first register with the other half of the second, so with both
// holding x, lane l sees x[l] in one and x[l ^ 32] in the other.
__device__ __forceinline__ void swap_halves(float x, float* a, float* b) {
  float u = x, v = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  *a = u;
  *b = v;
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

template <int D, int BN>
struct PPShape {
  static constexpr int NT = 512;            // 8 waves
  static constexpr int CH = D / 8;          // 16-byte chunks per row
  static constexpr int ROW = D * 2;         // bytes per K row in LDS
  static constexpr int KT = BN * ROW;       // bytes per K stage
  static constexpr int VROWB = D * 2 + 32;  // bytes per V row in LDS (fp16, padded)
  static constexpr int VT = BN * VROWB;     // bytes per V stage
  static constexpr int KSTAGES = 3;
  static constexpr int RSTAGES = 3;         // raw bf16 V stages (direct loads)
  static constexpr int VSTAGES = 2;         // converted fp16 V stages
  static constexpr int LDS = (KSTAGES + RSTAGES) * KT + VSTAGES * VT;
  static constexpr int KPW = KT / 1024 / 8;  // 1 KB direct loads per wave per tile (K, and raw V)
  static_assert(KPW >= 1, "tile too small for 8 waves");
  static_assert(CH >= 8 && 64 % CH == 0, "row shape");
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
  char* const sRb = smem + S::KSTAGES * S::KT;
  char* const sVb = sRb + S::RSTAGES * S::KT;
  const uint32_t lds0 = lds_addr(smem);  // LDS address of smem[0]

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

  const int rlast = min(r0 + 31, T - 1);
  int klo = 0, khi = p.causal ? min(T, r0 + 32) : T;
  if (p.window >= 0) {
    klo = max(0, r0 - p.window);
    khi = min(khi, rlast + p.window + 1);
  }

  const uint32_t kst_b = (uint32_t)(p.k_stride * 2);
  const uint32_t vst_b = (uint32_t)(p.v_stride * 2);
  const uint32_t qst_b = (uint32_t)(p.q_stride * 2);
  const i32x4 krs = pp_rsrc_words(p.k + ((int64_t)seg * p.k_stride + (int64_t)kvh * D) * 2, (uint32_t)T * kst_b);
  const i32x4 vrs = pp_rsrc_words(p.v + ((int64_t)seg * p.v_stride + (int64_t)kvh * D) * 2, (uint32_t)T * vst_b);
  const __amdgpu_buffer_rsrc_t qrs =
      pp_rsrc(p.q + ((int64_t)seg * p.q_stride + (int64_t)head * D) * 2, (uint32_t)T * qst_b);

  // ---- loads ----
  // K slice of tile t: 1 KB blocks i * 8 + wave; lane l fills LDS slot l of
  // its block, i.e. row blk * (64 / CH) + l / CH, physical chunk l % CH, and
  // so loads the logical chunk that the XOR swizzle puts there.
  auto issue_k = [&](int t) __attribute__((always_inline)) {
    const uint32_t sK = lds0 + ((t - lo_t) % S::KSTAGES) * S::KT;
    const int key0 = t * BN;
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) {
      const int blk = i * 8 + wave;
      const int row = blk * (64 / S::CH) + lane / S::CH;
      const int lc = (lane % S::CH) ^ (row & 7);
      dma_b128(krs, sK + blk * 1024, (uint32_t)(key0 + row) * kst_b + lc * 16);
    }
  };
  // Raw V slice of tile t: 1 KB blocks i * 8 + wave, linear (chunk
  // blk * 64 + lane is row (blk * 64 + lane) / CH, chunk % CH). The same lane
  // converts the chunk it loaded, so conversion waits only on its own loads.
  auto issue_v = [&](int t) __attribute__((always_inline)) {
    const uint32_t sR = lds0 + S::KSTAGES * S::KT + ((t - lo_t) % S::RSTAGES) * S::KT;
    const int key0 = t * BN;
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) {
      const int blk = i * 8 + wave;
      const int id = blk * 64 + lane;
      const int row = id / S::CH, c = id % S::CH;
      dma_b128(vrs, sR + blk * 1024, (uint32_t)(key0 + row) * vst_b + c * 16);
    }
  };
  // bf16 -> fp16 (exact below 65504 in magnitude), raw stage -> V stage of tile t.
  auto read_raw_v = [&](int t, u32x4* w) __attribute__((always_inline)) {
    const char* sR = sRb + ((t - lo_t) % S::RSTAGES) * S::KT;
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) w[i] = *reinterpret_cast<const u32x4*>(sR + ((i * 8 + wave) * 64 + lane) * 16);
  };
  auto store_v = [&](int t, const u32x4* w) __attribute__((always_inline)) {
    char* sV = sVb + ((t - lo_t) & 1) * S::VT;
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) {
      const int id = (i * 8 + wave) * 64 + lane;
      const int row = id / S::CH, c = id % S::CH;
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x2 x = {__builtin_bit_cast(float, w[i][j] << 16), __builtin_bit_cast(float, w[i][j] & 0xffff0000u)};
        o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
      }
      *reinterpret_cast<u32x4*>(sV + row * S::VROWB + c * 16) = o;
    }
  };

  // ---- prologue: tile lo in flight, Q^T operand into registers ----
  // Q rows past the text load as zero. The compiler-visible wait for the Q
  // loads also retires tile lo's loads; after it the compiler tracks no
  // outstanding global loads, so it never inserts waits of its own later.
  const int qrow = r0 + lq;
  u32x4 qreg[KST];
  if (lo_t < hi_t) {
    issue_k(lo_t);
    issue_v(lo_t);
  }
#pragma unroll
  for (int i = 0; i < KST; ++i)
    qreg[i] = __builtin_amdgcn_raw_buffer_load_b128(qrs, (uint32_t)qrow * qst_b + (2 * i + hf) * 16, 0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  if (lo_t + 1 < hi_t) {
    issue_k(lo_t + 1);
    issue_v(lo_t + 1);
  }
  lds_barrier();

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;
  f32x16 sacc[NKB];
  f16x8 pk[PKS];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
  for (int ks = 0; ks < PKS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) pk[ks][e] = (f16)0.f;

  const float c2 = p.scale_log2;
  const int g16 = lane >> 4;
  const int j16 = lane & 15;
  int koff[KST];
#pragma unroll
  for (int st = 0; st < KST; ++st) koff[st] = lq * S::ROW + (((2 * st + hf) ^ (lq & 7)) << 4);
  // V^T fragment (db, ks, half): rows ks*16 + 8*half + vrow, columns
  // db*32 + vcol, at a linear offset from this per-lane base.
  const int vcol = 16 * (g16 & 1) + 4 * (j16 & 3);
  const int vrow = 4 * hf + (j16 >> 2);
  const int vbase_off = vrow * S::VROWB + vcol * 2;

  auto tile_on = [&](int t) __attribute__((always_inline)) { return active && t * BN < khi && t * BN + BN > klo; };

  // ---- MFMA phase of tile j: O^T += V_{j-1}^T P^T, then S^T = K_j Q^T ----
  // LDS fragments are read two MFMA groups ahead of their use (V^T in two
  // register sets, K in a ring of three) and sched_barriers keep the
  // compiler from sinking the reads next to their MFMAs, so the matrix pipe
  // does not wait on LDS latency.
  auto vfrag = [&](const char* vptr, int ks, f16x8* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const char* vp = vptr + ks * 16 * S::VROWB + db * 64;
      s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp));
      s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(vp + 8 * S::VROWB));
      f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
      dst[db] = (f16x8){h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
    }
  };
  auto kfrag = [&](const char* sK, int st, bf16x8* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) dst[kb] = *reinterpret_cast<const bf16x8*>(sK + kb * 32 * S::ROW + koff[st]);
  };
  auto mphase = [&](int j) __attribute__((always_inline)) {
    const bool do_pv = j > lo_t && tile_on(j - 1);
    const bool do_qk = j < hi_t && tile_on(j);
    const char* sK = sKb + ((j - lo_t) % S::KSTAGES) * S::KT;
    bf16x8 kr[3][NKB];
    if (do_pv) {
      const char* vptr = sVb + ((j - 1 - lo_t) & 1) * S::VT + vbase_off;
      f16x8 vs[2][NDB];
      vfrag(vptr, 0, vs[0]);
      vfrag(vptr, 1, vs[1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vs[ks & 1][db], pk[ks], oacc[db], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + 2 < PKS) vfrag(vptr, ks + 2, vs[ks & 1]);
        else if (do_qk) kfrag(sK, ks + 2 - PKS, kr[ks + 2 - PKS]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (do_qk) {
      kfrag(sK, 0, kr[0]);
      kfrag(sK, 1, kr[1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (do_qk) {
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
    }
  };

  // P (fp16) and its per-lane sum over this tile, with reference max `base`.
  auto make_p = [&](float base) __attribute__((always_inline)) {
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
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
        pk[ks][e] = pair[0];
        pk[ks][e + 1] = pair[1];
        lt = __builtin_amdgcn_fdot2(pair, ones, lt, false);
      }
    }
    return lt;
  };

  // ---- softmax of tile j (S^T in sacc) ----
  auto softmax = [&](int j) __attribute__((always_inline)) {
    const int kt0 = j * BN;
    const bool need_mask =
        (kt0 + BN > T) || (p.causal && kt0 + BN - 1 > r0) ||
        (p.window >= 0 && (rlast - kt0 > p.window || kt0 + BN - 1 - r0 > p.window));
    if (need_mask) {
      // Key of element (kb, r) is kbase + c with c a compile-time offset, so
      // every test compares c against one per-lane difference.
      const int kbase = kt0 + 4 * hf;
      const int dT = T - kbase;                     // key < T     <=> c < dT
      const int dq = r0 + lq - kbase;               // key <= qi   <=> c <= dq
      const int whi = p.window >= 0 ? dq + p.window : 0x7fffffff;            // c <= whi
      const int wlo = p.window >= 0 ? dq - p.window : -0x7fffffff;           // c >= wlo
      const int chi = min(p.causal ? dq : 0x7fffffff, min(dT - 1, whi));     // c <= chi
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = kb * 32 + 8 * (r >> 2) + (r & 3);
          sacc[kb][r] = (c <= chi && c >= wlo) ? sacc[kb][r] : -INFINITY;
        }
    }
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

  // ---- VALU phase of tile j for this wave's group ----
  // The reads of the raw V slice to convert and the loads of tile x + 2 are
  // issued first, so their latency is hidden behind the softmax.
  auto vphase = [&](int j) __attribute__((always_inline)) {
    const int x = j + grp;  // V tile this group converts now (x >= lo_t)
    u32x4 w[S::KPW];
    if (x < hi_t) read_raw_v(x, w);
    const bool more = x + 2 < hi_t;
    if (more) {
      issue_v(x + 2);
      issue_k(x + 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j >= lo_t && j < hi_t && tile_on(j)) softmax(j);
    __builtin_amdgcn_sched_barrier(0);
    if (x < hi_t) store_v(x, w);
    if (more) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * S::KPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };

  // Half-slots, barrier-separated. Group 0: M(lo) V(lo) ... M(hi-1) V(hi-1)
  // M(hi) [PV of the last tile] and one empty half-slot; group 1 starts one
  // half-slot earlier with V(lo-1) (staging only) and ends with M(hi).
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
